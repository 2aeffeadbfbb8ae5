// The producers of the rule's inputs in the Qwen3.5 / Qwen3-Next linear-attention layer (the reference's
// layer/_conv.py:1-24 and layer/_gates.py:1-13, restated for MI355X):
//
//   convolution path: u[t, c] = sum_j w[c, j] x[t - 3 + j, c] (depthwise, causal, kernel 4, zero before the start;
//   float32), y = u sigmoid(u) rounded once, split into q, k (key_dim channels each) and v (value_dim channels);
//   gates: beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias) (softplus's threshold 20), both float32.
//
// Both are streaming element-wise work bound by HBM: a thread owns 4 adjacent channels and walks a tile of time steps
// with the convolution window in registers, issuing a group of steps' loads at once; no LDS, no barriers, one writer
// an element.  The backward recomputes u from x (nothing else is kept) and gathers dx with one writer an element; the
// weight's gradient, when it trains, goes through float32 partial sums a tile and a fixed-order second pass.
#include <hip/hip_runtime.h>

#include "gdr_abi.h"
#include "gdr_common.h"

namespace gdr {

typedef _Float16 f16;

// N = 4 or 8 consecutive elements <-> float (one 8- or 16-byte access for 2-byte types)
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
template <typename T, int N> struct VecOf;
template <> struct VecOf<bf16, 4> { typedef bf16x4 type; };
template <> struct VecOf<bf16, 8> { typedef bf16x8 type; };
template <> struct VecOf<f16, 4> { typedef f16x4 type; };
template <> struct VecOf<f16, 8> { typedef f16x8 type; };
template <int N>
__device__ __forceinline__ void ldn(const float* p, float (&x)[N]) {
#pragma unroll
  for (int h = 0; h < N / 4; ++h) {
    const f4 a = *reinterpret_cast<const f4*>(p + 4 * h);
#pragma unroll
    for (int i = 0; i < 4; ++i) x[4 * h + i] = a[i];
  }
}
template <int N, typename T>
__device__ __forceinline__ void ldn(const T* p, float (&x)[N]) {
  const typename VecOf<T, N>::type v = *reinterpret_cast<const typename VecOf<T, N>::type*>(p);
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] = (float)v[i];
}
template <int N>
__device__ __forceinline__ void stn(float* p, const float (&x)[N]) {
#pragma unroll
  for (int h = 0; h < N / 4; ++h)
    *reinterpret_cast<f4*>(p + 4 * h) = f4{x[4 * h], x[4 * h + 1], x[4 * h + 2], x[4 * h + 3]};
}
template <int N, typename T>
__device__ __forceinline__ void stn(T* p, const float (&x)[N]) {
  typename VecOf<T, N>::type v;
#pragma unroll
  for (int i = 0; i < N; ++i) v[i] = (T)x[i];
  *reinterpret_cast<typename VecOf<T, N>::type*>(p) = v;
}
template <typename T> __device__ __forceinline__ float ld1(const T* p) { return (float)*p; }
template <typename T> __device__ __forceinline__ void st1(T* p, float x) { *p = (T)x; }

constexpr int CONV_K = 4;        // taps
constexpr int CONV_CH = 4;       // channels a thread (8-byte accesses for 2-byte types)
constexpr int CONV_GROUP = 256;  // threads a workgroup (along the channels)
constexpr int CONV_U = 8;        // time steps whose loads a thread issues together (memory-level parallelism)

struct ConvArgs {
  const void* x;                 // [B, T, C] T
  const float* w;                // [C, 4] float32 taps
  void *q, *k, *v;               // q, k [B, T, KD * REP] T; v [B, T, C - 2 KD] TV
  const void *dq, *dk, *dv;      // the backward's upstream gradients (same layouts)
  void* dx;                      // [B, T, C] T
  float* dwp;                    // [B * ntiles, C, 4] float32 partials, or null
  int B, T, C, KD, DK, REP, L, ntiles;
};

// where a thread's 8 channels go: q or k (a key head written REP times, REP = 1: key heads only), or v
struct ConvMap {
  bool isv;
  int cc;                        // channel within q, k or v
  size_t row, col;               // row pitch and first column in the destination
  __device__ ConvMap(const ConvArgs& a, int c) {
    isv = c >= 2 * a.KD;
    cc = isv ? c - 2 * a.KD : (c >= a.KD ? c - a.KD : c);
    if (isv) {
      row = (size_t)(a.C - 2 * a.KD);
      col = cc;
    } else {
      row = (size_t)a.KD * a.REP;
      col = (size_t)(cc / a.DK) * a.REP * a.DK + cc % a.DK;
    }
  }
};

__device__ __forceinline__ void load_taps(const float* w, int c, float (&tap)[CONV_K][CONV_CH]) {
#pragma unroll
  for (int i = 0; i < CONV_CH; ++i) {
    const f4 r = *reinterpret_cast<const f4*>(w + (size_t)(c + i) * CONV_K);
#pragma unroll
    for (int j = 0; j < CONV_K; ++j) tap[j][i] = r[j];
  }
}

// u = w0 x[t-3] + w1 x[t-2] + w2 x[t-1] + w3 x[t], in the reference's order (layer/_conv.py:73).  With float32
// inputs (PRECISE) the sum is formed in double and rounded once, and sigmoid divides exactly: there the four roundings
// of a float sum would set the outputs' error (about 1 ulp of max |u|).  With 2-byte inputs the outputs' own rounding
// dominates, so the sum stays in float and exp / division take the fast forms (the work is then bound by HBM).
template <bool PRECISE>
__device__ __forceinline__ float conv_u(const float (&tap)[CONV_K][CONV_CH], int i, float xm3, float xm2, float xm1,
                                        float xt) {
  if constexpr (PRECISE)
    return (float)fma((double)tap[3][i], (double)xt,
                      fma((double)tap[2][i], (double)xm1, fma((double)tap[1][i], (double)xm2,
                                                              (double)tap[0][i] * (double)xm3)));
  else
    return fmaf(tap[3][i], xt, fmaf(tap[2][i], xm1, fmaf(tap[1][i], xm2, tap[0][i] * xm3)));
}
// w0 d0 + (w1 d1 + (w2 d2 + w3 d3)), with the same precision rule
template <bool PRECISE>
__device__ __forceinline__ float taps4(float w0, float d0, float w1, float d1, float w2, float d2, float w3, float d3) {
  if constexpr (PRECISE)
    return (float)fma((double)w0, (double)d0, fma((double)w1, (double)d1, fma((double)w2, (double)d2,
                                                                            (double)w3 * (double)d3)));
  else
    return fmaf(w0, d0, fmaf(w1, d1, fmaf(w2, d2, w3 * d3)));
}
template <bool PRECISE>
__device__ __forceinline__ float silu_of(float u) {
  if constexpr (PRECISE) return u / (1.0f + expf(-u));
  else return __fdividef(u, 1.0f + __expf(-u));
}
template <bool PRECISE>
__device__ __forceinline__ float sigmoid_of(float u) {
  if constexpr (PRECISE) return 1.0f / (1.0f + expf(-u));
  else return __fdividef(1.0f, 1.0f + __expf(-u));
}

template <typename T, typename TV>
__global__ void __launch_bounds__(CONV_GROUP) conv_fwd_kernel(ConvArgs a) {
  const int c = (blockIdx.x * CONV_GROUP + threadIdx.x) * CONV_CH;
  if (c >= a.C) return;
  const int t0 = blockIdx.y * a.L, b = blockIdx.z;
  float tap[CONV_K][CONV_CH];
  load_taps(a.w, c, tap);
  const T* xb = (const T*)a.x + (size_t)b * a.T * a.C + c;
  float xm3[CONV_CH] = {}, xm2[CONV_CH] = {}, xm1[CONV_CH] = {};
  if (t0 >= 3) ldn<CONV_CH>(xb + (size_t)(t0 - 3) * a.C, xm3);
  if (t0 >= 2) ldn<CONV_CH>(xb + (size_t)(t0 - 2) * a.C, xm2);
  if (t0 >= 1) ldn<CONV_CH>(xb + (size_t)(t0 - 1) * a.C, xm1);
  const ConvMap m(a, c);
  const int te = t0 + a.L < a.T ? t0 + a.L : a.T;
  for (int tb = t0; tb < te; tb += CONV_U) {
    float xs[CONV_U][CONV_CH];            // the group's inputs, all loads in flight before the first is used
#pragma unroll
    for (int s = 0; s < CONV_U; ++s)
      if (tb + s < te) ldn<CONV_CH>(xb + (size_t)(tb + s) * a.C, xs[s]);
#pragma unroll
    for (int s = 0; s < CONV_U; ++s) {
      if (tb + s >= te) break;
      const int t = tb + s;
      float y[CONV_CH];
#pragma unroll
      for (int i = 0; i < CONV_CH; ++i) {
        const float u = conv_u<sizeof(T) == 4>(tap, i, xm3[i], xm2[i], xm1[i], xs[s][i]);
        y[i] = silu_of<sizeof(T) == 4>(u);
        xm3[i] = xm2[i];
        xm2[i] = xm1[i];
        xm1[i] = xs[s][i];
      }
      const size_t bt = (size_t)b * a.T + t;
      if (m.isv) {
        stn<CONV_CH>((TV*)a.v + bt * m.row + m.col, y);
      } else {
        T* dst = (T*)(c >= a.KD ? a.k : a.q) + bt * m.row + m.col;
        for (int r = 0; r < a.REP; ++r) stn<CONV_CH>(dst + (size_t)r * a.DK, y);
      }
    }
  }
}

// dx[t] = sum_j w_j du[t + 3 - j] with du = dy sigmoid(u) (1 + u (1 - sigmoid(u))) (0 past the end; dy of q and k
// summed over the REP copies in copy order); dw partials a tile: sum over its t of du[t] x[t - 3 + j].
template <typename T, typename TV, bool DW>
__global__ void __launch_bounds__(CONV_GROUP) conv_bwd_kernel(ConvArgs a) {
  constexpr int U = 4;                    // time steps whose loads are issued together
  const int c = (blockIdx.x * CONV_GROUP + threadIdx.x) * CONV_CH;
  if (c >= a.C) return;
  const int t0 = blockIdx.y * a.L, b = blockIdx.z;
  float tap[CONV_K][CONV_CH];
  load_taps(a.w, c, tap);
  const T* xb = (const T*)a.x + (size_t)b * a.T * a.C + c;
  T* dxb = (T*)a.dx + (size_t)b * a.T * a.C + c;
  float xm3[CONV_CH] = {}, xm2[CONV_CH] = {}, xm1[CONV_CH] = {};
  if (t0 >= 3) ldn<CONV_CH>(xb + (size_t)(t0 - 3) * a.C, xm3);
  if (t0 >= 2) ldn<CONV_CH>(xb + (size_t)(t0 - 2) * a.C, xm2);
  if (t0 >= 1) ldn<CONV_CH>(xb + (size_t)(t0 - 1) * a.C, xm1);
  float dm1[CONV_CH] = {}, dm2[CONV_CH] = {}, dm3[CONV_CH] = {};   // du[t - 1], du[t - 2], du[t - 3]
  double acc[DW ? CONV_K : 1][CONV_CH] = {};                       // dw partials, in double (rounded once)
  const ConvMap m(a, c);
  const int tl = t0 + a.L < a.T ? t0 + a.L : a.T;                 // this tile's outputs: [t0, tl)
  const int tw = tl + 3 < a.T ? tl + 3 : a.T;                     // the inputs the walk reads: [t0, tw)
  for (int tb = t0; tb < tl + 3; tb += U) {
    // the group's inputs and upstream gradients, all loads in flight before the first is used
    float xs[U][CONV_CH], gs[U][CONV_CH];
#pragma unroll
    for (int s = 0; s < U; ++s) {
      if (tb + s < tw) {
        const size_t bt = (size_t)b * a.T + tb + s;
        ldn<CONV_CH>(xb + (size_t)(tb + s) * a.C, xs[s]);
        if (m.isv) ldn<CONV_CH>((const TV*)a.dv + bt * m.row + m.col, gs[s]);
        else ldn<CONV_CH>((const T*)(c >= a.KD ? a.dk : a.dq) + bt * m.row + m.col, gs[s]);
      }
    }
#pragma unroll
    for (int s = 0; s < U; ++s) {
    const int t = tb + s;
    if (t >= tl + 3) break;
    float du[CONV_CH] = {}, xt[CONV_CH] = {};
    if (t < a.T) {
      const size_t bt = (size_t)b * a.T + t;
      float gy[CONV_CH];
#pragma unroll
      for (int i = 0; i < CONV_CH; ++i) {
        xt[i] = xs[s][i];
        gy[i] = gs[s][i];
      }
      if (!m.isv) {                        // the other copies of a repeated key head, summed in copy order
        const T* src = (const T*)(c >= a.KD ? a.dk : a.dq) + bt * m.row + m.col;
        for (int r = 1; r < a.REP; ++r) {
          float g2[CONV_CH];
          ldn<CONV_CH>(src + (size_t)r * a.DK, g2);
#pragma unroll
          for (int i = 0; i < CONV_CH; ++i) gy[i] += g2[i];
        }
      }
#pragma unroll
      for (int i = 0; i < CONV_CH; ++i) {
        const float u = conv_u<sizeof(T) == 4>(tap, i, xm3[i], xm2[i], xm1[i], xt[i]);
        const float s = sigmoid_of<sizeof(T) == 4>(u);
        du[i] = gy[i] * s * (1.0f + u * (1.0f - s));
      }
      if constexpr (DW) {
        if (t < tl) {
#pragma unroll
          for (int i = 0; i < CONV_CH; ++i) {
            acc[0][i] = fma((double)du[i], (double)xm3[i], acc[0][i]);
            acc[1][i] = fma((double)du[i], (double)xm2[i], acc[1][i]);
            acc[2][i] = fma((double)du[i], (double)xm1[i], acc[2][i]);
            acc[3][i] = fma((double)du[i], (double)xt[i], acc[3][i]);
          }
        }
      }
    }
    if (t >= t0 + 3) {
      float dx[CONV_CH];
#pragma unroll
      for (int i = 0; i < CONV_CH; ++i)        // rounded once for float32 inputs (as u)
        dx[i] = taps4<sizeof(T) == 4>(tap[0][i], du[i], tap[1][i], dm1[i], tap[2][i], dm2[i], tap[3][i], dm3[i]);
      stn<CONV_CH>(dxb + (size_t)(t - 3) * a.C, dx);
    }
#pragma unroll
    for (int i = 0; i < CONV_CH; ++i) {
      xm3[i] = xm2[i];
      xm2[i] = xm1[i];
      xm1[i] = xt[i];
      dm3[i] = dm2[i];
      dm2[i] = dm1[i];
      dm1[i] = du[i];
    }
    }
  }
  if constexpr (DW) {
    float* p = a.dwp + ((size_t)(b * a.ntiles + blockIdx.y) * a.C + c) * CONV_K;
#pragma unroll
    for (int i = 0; i < CONV_CH; ++i)
      *reinterpret_cast<f4*>(p + i * CONV_K) = f4{(float)acc[0][i], (float)acc[1][i], (float)acc[2][i],
                                                  (float)acc[3][i]};
  }
}

// out[i] = sum over the P partial rows of p[., i], in row order, in double (one thread an element: deterministic)
__global__ void __launch_bounds__(256) sum_rows_kernel(const float* p, float* out, int P, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  double s = 0.0;
  int r = 0;
  for (; r + 8 <= P; r += 8) {           // eight rows' loads in flight, added in row order
    float v[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) v[k] = p[(size_t)(r + k) * n + i];
#pragma unroll
    for (int k = 0; k < 8; ++k) s += (double)v[k];
  }
  for (; r < P; ++r) s += (double)p[(size_t)r * n + i];
  out[i] = (float)s;
}

// ---- gates ------------------------------------------------------------------------------------------------------------
// softplus with PyTorch's threshold of 20 (the input itself above it), log1p below it
__device__ __forceinline__ float softplus20(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

template <typename T>
__global__ void __launch_bounds__(256) gates_fwd_kernel(const T* b, const T* a, const float* alog, const float* dtb,
                                                        float* beta, float* g, int64_t n, int H) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int h = (int)(i % H);
  beta[i] = 1.0f / (1.0f + expf(-ld1(b + i)));
  g[i] = -expf(alog[h]) * softplus20(ld1(a + i) + dtb[h]);
}

// db = dbeta beta (1 - beta); da = dg (-exp(A_log)) sigmoid(a + dt_bias) (1 above the threshold)
template <typename T>
__global__ void __launch_bounds__(256) gates_bwd_kernel(const T* b, const T* a, const float* alog, const float* dtb,
                                                        const float* dbeta, const float* dg, T* db, T* da, int64_t n,
                                                        int H) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int h = (int)(i % H);
  const float sb = 1.0f / (1.0f + expf(-ld1(b + i)));
  st1(db + i, dbeta[i] * sb * (1.0f - sb));
  const float xa = ld1(a + i) + dtb[h];
  const float sx = xa > 20.0f ? 1.0f : 1.0f / (1.0f + expf(-xa));
  st1(da + i, dg[i] * (-expf(alog[h])) * sx);
}

// A_log's and dt_bias's gradients, one workgroup a head: dA[h] = sum_t dg g, ddt[h] = sum_t dg (-exp(A_log)) sx over
// the n / H rows, each thread a strided part in order, then a fixed tree (deterministic)
template <typename T>
__global__ void __launch_bounds__(256) gates_param_kernel(const T* a, const float* alog, const float* dtb,
                                                          const float* dg, float* dA, float* ddt, int64_t rows,
                                                          int H) {
  const int h = blockIdx.x;
  const float ea = expf(alog[h]);
  float sa = 0.f, sd = 0.f;
  for (int64_t r = threadIdx.x; r < rows; r += 256) {
    const int64_t i = r * H + h;
    const float xa = ld1(a + i) + dtb[h];
    const float sx = xa > 20.0f ? 1.0f : 1.0f / (1.0f + expf(-xa));
    sa = fmaf(dg[i], -ea * softplus20(xa), sa);
    sd = fmaf(dg[i], -ea * sx, sd);
  }
  __shared__ float pa[256], pd[256];
  pa[threadIdx.x] = sa;
  pd[threadIdx.x] = sd;
  __syncthreads();
  for (int off = 128; off > 0; off >>= 1) {
    if ((int)threadIdx.x < off) {
      pa[threadIdx.x] += pa[threadIdx.x + off];
      pd[threadIdx.x] += pd[threadIdx.x + off];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    dA[h] = pa[0];
    ddt[h] = pd[0];
  }
}

}  // namespace gdr

using namespace gdr;

namespace {

int check_conv(const char* what, int64_t B, int64_t T, int64_t C, int64_t KD, int64_t DK, int64_t REP, int64_t DV,
               int32_t dtype, int32_t vdtype) {
  if (B < 1 || T < 1 || B > 65535 || T > 65535 * 16)
    return fail(MACAI_GDR_EINVAL, "%s: B in [1, 65535] and T in [1, 65535 x 16] (got %lld, %lld)", what, (long long)B,
                (long long)T);
  if (dtype < MACAI_GDR_F32 || dtype > MACAI_GDR_F16 || vdtype < MACAI_GDR_F32 || vdtype > MACAI_GDR_F16)
    return fail(MACAI_GDR_EUNSUP, "%s: dtype codes must be F32, BF16 or F16", what);
  const int64_t VD = C - 2 * KD;
  if (KD < 1 || DK < 1 || DV < 1 || REP < 1 || VD < 1 || KD % DK || VD % DV || KD % 8 || DK % 8 || DV % 8 || C % 8)
    return fail(MACAI_GDR_EINVAL,
                 "%s: need key_dim a multiple of the key head width, value_dim = C - 2 key_dim a multiple of the value "
                 "head width, all multiples of 8 (got C %lld, key_dim %lld, DK %lld, DV %lld, REP %lld)",
                 what, (long long)C, (long long)KD, (long long)DK, (long long)DV, (long long)REP);
  if (REP != 1 && (KD / DK) * REP != VD / DV)
    return fail(MACAI_GDR_EINVAL, "%s: REP must be 1 (key heads only) or value heads / key heads (%lld)", what,
                 (long long)(VD / DV / (KD / DK)));
  if (B * T * C >= (int64_t)1 << 31 || B * T * KD * REP >= (int64_t)1 << 31)
    return fail(MACAI_GDR_EINVAL, "%s: tensors past 2^31 elements are not supported", what);
  return MACAI_GDR_OK;
}

constexpr int CONV_TILE = 16;   // time steps a thread walks

}  // namespace

#define DISPATCH_PT(code, ...)                                             \
  switch (code) {                                                          \
    case MACAI_GDR_F32: { using PT = float; __VA_ARGS__; } break;          \
    case MACAI_GDR_BF16: { using PT = gdr::bf16; __VA_ARGS__; } break;     \
    default: { using PT = gdr::f16; __VA_ARGS__; } break;                  \
  }
#define DISPATCH_PV(code, ...)                                             \
  switch (code) {                                                          \
    case MACAI_GDR_F32: { using PV = float; __VA_ARGS__; } break;          \
    case MACAI_GDR_BF16: { using PV = gdr::bf16; __VA_ARGS__; } break;     \
    default: { using PV = gdr::f16; __VA_ARGS__; } break;                  \
  }

extern "C" {

int macai_gdr_conv_fwd(const void* x, const float* w, void* q, void* k, void* v, int64_t B, int64_t T, int64_t C,
                       int64_t KD, int64_t DK, int64_t REP, int64_t DV, int32_t dtype, int32_t vdtype, void* stream) {
  const char* what = "macai_gdr_conv_fwd";
  if (int rc = check_conv(what, B, T, C, KD, DK, REP, DV, dtype, vdtype)) return rc;
  if (!x || !w || !q || !k || !v) return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  const void* ps[] = {x, w, q, k, v};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  const int ntiles = (int)((T + CONV_TILE - 1) / CONV_TILE);
  ConvArgs a{x, w, q, k, v, nullptr, nullptr, nullptr, nullptr, nullptr, (int)B, (int)T, (int)C, (int)KD, (int)DK,
             (int)REP, CONV_TILE, ntiles};
  const dim3 grid((unsigned)((C / CONV_CH + CONV_GROUP - 1) / CONV_GROUP), (unsigned)ntiles, (unsigned)B);
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_PT(dtype, DISPATCH_PV(vdtype, hipLaunchKernelGGL((conv_fwd_kernel<PT, PV>), grid, dim3(CONV_GROUP), 0,
                                                            st, a)))
  return launched(what);
}

int macai_gdr_conv_bwd(const void* x, const float* w, const void* dq, const void* dk, const void* dv, void* dx,
                       float* dwp, float* dw, int64_t B, int64_t T, int64_t C, int64_t KD, int64_t DK, int64_t REP,
                       int64_t DV, int32_t dtype, int32_t vdtype, void* stream) {
  const char* what = "macai_gdr_conv_bwd";
  if (int rc = check_conv(what, B, T, C, KD, DK, REP, DV, dtype, vdtype)) return rc;
  if (!x || !w || !dq || !dk || !dv || !dx) return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  if (!dwp != !dw) return fail(MACAI_GDR_EINVAL, "%s: dwp and dw go together (both or neither)", what);
  const void* ps[] = {x, w, dq, dk, dv, dx, dwp};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  const int ntiles = (int)((T + CONV_TILE - 1) / CONV_TILE);
  ConvArgs a{x, w, nullptr, nullptr, nullptr, dq, dk, dv, dx, dwp, (int)B, (int)T, (int)C, (int)KD, (int)DK,
             (int)REP, CONV_TILE, ntiles};
  const dim3 grid((unsigned)((C / CONV_CH + CONV_GROUP - 1) / CONV_GROUP), (unsigned)ntiles, (unsigned)B);
  hipStream_t st = (hipStream_t)stream;
  if (dwp) {
    DISPATCH_PT(dtype, DISPATCH_PV(vdtype, hipLaunchKernelGGL((conv_bwd_kernel<PT, PV, true>), grid, dim3(CONV_GROUP),
                                                              0, st, a)))
  } else {
    DISPATCH_PT(dtype, DISPATCH_PV(vdtype, hipLaunchKernelGGL((conv_bwd_kernel<PT, PV, false>), grid,
                                                              dim3(CONV_GROUP), 0, st, a)))
  }
  if (int rc = launched(what)) return rc;
  if (dw) {
    const int n = (int)(C * CONV_K);
    hipLaunchKernelGGL(sum_rows_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dwp, dw,
                       (int)(B * ntiles), n);
    return launched(what);
  }
  return MACAI_GDR_OK;
}

int64_t macai_gdr_conv_partials(int64_t B, int64_t T, int64_t C) {
  return B * ((T + CONV_TILE - 1) / CONV_TILE) * C * CONV_K;
}

int macai_gdr_gates_fwd(const void* b, const void* a, const float* A_log, const float* dt_bias, float* beta, float* g,
                        int64_t n, int64_t H, int32_t dtype, void* stream) {
  const char* what = "macai_gdr_gates_fwd";
  if (n < 1 || H < 1 || n % H) return fail(MACAI_GDR_EINVAL, "%s: need n >= 1 a multiple of H >= 1", what);
  if (dtype < MACAI_GDR_F32 || dtype > MACAI_GDR_F16) return fail(MACAI_GDR_EUNSUP, "%s: dtype code", what);
  if (!b || !a || !A_log || !dt_bias || !beta || !g) return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((n + 255) / 256));
  DISPATCH_PT(dtype, hipLaunchKernelGGL((gates_fwd_kernel<PT>), grid, dim3(256), 0, st, (const PT*)b, (const PT*)a,
                                        A_log, dt_bias, beta, g, n, (int)H))
  return launched(what);
}

int macai_gdr_gates_bwd(const void* b, const void* a, const float* A_log, const float* dt_bias, const float* dbeta,
                        const float* dg, void* db, void* da, float* dA_log, float* ddt_bias, int64_t n, int64_t H,
                        int32_t dtype, void* stream) {
  const char* what = "macai_gdr_gates_bwd";
  if (n < 1 || H < 1 || n % H) return fail(MACAI_GDR_EINVAL, "%s: need n >= 1 a multiple of H >= 1", what);
  if (dtype < MACAI_GDR_F32 || dtype > MACAI_GDR_F16) return fail(MACAI_GDR_EUNSUP, "%s: dtype code", what);
  if (!b || !a || !A_log || !dt_bias || !dbeta || !dg || !db || !da)
    return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  if (!dA_log != !ddt_bias) return fail(MACAI_GDR_EINVAL, "%s: dA_log and ddt_bias go together", what);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((n + 255) / 256));
  DISPATCH_PT(dtype, hipLaunchKernelGGL((gates_bwd_kernel<PT>), grid, dim3(256), 0, st, (const PT*)b, (const PT*)a,
                                        A_log, dt_bias, dbeta, dg, (PT*)db, (PT*)da, n, (int)H))
  if (int rc = launched(what)) return rc;
  if (dA_log) {
    DISPATCH_PT(dtype, hipLaunchKernelGGL((gates_param_kernel<PT>), dim3((unsigned)H), dim3(256), 0, st,
                                          (const PT*)a, A_log, dt_bias, dg, dA_log, ddt_bias, n / H, (int)H))
    return launched(what);
  }
  return MACAI_GDR_OK;
}

}  // extern "C"

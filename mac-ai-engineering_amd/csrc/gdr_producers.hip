// The producers of the rule's inputs in the Qwen3.5 / Qwen3-Next linear-attention layer, for MI355X (gfx950):
//
//   convolution path  u[t, c] = sum_j w[c, j] x[t - 3 + j, c] (depthwise, causal, 4 taps, zero before the start),
//                     y = u sigmoid(u) rounded once, split into q, k (key_dim channels each) and v (value_dim);
//   gates             beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias) (softplus's threshold 20).
//   (The reference's layer/_conv.py:1-24 and layer/_gates.py:1-13 state the same functions.)
//
// The convolution is an HBM stream: every input and output byte crosses once (the 3-row halos come again through L2).
// Work goes by 16-byte channel vectors (8 bf16 / f16 or 4 fp32 channels).  The forward gives a lane one vector over 8
// consecutive time steps, all 11 input rows loaded at once, a wave 64 consecutive vectors (conv_fwd_kernel).  The
// backward needs du = dy silu'(u) at 3 rows past each output row and shares it between neighbouring outputs, so it runs
// on LDS tiles: a workgroup stages x (64 + 6 rows: a 3-row halo each side, by asynchronous global -> LDS copies) and the
// upstream gradient (67 rows, a key head's copies summed) of 8 vectors, forms du for the tile in LDS (float32) and
// gathers dx from du's windows, every lane in parallel over time: one writer an element.  The taps' gradient is a
// per-tile correlation of du with x from the same LDS tiles, reduced over the tile's rows in a fixed order (lane pairs,
// then the four waves through LDS); sum_columns_kernel adds the tiles' partials in tile order: deterministic.
// The gates are one pass each way, an element a lane; A_log's and dt_bias's gradients take one
// workgroup a head, rows split over its waves and summed in a fixed tree.
#include <hip/hip_runtime.h>

#include "gdr_abi.h"
#include "gdr_common.h"

namespace gdr {

typedef _Float16 f16;

// ---- 16-byte vectors of 2- or 4-byte elements, as floats -----------------------------------------------------------
template <typename T> struct V16 {
  static constexpr int N = 16 / (int)sizeof(T);   // elements in 16 bytes
};
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));

// The 32-bit words of N values of T (N * sizeof(T) a multiple of 4), and back.
template <typename T, int N>
__device__ __forceinline__ void to_words(const float (&x)[N], unsigned (&wd)[N * sizeof(T) / 4]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < N; ++i) wd[i] = __float_as_uint(x[i]);
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      const unsigned short lo = __builtin_bit_cast(unsigned short, (T)x[2 * i]);
      const unsigned short hi = __builtin_bit_cast(unsigned short, (T)x[2 * i + 1]);
      wd[i] = (unsigned)lo | ((unsigned)hi << 16);
    }
  }
}
template <typename T, int N>
__device__ __forceinline__ void from_words(const unsigned (&wd)[N * sizeof(T) / 4], float (&x)[N]) {
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] = __uint_as_float(wd[i]);
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) {
      x[2 * i] = (float)__builtin_bit_cast(T, (unsigned short)(wd[i] & 0xffffu));
      x[2 * i + 1] = (float)__builtin_bit_cast(T, (unsigned short)(wd[i] >> 16));
    }
  }
}
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
// N floats written as T: N * sizeof(T) bytes (8, 16 or 32) in 16-byte stores and at most one 8-byte store.
template <typename T, int N>
__device__ __forceinline__ void store_as(T* p, const float (&x)[N]) {
  constexpr int NW = N * (int)sizeof(T) / 4;
  static_assert(NW % 2 == 0, "whole 8-byte pieces");
  unsigned wd[NW];
  to_words<T, N>(x, wd);
  unsigned* q = reinterpret_cast<unsigned*>(p);
#pragma unroll
  for (int s = 0; s + 4 <= NW; s += 4)
    *reinterpret_cast<u32x4_t*>(q + s) = u32x4_t{wd[s], wd[s + 1], wd[s + 2], wd[s + 3]};
  if constexpr (NW % 4 == 2) *reinterpret_cast<u32x2_t*>(q + NW - 2) = u32x2_t{wd[NW - 2], wd[NW - 1]};
}
// N values of T from memory as floats, with the same access widths.
template <typename T, int N>
__device__ __forceinline__ void load_as(const T* p, float (&x)[N]) {
  constexpr int NW = N * (int)sizeof(T) / 4;
  static_assert(NW % 2 == 0, "whole 8-byte pieces");
  unsigned wd[NW];
  const unsigned* q = reinterpret_cast<const unsigned*>(p);
#pragma unroll
  for (int s = 0; s + 4 <= NW; s += 4) {
    const u32x4_t r = *reinterpret_cast<const u32x4_t*>(q + s);
#pragma unroll
    for (int i = 0; i < 4; ++i) wd[s + i] = r[i];
  }
  if constexpr (NW % 4 == 2) {
    const u32x2_t r = *reinterpret_cast<const u32x2_t*>(q + NW - 2);
    wd[NW - 2] = r[0];
    wd[NW - 1] = r[1];
  }
  from_words<T, N>(wd, x);
}

// The V16<T>::N values of T in the 16 bytes `raw`, as floats.
template <typename T>
__device__ __forceinline__ void unpack(const u32x4_t& raw, float (&x)[V16<T>::N]) {
  const unsigned wd[4] = {raw[0], raw[1], raw[2], raw[3]};
  from_words<T, V16<T>::N>(wd, x);
}

// ---- the convolution path ----------------------------------------------------------------------------------------
constexpr int CV_TAPS = 4;
constexpr int CV_ROWS = 64;       // output time steps a tile
constexpr int CV_VECS = 8;        // 16-byte channel vectors a tile row
constexpr int CV_THREADS = 256;   // 32 row groups x 8 vectors; a lane computes rows rg and rg + 32
constexpr int CV_HALO = CV_TAPS - 1;

struct ConvArgs {
  const void* x;                  // [B, T, C] in T
  const float* w;                 // [C, 4] float32 taps
  void *q, *k, *v;                // forward outputs: q, k [B, T, KD * REP] in T, v [B, T, C - 2 KD] in TV
  const void *dq, *dk, *dv;       // backward inputs, same layouts
  void* dx;                       // [B, T, C] in T
  float* part;                    // [B * ntiles, C * 4] per-tile taps' gradient, or null
  int B, T, C, KD, DK, REP, ntiles;
};

// Where a 16-byte channel vector lives among the outputs: q, k (key heads, each written REP times: REP = 1 keeps key
// heads only) or v.  A vector never straddles a head (head widths are multiples of the vector).
struct Dest {
  int which;                      // 0 q, 1 k, 2 v
  size_t pitch;                   // row pitch of the destination (elements)
  size_t col;                     // the vector's first column there (copy 0)
  __device__ Dest(int c, int KD, int DK, int REP, int C) {
    if (c < 2 * KD) {
      which = c < KD ? 0 : 1;
      const int cc = c - which * KD;
      pitch = (size_t)KD * REP;
      col = (size_t)(cc / DK) * REP * DK + cc % DK;
    } else {
      which = 2;
      pitch = (size_t)(C - 2 * KD);
      col = (size_t)(c - 2 * KD);
    }
  }
};

// The tile's taps, tap-major: tw[j][i] = w[c + i, j] for the lane's N channels.
template <int N>
__device__ __forceinline__ void tile_taps(const float* w, int c, float (&tw)[CV_TAPS][N]) {
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const f4 r = *reinterpret_cast<const f4*>(w + (size_t)(c + i) * CV_TAPS);
#pragma unroll
    for (int j = 0; j < CV_TAPS; ++j) tw[j][i] = r[j];
  }
}

// sum_j tw[j][i] win[j][i], j = 3 first.  float32 inputs (EXACT) sum in double and round once, so that the result is
// within an ulp of the exact value (their error bar is twice PyTorch's fp32 path); 2-byte inputs sum in float, whose
// rounding is far below the output's.
template <bool EXACT, int N>
__device__ __forceinline__ float tap_dot(const float (&tw)[CV_TAPS][N], int i, float w0, float w1, float w2, float w3) {
  if constexpr (EXACT) {
    double s = (double)tw[3][i] * (double)w3;
    s = fma((double)tw[2][i], (double)w2, s);
    s = fma((double)tw[1][i], (double)w1, s);
    return (float)fma((double)tw[0][i], (double)w0, s);
  } else {
    return fmaf(tw[0][i], w0, fmaf(tw[1][i], w1, fmaf(tw[2][i], w2, tw[3][i] * w3)));
  }
}
template <bool EXACT>
__device__ __forceinline__ float logistic(float u) {
  if constexpr (EXACT) return 1.0f / (1.0f + expf(-u));
  else return __frcp_rn(1.0f + __expf(-u));
}
// u sigmoid(u) with one rounding after the exponential for float32 inputs (a division, not u times a rounded
// reciprocal, whose two roundings put the float32 output past twice PyTorch's silu error)
template <bool EXACT>
__device__ __forceinline__ float silu(float u) {
  if constexpr (EXACT) return u / (1.0f + expf(-u));
  else return u * __frcp_rn(1.0f + __expf(-u));
}

// Stage rows [t_lo, t_lo + NROWS) x the tile's CV_VECS vectors of x (batch row b) into LDS by asynchronous 16-byte
// copies (global -> LDS, no registers), all of a thread's issued back to back; units outside [0, T) or past the
// channels are zeroed by LDS stores instead.  Unit u = row * CV_VECS + vector.  The caller waits (wait_copies) and
// synchronises before reading.
template <typename T, int NROWS>
__device__ __forceinline__ void stage_x(u32x4_t* dst, const T* xb, int t_lo, int c0, int T_, int C) {
  constexpr int VE = V16<T>::N;
  constexpr int UNITS = NROWS * CV_VECS, PER = (UNITS + CV_THREADS - 1) / CV_THREADS;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int u = threadIdx.x + i * CV_THREADS;
    if (u < UNITS) {
      const int row = u / CV_VECS, c = c0 + (u % CV_VECS) * VE, t = t_lo + row;
      if (t >= 0 && t < T_ && c < C)
        __builtin_amdgcn_global_load_lds((const void*)(xb + (size_t)t * C + c),
                                         (__attribute__((address_space(3))) void*)(dst + u - threadIdx.x % 64), 16,
                                         0, 0);
      else
        dst[u] = u32x4_t{0u, 0u, 0u, 0u};
    }
  }
}
__device__ __forceinline__ void wait_copies() { __builtin_amdgcn_s_waitcnt(0); }

// The forward needs no staging: a lane owns one 16-byte channel vector over CV_FWD_STEPS consecutive time steps and
// issues the loads of all its CV_FWD_STEPS + 3 input rows at once (the 3 halo rows come again through L2), then forms
// each output from them.  A wave spans 64 consecutive vectors (1 KB of a bf16 row), a workgroup four consecutive time
// blocks.  Measured at config 1's widths this ran at the box's mixed read/write rate, ahead of LDS-staged tiles (whose
// staging and barrier put each tile's loads and stores in separate phases).
constexpr int CV_FWD_STEPS = 8;
template <typename T, typename TV>
__global__ void __launch_bounds__(256) conv_fwd_kernel(ConvArgs a) {
  constexpr int VE = V16<T>::N;
  constexpr bool EXACT = sizeof(T) == 4;
  constexpr int NR = CV_FWD_STEPS + CV_HALO;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = (blockIdx.x * 64 + lane) * VE;
  const int t0 = (blockIdx.y * 4 + wave) * CV_FWD_STEPS, b = blockIdx.z;
  if (c >= a.C || t0 >= a.T) return;
  const T* xb = (const T*)a.x + (size_t)b * a.T * a.C + c;
  u32x4_t raw[NR];                                    // x[t0 - 3 + i], zero outside the sequence
#pragma unroll
  for (int i = 0; i < NR; ++i) {
    const int t = t0 - CV_HALO + i;
    raw[i] = (t >= 0 && t < a.T) ? *reinterpret_cast<const u32x4_t*>(xb + (size_t)t * a.C) : u32x4_t{0u, 0u, 0u, 0u};
  }
  float tw[CV_TAPS][VE];
  tile_taps<VE>(a.w, c, tw);
  const Dest d(c, a.KD, a.DK, a.REP, a.C);
#pragma unroll
  for (int s = 0; s < CV_FWD_STEPS; ++s) {
    const int t = t0 + s;
    if (t >= a.T) break;
    float w0[VE], w1[VE], w2[VE], w3[VE];             // x[t - 3] .. x[t]
    unpack<T>(raw[s], w0);
    unpack<T>(raw[s + 1], w1);
    unpack<T>(raw[s + 2], w2);
    unpack<T>(raw[s + 3], w3);
    float y[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) y[i] = silu<EXACT>(tap_dot<EXACT, VE>(tw, i, w0[i], w1[i], w2[i], w3[i]));
    const size_t row = (size_t)b * a.T + t;
    if (d.which == 2) {
      store_as<TV, VE>((TV*)a.v + row * d.pitch + d.col, y);
    } else {
      T* dst = (T*)(d.which == 0 ? a.q : a.k) + row * d.pitch + d.col;
      for (int rep = 0; rep < a.REP; ++rep) store_as<T, VE>(dst + (size_t)rep * a.DK, y);
    }
  }
}

// The backward of a tile of 64 output rows t0 .. t0 + 63 (dx there, and the tile's share of the taps' gradient):
//   x staged for t0 - 3 .. t0 + 66, the upstream gradient dy (q's and k's copies summed in copy order) for
//   t0 .. t0 + 66, then du = dy s (1 + u (1 - s)), s = sigmoid(u), in place (0 past the end), then
//   dx[t] = w0 du[t + 3] + w1 du[t + 2] + w2 du[t + 1] + w3 du[t],
//   part[tile][c, j] = sum over the tile's t of du[t] x[t - 3 + j].
template <typename T, typename TV, bool TAPS>
__global__ void __launch_bounds__(CV_THREADS) conv_bwd_tile_kernel(ConvArgs a) {
  constexpr int VE = V16<T>::N;
  constexpr bool EXACT = sizeof(T) == 4;
  constexpr int XR = CV_ROWS + 2 * CV_HALO;          // x rows t0 - 3 .. t0 + 66
  constexpr int DR = CV_ROWS + CV_HALO;              // du rows t0 .. t0 + 66
  __shared__ u32x4_t xs[XR * CV_VECS];
  __shared__ float du[DR * CV_VECS * VE];            // [row][vector][element]
  __shared__ double red[4][32][TAPS ? VE : 1];       // the taps' gradient: one row of partials a wave
  const int c0 = blockIdx.x * CV_VECS * VE, t0 = blockIdx.y * CV_ROWS, b = blockIdx.z;
  const T* xb = (const T*)a.x + (size_t)b * a.T * a.C;
  stage_x<T, XR>(xs, xb, t0 - CV_HALO, c0, a.T, a.C);
  // dy for rows t0 .. t0 + 66 (zero past the end or past the channels): every unit's first-copy load is issued
  // before any is used (a thread's units keep its vector, so they share one destination map)
  {
    constexpr int UNITS = DR * CV_VECS, PER = (UNITS + CV_THREADS - 1) / CV_THREADS;
    const int vec = threadIdx.x % CV_VECS, c = c0 + vec * VE;
    const Dest d(c < a.C ? c : 0, a.KD, a.DK, a.REP, a.C);
    const T* qk = (const T*)(d.which == 0 ? a.dq : a.dk);
    float g[PER][VE];
    bool live[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = threadIdx.x + i * CV_THREADS, t = t0 + u / CV_VECS;
      live[i] = u < UNITS && t < a.T && c < a.C;
      const size_t r = (size_t)b * a.T + (live[i] ? t : 0);
      if (d.which == 2) load_as<TV, VE>((const TV*)a.dv + r * d.pitch + d.col, g[i]);
      else load_as<T, VE>(qk + r * d.pitch + d.col, g[i]);
    }
    if (d.which != 2)
      for (int rep = 1; rep < a.REP; ++rep)   // the other copies of a repeated key head, added in copy order
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int t = t0 + (threadIdx.x + i * CV_THREADS) / CV_VECS;
          const size_t r = (size_t)b * a.T + (live[i] ? t : 0);
          float h[VE];
          load_as<T, VE>(qk + r * d.pitch + d.col + (size_t)rep * a.DK, h);
#pragma unroll
          for (int e = 0; e < VE; ++e) g[i][e] += h[e];
        }
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int u = threadIdx.x + i * CV_THREADS;
      if (u < UNITS)
#pragma unroll
        for (int e = 0; e < VE; ++e) du[u * VE + e] = live[i] ? g[i][e] : 0.f;
    }
  }
  wait_copies();
  __syncthreads();
  float tw[CV_TAPS][VE];
  {
    const int vec = threadIdx.x % CV_VECS, c = c0 + vec * VE;
    if (c < a.C) tile_taps<VE>(a.w, c, tw);
    else
#pragma unroll
      for (int j = 0; j < CV_TAPS; ++j)
#pragma unroll
        for (int i = 0; i < VE; ++i) tw[j][i] = 0.f;
  }
  // du in place: unit u's row sees x rows row .. row + 3 (t - 3 .. t); the lanes of a unit keep their vector, so tw
  // is the lane's own taps
  for (int u = threadIdx.x; u < DR * CV_VECS; u += CV_THREADS) {
    const int row = u / CV_VECS, vec = u % CV_VECS;
    float w0[VE], w1[VE], w2[VE], w3[VE];
    unpack<T>(xs[(row + 0) * CV_VECS + vec], w0);
    unpack<T>(xs[(row + 1) * CV_VECS + vec], w1);
    unpack<T>(xs[(row + 2) * CV_VECS + vec], w2);
    unpack<T>(xs[(row + 3) * CV_VECS + vec], w3);
#pragma unroll
    for (int i = 0; i < VE; ++i) {
      const float uu = tap_dot<EXACT, VE>(tw, i, w0[i], w1[i], w2[i], w3[i]);
      const float s = logistic<EXACT>(uu);
      du[u * VE + i] *= s * (1.0f + uu * (1.0f - s));   // dy was staged there (0 past the end)
    }
  }
  __syncthreads();

  // dx for the lane's rows rg, rg + 32
  {
    const int vec = threadIdx.x % CV_VECS, rg = threadIdx.x / CV_VECS, c = c0 + vec * VE;
    if (c < a.C) {
      T* dxb = (T*)a.dx + (size_t)b * a.T * a.C + c;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int r = rg + 32 * h, t = t0 + r;
        if (t >= a.T) break;
        float o[VE];
        const float* d0 = du + ((r + 3) * CV_VECS + vec) * VE;   // du[t + 3]
        const float* d1 = du + ((r + 2) * CV_VECS + vec) * VE;
        const float* d2 = du + ((r + 1) * CV_VECS + vec) * VE;
        const float* d3 = du + ((r + 0) * CV_VECS + vec) * VE;   // du[t]
#pragma unroll
        for (int i = 0; i < VE; ++i) o[i] = tap_dot<EXACT, VE>(tw, i, d0[i], d1[i], d2[i], d3[i]);
        store_as<T, VE>(dxb + (size_t)t * a.C, o);
      }
    }
  }
  if constexpr (TAPS) {
    // combo = (vector, tap) = lane % 32; part = thread / 32 sums rows 8 part .. 8 part + 7 in double
    const int combo = threadIdx.x % 32, part = threadIdx.x / 32, vec = combo % CV_VECS, j = combo / CV_VECS;
    double acc[VE];
#pragma unroll
    for (int i = 0; i < VE; ++i) acc[i] = 0.0;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int r = 8 * part + s;                     // x[t - 3 + j] is staged row r + j
      float xv[VE];
      unpack<T>(xs[(r + j) * CV_VECS + vec], xv);
      const float* dd = du + (r * CV_VECS + vec) * VE;
#pragma unroll
      for (int i = 0; i < VE; ++i) acc[i] = fma((double)dd[i], (double)xv[i], acc[i]);
    }
    // parts 2w and 2w + 1 are lanes l and l + 32 of wave w: add them, then the four waves in order through LDS
#pragma unroll
    for (int i = 0; i < VE; ++i) acc[i] += __shfl_xor(acc[i], 32, 64);
    const int w = threadIdx.x / 64;
    if ((threadIdx.x & 63) < 32)
#pragma unroll
      for (int i = 0; i < VE; ++i) red[w][combo][i] = acc[i];
    __syncthreads();
    if (threadIdx.x < 32) {
      const int c = c0 + vec * VE;
      if (c < a.C) {
        float* out = a.part + (size_t)(b * a.ntiles + blockIdx.y) * a.C * CV_TAPS;
#pragma unroll
        for (int i = 0; i < VE; ++i)
          out[(size_t)(c + i) * CV_TAPS + j] =
              (float)(((red[0][combo][i] + red[1][combo][i]) + red[2][combo][i]) + red[3][combo][i]);
      }
    }
  }
}

// out[i] = the sum over rows p = 0 .. P - 1 of in[p * n + i], in row order, in double, rounded once: the fixed-order
// second stage of the taps' gradient.  A lane an output; each row's loads for a group of eight rows are in flight
// together.
__global__ void __launch_bounds__(256) sum_columns_kernel(const float* in, float* out, int P, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  double s = 0.0;
  int p = 0;
  for (; p + 8 <= P; p += 8) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = in[(size_t)(p + e) * n + i];
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (double)v[e];
  }
  for (; p < P; ++p) s += (double)in[(size_t)p * n + i];
  out[i] = (float)s;
}

// ---- the gates -----------------------------------------------------------------------------------------------------
// PyTorch's softplus with threshold 20: x above it, log1p(exp(x)) below; and its derivative with the same
// threshold: 1 above it, sigmoid(x) below.  The gates compute in double, a + dt_bias included, and round each result
// once: they are a few elements a token-head, so the kernels are bound by latency, and in float32 the sums', the
// exponentials' and the quotients' roundings put the gradients at up to twice the PyTorch path's error on short
// rows.
__device__ __forceinline__ double softplus_t20(double x) { return x > 20.0 ? x : log1p(exp(x)); }
__device__ __forceinline__ double softplus_t20_grad(double x) { return x > 20.0 ? 1.0 : 1.0 / (1.0 + exp(-x)); }

// The gates move under a megabyte per layer, so they are bound by latency, not bandwidth: one element a lane, so
// that a layer's elements spread over every lane of the chip and each lane runs one exponential chain.
constexpr int GATE_THREADS = 256;
template <typename T>
__global__ void __launch_bounds__(GATE_THREADS) gates_fwd_kernel(const T* b, const T* a, const float* alog,
                                                                 const float* dtb, float* beta, float* g, int64_t n,
                                                                 int H) {
  const int64_t i = (int64_t)blockIdx.x * GATE_THREADS + threadIdx.x;
  if (i >= n) return;
  const int head = (int)(i % H);             // heads run fastest: element i is head i mod H
  const double rate = -exp((double)alog[head]);
  beta[i] = (float)(1.0 / (1.0 + exp(-(double)(float)b[i])));
  g[i] = (float)(rate * softplus_t20((double)(float)a[i] + (double)dtb[head]));
}

template <typename T>
__global__ void __launch_bounds__(GATE_THREADS) gates_bwd_kernel(const T* b, const T* a, const float* alog,
                                                                 const float* dtb, const float* dbeta,
                                                                 const float* dg, T* db, T* da, int64_t n, int H) {
  const int64_t i = (int64_t)blockIdx.x * GATE_THREADS + threadIdx.x;
  if (i >= n) return;
  const int head = (int)(i % H);
  const double rate = -exp((double)alog[head]);
  const double sig = 1.0 / (1.0 + exp(-(double)(float)b[i]));
  db[i] = (T)(float)((double)dbeta[i] * (sig - sig * sig));          // d sigmoid = s (1 - s)
  da[i] = (T)(float)((double)dg[i] * rate * softplus_t20_grad((double)(float)a[i] + (double)dtb[head]));
}

// dA_log[h] = sum over rows of dg g and ddt[h] = sum over rows of dg (-exp(A_log)) softplus'(a + dt_bias): one
// workgroup a head; thread i takes rows i, i + 256, ... in order, then a wave sums its lanes by a fixed butterfly and
// the four waves add in order.  Deterministic.  Terms and sums in double, rounded once: a head's rows of dg carry both
// signs, so the sums can cancel.
template <typename T>
__global__ void __launch_bounds__(256) gates_params_kernel(const T* a, const float* alog, const float* dtb,
                                                           const float* dg, float* dA, float* ddt, int64_t rows,
                                                           int H) {
  const int h = blockIdx.x;
  const double rate = -exp((double)alog[h]), bias = (double)dtb[h];
  double s_a = 0.0, s_d = 0.0;
  for (int64_t r = threadIdx.x; r < rows; r += 256) {
    const int64_t i = r * H + h;
    const double x = (double)(float)a[i] + bias, gv = (double)dg[i];
    s_a = fma(gv, rate * softplus_t20(x), s_a);
    s_d = fma(gv, rate * softplus_t20_grad(x), s_d);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    s_a += __shfl_xor(s_a, off, 64);
    s_d += __shfl_xor(s_d, off, 64);
  }
  __shared__ double wa[4], wd[4];
  if ((threadIdx.x & 63) == 0) {
    wa[threadIdx.x >> 6] = s_a;
    wd[threadIdx.x >> 6] = s_d;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    dA[h] = (float)(((wa[0] + wa[1]) + wa[2]) + wa[3]);
    ddt[h] = (float)(((wd[0] + wd[1]) + wd[2]) + wd[3]);
  }
}

}  // namespace gdr

using namespace gdr;

namespace {

int check_conv(const char* what, int64_t B, int64_t T, int64_t C, int64_t KD, int64_t DK, int64_t REP, int64_t DV,
               int32_t dtype, int32_t vdtype) {
  constexpr int64_t T_MAX = (int64_t)65535 * 4 * CV_FWD_STEPS;   // the forward's grid rows of time blocks
  if (B < 1 || T < 1 || B > 65535 || T > T_MAX)
    return fail(MACAI_GDR_EINVAL, "%s: B in [1, 65535] and T in [1, %lld] (got %lld, %lld)", what, (long long)T_MAX,
                (long long)B, (long long)T);
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

int64_t conv_tiles(int64_t T) { return (T + CV_ROWS - 1) / CV_ROWS; }

// the launch grid of the conv kernels for element size es: channel tiles, time tiles, batch rows
dim3 conv_grid(int64_t B, int64_t T, int64_t C, int es) {
  const int64_t per = (int64_t)CV_VECS * (16 / es);
  return dim3((unsigned)((C + per - 1) / per), (unsigned)conv_tiles(T), (unsigned)B);
}

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
  ConvArgs a{x, w, q, k, v, nullptr, nullptr, nullptr, nullptr, nullptr, (int)B, (int)T, (int)C, (int)KD, (int)DK,
             (int)REP, (int)conv_tiles(T)};
  hipStream_t st = (hipStream_t)stream;
  const int es = dtype == MACAI_GDR_F32 ? 4 : 2;
  const dim3 grid((unsigned)((C / (16 / es) + 63) / 64), (unsigned)((T + 4 * CV_FWD_STEPS - 1) / (4 * CV_FWD_STEPS)),
                  (unsigned)B);
  DISPATCH_PT(dtype, DISPATCH_PV(vdtype, hipLaunchKernelGGL((conv_fwd_kernel<PT, PV>), grid, dim3(256), 0, st, a)))
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
  const int ntiles = (int)conv_tiles(T);
  ConvArgs a{x, w, nullptr, nullptr, nullptr, dq, dk, dv, dx, dwp, (int)B, (int)T, (int)C, (int)KD, (int)DK,
             (int)REP, ntiles};
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid = conv_grid(B, T, C, dtype == MACAI_GDR_F32 ? 4 : 2);
  if (dwp) {
    DISPATCH_PT(dtype, DISPATCH_PV(vdtype, hipLaunchKernelGGL((conv_bwd_tile_kernel<PT, PV, true>), grid,
                                                              dim3(CV_THREADS), 0, st, a)))
  } else {
    DISPATCH_PT(dtype, DISPATCH_PV(vdtype, hipLaunchKernelGGL((conv_bwd_tile_kernel<PT, PV, false>), grid,
                                                              dim3(CV_THREADS), 0, st, a)))
  }
  if (int rc = launched(what)) return rc;
  if (dw) {
    const int n = (int)(C * CV_TAPS);
    hipLaunchKernelGGL(sum_columns_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dwp, dw,
                       (int)(B * ntiles), n);
    return launched(what);
  }
  return MACAI_GDR_OK;
}

int64_t macai_gdr_conv_partials(int64_t B, int64_t T, int64_t C) { return B * conv_tiles(T) * C * CV_TAPS; }

int macai_gdr_gates_fwd(const void* b, const void* a, const float* A_log, const float* dt_bias, float* beta, float* g,
                        int64_t n, int64_t H, int32_t dtype, void* stream) {
  const char* what = "macai_gdr_gates_fwd";
  if (n < 1 || H < 1 || n % H) return fail(MACAI_GDR_EINVAL, "%s: need n >= 1 a multiple of H >= 1", what);
  if (dtype < MACAI_GDR_F32 || dtype > MACAI_GDR_F16) return fail(MACAI_GDR_EUNSUP, "%s: dtype code", what);
  if (!b || !a || !A_log || !dt_bias || !beta || !g) return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  const void* ps[] = {b, a, beta, g};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((n + GATE_THREADS - 1) / GATE_THREADS));
  DISPATCH_PT(dtype, hipLaunchKernelGGL((gates_fwd_kernel<PT>), grid, dim3(GATE_THREADS), 0, st, (const PT*)b,
                                        (const PT*)a, A_log, dt_bias, beta, g, n, (int)H))
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
  const void* ps[] = {b, a, dbeta, dg, db, da};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)((n + GATE_THREADS - 1) / GATE_THREADS));
  DISPATCH_PT(dtype, hipLaunchKernelGGL((gates_bwd_kernel<PT>), grid, dim3(GATE_THREADS), 0, st, (const PT*)b,
                                        (const PT*)a, A_log, dt_bias, dbeta, dg, (PT*)db, (PT*)da, n, (int)H))
  if (int rc = launched(what)) return rc;
  if (dA_log) {
    DISPATCH_PT(dtype, hipLaunchKernelGGL((gates_params_kernel<PT>), dim3((unsigned)H), dim3(256), 0, st,
                                          (const PT*)a, A_log, dt_bias, dg, dA_log, ddt_bias, n / H, (int)H))
    return launched(what);
  }
  return MACAI_GDR_OK;
}

}  // extern "C"

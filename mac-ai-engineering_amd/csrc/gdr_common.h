// Device helpers shared by the gated-delta-rule kernels (gfx950 / CDNA4, wave64).
//
// MFMA tiles.  Every product is built from 16 x 16 output tiles accumulated in fp32 over 32-deep k-blocks:
//   * fp32 operands: 8 x v_mfma_f32_16x16x4_f32 per k-block;
//   * bf16 operands: 1 x v_mfma_f32_16x16x32_bf16 per k-block.
// Lane l (j = l / 16) holds, for an A operand, row l % 16 and the 8 k-values kmap(j, 0..7); for a B operand, column
// l % 16 and the same 8 k-values.  kmap(j, r) = 4j + r for r < 4 and 16 + 4j + (r - 4) for r >= 4: the same bijection
// of the k-block is used for A and B, so any of them gives the product.  It is chosen so that the fp32 accumulator of
// a 16 x 16 tile (lane l, register r holds D[4j + r][l % 16]) -- two tiles stacked along k -- IS a B-operand fragment
// (rows = k) and an A-operand fragment of the transpose, with no data movement: the state S and the per-token
// corrections stay in registers across the sequential chunk loop.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdr {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

constexpr int C = 64;          // chunk length (tokens); one wave lane per chunk row in the scans
constexpr float L2_EPS = 1e-6f; // l2norm epsilon of the reference prologue (_norm.py:17)

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }

// Workgroup barrier for LDS data: each wave's LDS accesses complete (lgkmcnt(0)) before s_barrier, and the compiler
// moves no memory access across it.  Unlike __syncthreads() it does not wait for outstanding global loads and stores,
// nor for asynchronous global->LDS copies (vmcnt): the waves that issued a copy wait for it (wait_vmcnt / wait_dma)
// before the barrier that publishes its tile.  (A workgroup release fence on LDS would wait for every copy in flight.)
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);      // lgkmcnt(0); vmcnt and expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// ---- scalar conversions -------------------------------------------------------------------------------------------
__device__ __forceinline__ float to_f(float x) { return x; }
__device__ __forceinline__ float to_f(bf16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f(float x);
template <> __device__ __forceinline__ float from_f<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f<bf16>(float x) { return (bf16)x; }

// ---- fragments ----------------------------------------------------------------------------------------------------
__device__ __forceinline__ int kmap(int j, int r) { return r < 4 ? 4 * j + r : 12 + 4 * j + r; }

template <typename MT> struct Frag;
template <> struct Frag<float> {
  float v[8];
  __device__ __forceinline__ void set(int r, float x) { v[r] = x; }
  __device__ __forceinline__ float get(int r) const { return v[r]; }
};
template <> struct Frag<bf16> {
  bf16x8 v;
  __device__ __forceinline__ void set(int r, float x) { v[r] = (bf16)x; }
  __device__ __forceinline__ float get(int r) const { return (float)v[r]; }
};

__device__ __forceinline__ void mma(f4& acc, const Frag<float>& a, const Frag<float>& b) {
#pragma unroll
  for (int r = 0; r < 8; ++r) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.v[r], b.v[r], acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f4& acc, const Frag<bf16>& a, const Frag<bf16>& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, acc, 0, 0, 0);
}

// 4 contiguous values from memory (global or LDS) as floats
__device__ __forceinline__ f4 load4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ f4 load4(const bf16* p) {
  bf16x4 x = *reinterpret_cast<const bf16x4*>(p);
  return f4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
}
// 4 contiguous values to memory (one 16-byte store for fp32, one 8-byte store for bf16)
template <typename T> __device__ __forceinline__ void store4(T* p, const f4& x);
template <> __device__ __forceinline__ void store4<float>(float* p, const f4& x) { *reinterpret_cast<f4*>(p) = x; }
template <> __device__ __forceinline__ void store4<bf16>(bf16* p, const f4& x) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)x[0], (bf16)x[1], (bf16)x[2], (bf16)x[3]};
}

// Fragment of a k-contiguous ("row-major along k") matrix X: lane takes row `row0 + l % 16`, k-block at k0.  For an A
// operand X = A ([m][k]); for a B operand X = B^T ([n][k]).  `scale` multiplies the values before rounding to MT.
template <typename MT, typename ST>
__device__ __forceinline__ Frag<MT> frag_k(const ST* base, int pitch, int row0, int k0, float scale = 1.0f,
                                           int l = lane_id()) {
  const int j = l >> 4;
  const ST* p = base + (size_t)(row0 + (l & 15)) * pitch + k0 + 4 * j;
  f4 lo = load4(p), hi = load4(p + 16);
  Frag<MT> f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    f.set(r, lo[r] * scale);
    f.set(r + 4, hi[r] * scale);
  }
  return f;
}

// Specialisation for bf16 LDS/global data feeding bf16 MFMA without a scale: plain 8-byte moves.
__device__ __forceinline__ Frag<bf16> frag_k_raw(const bf16* base, int pitch, int row0, int k0, int l = lane_id()) {
  const int j = l >> 4;
  const bf16* p = base + (size_t)(row0 + (l & 15)) * pitch + k0 + 4 * j;
  bf16x4 lo = *reinterpret_cast<const bf16x4*>(p), hi = *reinterpret_cast<const bf16x4*>(p + 16);
  Frag<bf16> f;
  f.v = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return f;
}
__device__ __forceinline__ Frag<float> frag_k_raw(const float* base, int pitch, int row0, int k0) {
  return frag_k<float, float>(base, pitch, row0, k0);
}

// Fragment from two stacked accumulator tiles (rows 0-15 in `lo`, rows 16-31 in `hi`): B operand with k = the tiles'
// rows, or A operand of their transpose.
template <typename MT>
__device__ __forceinline__ Frag<MT> frag_acc(const f4& lo, const f4& hi, float scale = 1.0f) {
  Frag<MT> f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    f.set(r, lo[r] * scale);
    f.set(r + 4, hi[r] * scale);
  }
  return f;
}

// hi/lo split of fp32 values for bf16 MFMA: x = hi + lo with both representable in bf16 (relative residual ~2^-16)
template <typename MT>
__device__ __forceinline__ void frag_split(const Frag<float>& x, Frag<MT>& hi, Frag<MT>& lo) {
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    float h = (float)from_f<MT>(x.v[r]);
    hi.set(r, h);
    lo.set(r, x.v[r] - h);
  }
}

// fp32 fragment of a k-contiguous fp32 matrix (no rounding), for split products
__device__ __forceinline__ Frag<float> frag_k_f32(const float* base, int pitch, int row0, int k0, int l = lane_id()) {
  return frag_k<float, float>(base, pitch, row0, k0, 1.0f, l);
}

// ---- wave-level scans and reductions -------------------------------------------------------------------------------
// Inclusive scans over the wave's 64 lanes by DPP (GFX9), with no LDS round trip: in-row shifts by 1, 2, 4, 8 (a lane
// whose source falls before its 16-lane row adds 0), then lane 15's sum into rows 1 and 3 (row_bcast:15) and lane
// 31's into rows 2 and 3 (row_bcast:31) -- the published GCN cross-lane scan (AMD GPUOpen, "AMD GCN Assembly:
// Cross-Lane Operations").  Rows a mask leaves out receive 0.
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ int dpp_z(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, ROWS, 0xF, true);
}
enum : int { DPP_ROW_SHR1 = 0x111, DPP_ROW_SHR2 = 0x112, DPP_ROW_SHR4 = 0x114, DPP_ROW_SHR8 = 0x118,
             DPP_ROW_BCAST15 = 0x142, DPP_ROW_BCAST31 = 0x143, DPP_WAVE_SHR1 = 0x138 };
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_zf(float x) { return __int_as_float(dpp_z<CTRL, ROWS>(__float_as_int(x))); }
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ double dpp_zd(double x) {
  const long long b = __double_as_longlong(x);
  const int lo = dpp_z<CTRL, ROWS>((int)b), hi = dpp_z<CTRL, ROWS>((int)(b >> 32));
  return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
__device__ __forceinline__ float wave_incl_scan(float x, int = 0) {
  x += dpp_zf<DPP_ROW_SHR1>(x);
  x += dpp_zf<DPP_ROW_SHR2>(x);
  x += dpp_zf<DPP_ROW_SHR4>(x);
  x += dpp_zf<DPP_ROW_SHR8>(x);
  x += dpp_zf<DPP_ROW_BCAST15, 0xA>(x);
  x += dpp_zf<DPP_ROW_BCAST31, 0xC>(x);
  return x;
}
// x of lane l - 1 (0 in lane 0)
__device__ __forceinline__ float wave_shift_up1(float x) { return dpp_zf<DPP_WAVE_SHR1>(x); }
// lane permutations inside each 16-lane DPP row (no LDS round trip): quad_perm [1,0,3,2] and [2,3,0,1], row_half_mirror
// (lane i <-> 7 - i within each 8), row_mirror (i <-> 15 - i)
enum : int { DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140 };
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, true));
}
// sum over the 16 lanes of a lane group (lanes with equal l / 16), result in every lane of the group.  A pairwise tree:
// pairs, quads, halves, the row; every lane of the group ends with the same bits.
__device__ __forceinline__ float group16_sum(float x) {
  x += dpp<DPP_XOR1>(x);
  x += dpp<DPP_XOR2>(x);
  x += dpp<DPP_HALF_MIRROR>(x);
  x += dpp<DPP_MIRROR>(x);
  return x;
}
// Eight sums over the 16 lanes of a lane group at once, by a butterfly that halves the values at every exchange
// (partners l ^ 15, l ^ 7, l ^ 2, l ^ 1 -- they span the group): lane l returns the group's sum of v[(l % 16) / 2];
// lanes l and l ^ 1 hold the same bits.  30 VALU operations where eight group16_sum take 64.
__device__ __forceinline__ float group16_sum8(const float (&v)[8], int l = lane_id()) {
  const int i = l & 15;
  const bool b3 = i & 8, b2 = i & 4, b1 = i & 2;
  float u[4], w[2];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float keep = b3 ? v[4 + k] : v[k], send = b3 ? v[k] : v[4 + k];
    u[k] = keep + dpp<DPP_MIRROR>(send);
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const float keep = b2 ? u[2 + k] : u[k], send = b2 ? u[k] : u[2 + k];
    w[k] = keep + dpp<DPP_HALF_MIRROR>(send);
  }
  const float keep = b1 ? w[1] : w[0], send = b1 ? w[0] : w[1];
  const float x = keep + dpp<DPP_XOR2>(send);
  return x + dpp<DPP_XOR1>(x);
}
// sum over lanes with equal l % 16 (the 4 lane groups), result in every lane: x + x[l ^ 16], then the same with
// l ^ 32, by gfx950's row swaps (v_permlane16_swap: odd 16-lane rows of one copy with even rows of the other;
// v_permlane32_swap: the halves), which exchange lanes in registers where a shuffle goes through LDS
__device__ __forceinline__ float across_groups_sum(float x) {
  const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  const auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

// ---- chunk scalars ------------------------------------------------------------------------------------------------
// One wave: lane t = chunk row t.  g is the log decay (0 on padding rows).  G (the in-chunk cumulative log decay) is
// scanned in double: under strong decay |G| reaches ~1e3 within a chunk, where one fp32 ulp (6e-5) would become a
// relative error of exp(G_i - G_j) -- the decays are formed from the double differences.  G_last is G of the last
// valid row exactly (padding rows copy it), so e = exp(G_last - G) is exactly 1 on that row.
struct __attribute__((aligned(16))) ChunkScalars {   // 16-byte aligned: rows are read 4 at a time
  double G[C];
  float gam[C];    // exp(G_r)
  float e[C];      // exp(G_last - G_r)
  float beta[C];
  // exp(G_i - G_j) for i >= j (masked before the exponent by the caller)
  __device__ __forceinline__ float decay(int i, int j) const { return expf((float)(G[i] - G[j])); }
};

__device__ __forceinline__ double wave_incl_scan_d(double x) {
  x += dpp_zd<DPP_ROW_SHR1>(x);
  x += dpp_zd<DPP_ROW_SHR2>(x);
  x += dpp_zd<DPP_ROW_SHR4>(x);
  x += dpp_zd<DPP_ROW_SHR8>(x);
  x += dpp_zd<DPP_ROW_BCAST15, 0xA>(x);
  x += dpp_zd<DPP_ROW_BCAST31, 0xC>(x);
  return x;
}

// from this lane's g and beta (0 past the sequence end)
__device__ __forceinline__ void chunk_scalars_from(ChunkScalars& cs, float gv, float bv, int t0, int T,
                                                   int l = lane_id()) {
  const int last = (T - t0 < C ? T - t0 : C) - 1;
  double G = wave_incl_scan_d((double)gv);
  const long long gb = __double_as_longlong(G);   // G of the last valid row, read from its lane (last is uniform)
  const double Gl = __longlong_as_double(((long long)__builtin_amdgcn_readlane((int)(gb >> 32), last) << 32) |
                                         (unsigned)__builtin_amdgcn_readlane((int)gb, last));
  if (l > last) G = Gl;
  cs.G[l] = G;
  cs.gam[l] = (float)exp(G);
  cs.e[l] = (float)exp(Gl - G);
  cs.beta[l] = bv;
}
__device__ __forceinline__ void chunk_scalars(ChunkScalars& cs, const float* g, const float* beta, size_t row_base,
                                              size_t row_stride, int t0, int T) {
  const int t = t0 + lane_id();
  float gv = 0.f, bv = 0.f;
  if (t < T) {
    gv = g[row_base + (size_t)t * row_stride];
    if (beta) bv = beta[row_base + (size_t)t * row_stride];
  }
  chunk_scalars_from(cs, gv, bv, t0, T);
}

// ---- row norms ----------------------------------------------------------------------------------------------------
// 1 / sqrt(|x_r|^2 + eps) of chunk rows r (the prologue's l2norm, eps 1e-6), 0 past the sequence end.  One pass covers
// 16 rows per wave: lane l takes row l / 4 and sums the squares of x[r][32 s + 8 (l % 4) + i] in (s, i) order; the
// four partial sums of a row combine as (a + b) + (c + d) in every lane.  The global and the LDS versions follow the
// same order, so every kernel computes the same bits.
__device__ __forceinline__ float row4_sum(float x) {
  const float y = x + dpp<DPP_XOR1>(x);
  return y + dpp<DPP_XOR2>(y);
}
template <typename IT, int D>
__device__ __forceinline__ void row_rnorms(float* out, const IT* x, size_t row_base, size_t row_stride, int t0, int T,
                                           int nwaves, int w = wave_id()) {
  const int l = lane_id(), part = l & 3;
  for (int r0 = 16 * w; r0 < C; r0 += 16 * nwaves) {
    const int r = r0 + (l >> 2), t = t0 + r;
    const IT* p = x + row_base + (size_t)(t < T ? t : T - 1) * row_stride + 8 * part;   // rows past T: masked below
    float ss = 0.f;
#pragma unroll
    for (int st = 0; st < D / 32; ++st)
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = to_f(p[32 * st + i]);
        ss = fmaf(v, v, ss);
      }
    ss = row4_sum(ss);
    if (part == 0) out[r] = (t < T) ? 1.0f / sqrtf(ss + L2_EPS) : 0.f;
  }
}
// The same over a bf16 tile already in LDS (row pitch `pitch` elements; rows < nrows, 0 past them).
template <int D>
__device__ __forceinline__ void row_rnorms_lds(float* out, const bf16* tile, int pitch, int nrows, int nwaves, int w,
                                               int l = lane_id()) {
  const int part = l & 3;
  for (int r0 = 16 * w; r0 < C; r0 += 16 * nwaves) {
    const int r = r0 + (l >> 2);
    const bf16* p = tile + r * pitch + 8 * part;   // rows past nrows hold copies of a valid row: masked below
    float ss = 0.f;
#pragma unroll
    for (int st = 0; st < D / 32; ++st) {
      // two 8-byte reads (rows need only be 8-byte aligned), the same summation order
      const bf16x4 x0 = *reinterpret_cast<const bf16x4*>(p + 32 * st), x1 = *reinterpret_cast<const bf16x4*>(p + 32 * st + 4);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = (float)(i < 4 ? x0[i] : x1[i - 4]);
        ss = fmaf(v, v, ss);
      }
    }
    ss = row4_sum(ss);
    if (part == 0) out[r] = (r < nrows) ? 1.0f / sqrtf(ss + L2_EPS) : 0.f;
  }
}

// ---- global I/O helpers -------------------------------------------------------------------------------------------
template <typename T> __device__ __forceinline__ void store(T* p, float x) { *p = from_f<T>(x); }

}  // namespace gdr

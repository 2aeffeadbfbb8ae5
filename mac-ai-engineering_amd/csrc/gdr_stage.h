// Global -> LDS staging of chunk tiles and fragment loaders that read global memory directly (gfx950).
#pragma once
#include "gdr_common.h"

namespace gdr {

// 8 consecutive elements from global memory as floats
__device__ __forceinline__ void load8(const float* p, float* x) {
  f4 a = *reinterpret_cast<const f4*>(p), b = *reinterpret_cast<const f4*>(p + 4);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    x[i] = a[i];
    x[i + 4] = b[i];
  }
}
__device__ __forceinline__ void load8(const bf16* p, float* x) {
  bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (float)a[i];
}
// 8 consecutive MT values into LDS (16-byte aligned for bf16, two 16-byte stores for fp32)
__device__ __forceinline__ void store8(float* p, const float* x) {
  *reinterpret_cast<f4*>(p) = f4{x[0], x[1], x[2], x[3]};
  *reinterpret_cast<f4*>(p + 4) = f4{x[4], x[5], x[6], x[7]};
}
__device__ __forceinline__ void store8(bf16* p, const float* x) {
  bf16x8 a;
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = (bf16)x[i];
  *reinterpret_cast<bf16x8*>(p) = a;
}

// dst[r][0..ncols) (pitch dp, MT) = src[t0 + r][0..ncols) * scale(r)   for r < C; rows t0 + r >= T are zero.
// src points at row 0 of the sequence (row pitch `pitch` elements).  ncols is a multiple of 8.
template <typename MT, typename IT, typename F>
__device__ __forceinline__ void stage_rows(MT* dst, int dp, const IT* src, size_t pitch, int t0, int T, int ncols,
                                           F scale) {
  const int pr = ncols >> 3;
  for (int i = threadIdx.x; i < C * pr; i += blockDim.x) {
    const int r = i / pr, c8 = (i - r * pr) << 3;
    const int t = t0 + r;
    float x[8];
    if (t < T) {
      load8(src + (size_t)t * pitch + c8, x);
      const float s = scale(r);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= s;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.f;
    }
    store8(dst + r * dp + c8, x);
  }
}

// Transposed: dst[c][r] (pitch dp) = src[t0 + r][c] * scale(r); rows t0 + r >= T are zero.
template <typename MT, typename IT, typename F>
__device__ __forceinline__ void stage_rows_T(MT* dst, int dp, const IT* src, size_t pitch, int t0, int T, int ncols,
                                             F scale) {
  const int pr = ncols >> 3;
  for (int i = threadIdx.x; i < C * pr; i += blockDim.x) {
    const int r = i % C, c8 = (i / C) << 3;   // consecutive threads take consecutive rows: spreads LDS banks
    const int t = t0 + r;
    float x[8];
    if (t < T) {
      load8(src + (size_t)t * pitch + c8, x);
      const float s = scale(r);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= s;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[(c8 + e) * dp + r] = from_f<MT>(x[e]);
  }
}

// Plain copy of a dense [nrows][ncols] MT block (global, pitch = ncols) into LDS (pitch dp).
template <typename MT>
__device__ __forceinline__ void stage_copy(MT* dst, int dp, const MT* src, int nrows, int ncols) {
  const int pr = ncols >> 3;
  for (int i = threadIdx.x; i < nrows * pr; i += blockDim.x) {
    const int r = i / pr, c8 = (i - r * pr) << 3;
    float x[8];
    load8(src + (size_t)r * ncols + c8, x);
    store8(dst + r * dp + c8, x);
  }
}
// Transposed copy: dst[c][r] = src[r][c] for a dense [nrows][ncols] MT block.
template <typename MT>
__device__ __forceinline__ void stage_copy_T(MT* dst, int dp, const MT* src, int nrows, int ncols) {
  const int pr = ncols >> 3;
  for (int i = threadIdx.x; i < nrows * pr; i += blockDim.x) {
    const int r = i % nrows, c8 = (i / nrows) << 3;
    float x[8];
    load8(src + (size_t)r * ncols + c8, x);
#pragma unroll
    for (int e = 0; e < 8; ++e) dst[(c8 + e) * dp + r] = from_f<MT>(x[e]);
  }
}

// Fragment of a k-contiguous matrix in global memory whose rows are sequence rows: lane row = row0 + l % 16 (relative
// to the chunk start t0); rows with t0 + row >= T give zeros.  Row r is multiplied by rs(r).
template <typename MT, typename ST, typename F>
__device__ __forceinline__ Frag<MT> frag_k_seq(const ST* src, size_t pitch, int t0, int T, int row0, int k0, F rs) {
  const int l = lane_id(), j = l >> 4;
  const int r = row0 + (l & 15);
  Frag<MT> f;
  if (t0 + r < T) {
    const ST* p = src + (size_t)(t0 + r) * pitch + k0 + 4 * j;
    f4 lo = load4(p), hi = load4(p + 16);
    const float s = rs(r);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f.set(e, lo[e] * s);
      f.set(e + 4, hi[e] * s);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) f.set(e, 0.f);
  }
  return f;
}

// Fragment whose k index runs over ROWS of a row-major matrix (B operand with k = row, or A operand of a transpose):
// slot r takes row krow0 + kmap(j, r), column col.  Rows with t0 + row >= T give zeros; row r is scaled by rs(r).
template <typename MT, typename ST, typename F>
__device__ __forceinline__ Frag<MT> frag_rows(const ST* src, size_t pitch, int t0, int T, int krow0, int col, F rs) {
  const int l = lane_id(), j = l >> 4;
  Frag<MT> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int r = krow0 + kmap(j, e);
    float x = 0.f;
    if (t0 + r < T) x = to_f(src[(size_t)(t0 + r) * pitch + col]) * rs(r);
    f.set(e, x);
  }
  return f;
}

// frag_rows with its eight loads issued unconditionally (a row past the end reads row T - 1; the caller's chunk has
// t0 < T) and masked after.  In frag_rows each load sits in a per-row branch and the compiler waits for it before the
// branch closes, so the eight loads do not overlap: this form took the float32 per-chunk backward from 410 to 342 us
// at config 1.  Where registers are already short (key width 256, which spills) the loads it holds in flight made
// that kernel 20% slower, so it is not the default.
template <typename MT, typename ST, typename F>
__device__ __forceinline__ Frag<MT> frag_rows_eager(const ST* src, size_t pitch, int t0, int T, int krow0, int col,
                                                    F rs) {
  const int l = lane_id(), j = l >> 4;
  ST raw[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int t = t0 + krow0 + kmap(j, e);
    raw[e] = src[(size_t)(t < T ? t : T - 1) * pitch + col];
  }
  Frag<MT> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int r = krow0 + kmap(j, e);
    f.set(e, (t0 + r < T) ? to_f(raw[e]) * rs(r) : 0.f);
  }
  return f;
}

struct One {
  __device__ __forceinline__ float operator()(int) const { return 1.0f; }
};

}  // namespace gdr

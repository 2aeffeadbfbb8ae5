// Asynchronous global -> LDS tile copies (gfx950 global_load_lds_dwordx4) into XOR-swizzled, unpadded LDS tiles.
//
// One wave instruction moves 64 x 16 bytes: lane l writes the 16-byte unit at LDS base + 16 l, from any global address
// of its own.  A tile of R rows x COLS elements is kept in LDS as R * PU 16-byte units (PU units per row, no padding);
// logical unit cu of row r sits at physical unit r * PU + (cu ^ s(r)).  The swizzle s(r) spreads the 16 rows that one
// MFMA fragment read touches over the 16 distinct units of a 256-byte bank window, so fragment reads are free of bank
// conflicts.  The swizzle is applied on the global side (each lane fetches the logical unit that belongs at its
// physical place), so the copy needs no registers and overlaps the MFMA work of the previous chunk.
#pragma once
#include "gdr_common.h"

namespace gdr {

typedef __attribute__((address_space(3))) void lds_void;

template <typename T, int R, int COLS>
struct Swz {
  static constexpr int EPU = 16 / (int)sizeof(T);        // elements per 16-byte unit
  static constexpr int PU = COLS / EPU;                   // units per row
  static constexpr int NU = R * PU;                       // units in the tile
  static constexpr int NI = NU / 64;                      // wave instructions to copy it
  static constexpr int ELEMS = NU * EPU;                  // elements (LDS footprint / sizeof(T))
  static constexpr int RW = PU >= 16 ? 1 : 16 / PU;       // rows per 256-byte window
  static constexpr int SM = PU >= 16 ? 15 : PU - 1;       // swizzle mask
  static_assert(COLS % EPU == 0 && NU % 64 == 0, "tile must be a whole number of 1 KiB wave copies");

  __device__ static __forceinline__ int s(int row) { return (row / RW) & SM; }
  __device__ static __forceinline__ int offset(int row, int col) {
    return (row * PU + ((col / EPU) ^ s(row))) * EPU + (col % EPU);
  }
  // Copy a global tile (row r at g + r * gpitch; rows >= nrows re-read row nrows - 1, to be masked by the reader) into
  // LDS `base`; waves w, w + nw, ... share the wave instructions.
  __device__ static __forceinline__ void dma(T* base, const T* g, size_t gpitch, int w, int nw, int nrows = R) {
    const int l = lane_id();
    for (int i = w; i < NI; i += nw) {
      const int u = i * 64 + l;
      const int row = u / PU, cu = (u % PU) ^ s(row);
      const int rr = row < nrows ? row : nrows - 1;
      __builtin_amdgcn_global_load_lds((const void*)(g + (size_t)rr * gpitch + cu * EPU),
                                       (lds_void*)(base + i * 64 * EPU), 16, 0, 0);
    }
  }
};

// Fragment (A operand rows, or B operand columns = rows of B^T) of a k-contiguous swizzled tile.
template <typename MT, typename G>
__device__ __forceinline__ Frag<MT> frag_swz(const MT* base, int row0, int k0) {
  const int l = lane_id(), j = l >> 4, row = row0 + (l & 15);
  const MT* lo = base + G::offset(row, k0 + 4 * j);
  const MT* hi = base + G::offset(row, k0 + 16 + 4 * j);
  Frag<MT> f;
  if constexpr (sizeof(MT) == 2) {
    bf16x4 a = *reinterpret_cast<const bf16x4*>(lo), b = *reinterpret_cast<const bf16x4*>(hi);
    f.v = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  } else {
    f4 a = *reinterpret_cast<const f4*>(lo), b = *reinterpret_cast<const f4*>(hi);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f.set(r, a[r]);
      f.set(r + 4, b[r]);
    }
  }
  return f;
}

// Fragment whose k runs over the ROWS of a swizzled tile (B operand with k = row): slot r = row krow0 + kmap(j, r),
// column col; rows with t0 + row >= T read as zero.
template <typename MT, typename T, typename G>
__device__ __forceinline__ Frag<MT> frag_swz_rows(const T* base, int krow0, int col, int t0, int Tn) {
  const int l = lane_id(), j = l >> 4;
  Frag<MT> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int row = krow0 + kmap(j, e);
    f.set(e, (t0 + row < Tn) ? to_f(base[G::offset(row, col)]) : 0.f);
  }
  return f;
}

__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0); }

}  // namespace gdr

// Asynchronous global -> LDS tile copies (gfx950 global_load_lds_dwordx4) into padded LDS tiles.
//
// One wave instruction moves 64 x 16 bytes: lane l writes the 16-byte unit at LDS base + 16 l, from any global address
// of its own.  A tile of R rows x COLS elements is kept in LDS with one pad unit after every row (PU data units + 1):
// the DMA simply skips the pad units (those lanes re-read a valid address of the tile), and the odd row pitch spreads
// the 16 rows an MFMA fragment read touches over distinct LDS banks.  A fragment read is then a per-lane base plus
// compile-time offsets -- no address arithmetic per read -- and the copy needs no registers and overlaps MFMA work.
#pragma once
#include "gdr_common.h"

namespace gdr {

typedef __attribute__((address_space(3))) void lds_void;

template <typename T, int R, int COLS>
struct Tile {
  static constexpr int EPU = 16 / (int)sizeof(T);        // elements per 16-byte unit
  static constexpr int PU = COLS / EPU;                   // data units per row
  static constexpr int RU = PU + 1;                       // units per row with the pad unit
  static constexpr int PITCH = RU * EPU;                  // row pitch in elements
  static constexpr int NI = (R * RU + 63) / 64;           // wave instructions to copy the tile
  static constexpr int ELEMS = NI * 64 * EPU;             // LDS footprint in elements
  static_assert(COLS % EPU == 0, "tile rows must be whole 16-byte units");

  __device__ static __forceinline__ int offset(int row, int col) { return row * PITCH + col; }
  static constexpr int per_wave(int nw) { return (NI + nw - 1) / nw; }

  // The element offsets (from the tile's global base, row pitch gpitch) that this lane copies in the wave's
  // instructions w, w + NW, ...: the same for every chunk of a dense tile, so the sequential passes compute them once.
  template <int NW>
  __device__ static __forceinline__ void plan(int (&off)[per_wave(NW)], int w, int gpitch) {
    const int l = lane_id();
#pragma unroll
    for (int k = 0; k < per_wave(NW); ++k) {
      const int i = w + k * NW;
      const int u = i * 64 + l, row = u / RU, cu = u - row * RU;
      off[k] = (i < NI && row < R && cu < PU) ? row * gpitch + cu * EPU : 0;
    }
  }
  template <int NW>
  __device__ static __forceinline__ void dma_planned(T* base, const T* g, const int (&off)[per_wave(NW)], int w) {
#pragma unroll
    for (int k = 0; k < per_wave(NW); ++k) {
      const int i = w + k * NW;
      if (i < NI)
        __builtin_amdgcn_global_load_lds((const void*)(g + off[k]), (lds_void*)(base + i * 64 * EPU), 16, 0, 0);
    }
  }
  // Copy a global tile (row r at g + r * gpitch; rows >= nrows re-read row nrows - 1, to be masked by the reader) into
  // LDS `base`; waves w, w + nw, ... share the wave instructions.
  __device__ static __forceinline__ void dma(T* base, const T* g, size_t gpitch, int w, int nw, int nrows = R) {
    const int l = lane_id();
    for (int i = w; i < NI; i += nw) {
      const int u = i * 64 + l;
      const int row = u / RU, cu = u - row * RU;
      const T* src = g;
      if (row < R && cu < PU) src = g + (size_t)(row < nrows ? row : nrows - 1) * gpitch + cu * EPU;
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(base + i * 64 * EPU), 16, 0, 0);
    }
  }
};

// Fragment (A operand rows, or B operand columns = rows of B^T) of a k-contiguous tile.
template <typename MT, typename G>
__device__ __forceinline__ Frag<MT> frag_tile(const MT* base, int row0, int k0) {
  const int l = lane_id(), j = l >> 4;
  const MT* p = base + (row0 + (l & 15)) * G::PITCH + k0 + 4 * j;
  Frag<MT> f;
  if constexpr (sizeof(MT) == 2) {
    bf16x4 a = *reinterpret_cast<const bf16x4*>(p), b = *reinterpret_cast<const bf16x4*>(p + 16);
    f.v = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  } else {
    f4 a = *reinterpret_cast<const f4*>(p), b = *reinterpret_cast<const f4*>(p + 16);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f.set(r, a[r]);
      f.set(r + 4, b[r]);
    }
  }
  return f;
}

// Fragment whose k runs over the ROWS of a tile (B operand with k = row): slot r = row krow0 + kmap(j, r), column col.
template <typename MT, typename G>
__device__ __forceinline__ Frag<MT> frag_tile_rows(const MT* base, int krow0, int col) {
  const int l = lane_id(), j = l >> 4;
  const MT* p = base + (krow0 + 4 * j) * G::PITCH + col;
  Frag<MT> f;
#pragma unroll
  for (int e = 0; e < 8; ++e) f.set(e, to_f(p[(e < 4 ? e : 12 + e) * G::PITCH]));
  return f;
}

__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0); }

}  // namespace gdr

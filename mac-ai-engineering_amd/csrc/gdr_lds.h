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
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// SW (bf16 tiles of whole 128-byte row blocks): odd rows hold the two 64-byte halves of every 128-byte block swapped --
// LDS unit u of row r holds the row's unit u ^ (4 (r & 1)).  A row pitch of whole 16-byte units puts the 16 rows of a
// fragment read two to a bank group; with the swap the 8-byte fragment reads run conflict-free (measured on gfx950:
// 142-144 against 70-72 bytes a clock a CU at 272- and 144-byte pitches; transpose reads 126-128 against 131-134).
// Swapping single 16-byte units instead measured as fast in LDS but made the copies slow: each 64-byte run of the
// copy's lanes must stay in address order.  The readers (frag_tile, frag_tile_tr) take the swap from the layout.
template <typename T, int R, int COLS, bool SW = false>
struct Tile {
  static constexpr int EPU = 16 / (int)sizeof(T);        // elements per 16-byte unit
  static constexpr int PU = COLS / EPU;                   // data units per row
  static constexpr int RU = PU + 1;                       // units per row with the pad unit
  static constexpr int PITCH = RU * EPU;                  // row pitch in elements
  static constexpr int NI = (R * RU + 63) / 64;           // wave instructions to copy the tile
  static constexpr int ELEMS = NI * 64 * EPU;             // LDS footprint in elements
  static constexpr bool SWZ = SW;
  static_assert(COLS % EPU == 0, "tile rows must be whole 16-byte units");
  static constexpr int SWK = SW ? 4 : 0;                 // odd rows: LDS unit u holds the row's unit u ^ SWK
  static_assert(!SW || (sizeof(T) == 2 && PU % 8 == 0), "unit swap: bf16 rows of whole 128-byte blocks");

  // the row's data unit that LDS unit cu (< PU) of row `row` holds
  __device__ static __forceinline__ int src_unit(int row, int cu) { return cu ^ (SWK * (row & 1)); }
  __device__ static __forceinline__ int offset(int row, int col) {
    return row * PITCH + src_unit(row, col / EPU) * EPU + col % EPU;
  }
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
      off[k] = (i < NI && row < R && cu < PU) ? row * gpitch + src_unit(row, cu) * EPU : 0;
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
  // dma() with every wave issuing exactly per_wave(NW) copy instructions, unrolled and branch-free (a wave past the
  // tile's last instruction repeats it, writing the same bytes again), so that the number of loads a wave has issued
  // after the copy is a compile-time constant and a partial vmcnt wait can follow it.  The copies are buffer loads
  // (buffer_load_dwordx4 ... lds, LDS base in M0) rather than global_load_lds: with a FLAT-encoded copy in flight the
  // compiler can no longer order the vector-memory counter and waits for zero before every use of a loaded register.
  // Byte offsets within the tile must fit 31 bits.
  template <int NW>
  __device__ static __forceinline__ void dma_exact(T* base, const T* g, size_t gpitch, int w, int nrows = R,
                                                   int l = lane_id()) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void*)g, 0, 0x7fffffff, 0x00020000);
#pragma unroll
    for (int k = 0; k < per_wave(NW); ++k) {
      const int i = w + k * NW < NI ? w + k * NW : NI - 1;
      const int u = i * 64 + l;
      const int row = u / RU, cu = u - row * RU;
      int off = 0;
      if (row < R && cu < PU) off = (int)(((size_t)(row < nrows ? row : nrows - 1) * gpitch + src_unit(row, cu) * EPU) * sizeof(T));
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)(base + i * 64 * EPU), 16, off, 0, 0, 0);
    }
  }
  // dma_exact() issued through inline assembly, unseen by the compiler: it then does not make every later LDS read
  // wait for the copy (which it does for a copy into LDS it knows of).  The caller waits for it explicitly (wait_dma,
  // wait_vmcnt) before the barrier that publishes the tile.  The buffer resource is dma_exact's (base g, no stride,
  // 2^31 - 1 bytes, the same flags word); M0 holds the LDS address of the instruction's 64 x 16 bytes.
  template <int NW>
  __device__ static __forceinline__ void dma_exact_opaque(T* base, const T* g, size_t gpitch, int w, int nrows = R,
                                                          int l = lane_id()) {
    const unsigned long long ga = (unsigned long long)(const void*)g;
    const u32x4 rs = {(unsigned)__builtin_amdgcn_readfirstlane((unsigned)ga),
                      (unsigned)__builtin_amdgcn_readfirstlane((unsigned)(ga >> 32) & 0xffffu), 0x7fffffffu, 0x00020000u};
#pragma unroll
    for (int k = 0; k < per_wave(NW); ++k) {
      const int i = w + k * NW < NI ? w + k * NW : NI - 1;
      const int u = i * 64 + l;
      const int row = u / RU, cu = u - row * RU;
      int off = 0;
      if (row < R && cu < PU) off = (int)(((size_t)(row < nrows ? row : nrows - 1) * gpitch + src_unit(row, cu) * EPU) * sizeof(T));
      const unsigned lds = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_void*)(base + i * 64 * EPU));
      // s_nop: one wait state between an SALU write of M0 and an LDS-DMA read of it
      asm volatile("s_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(off), "s"(rs), "{m0}"(lds) : "memory");
    }
  }
  // The same copy through registers, one instruction's unit at a time: load_unit(k) reads the 16 bytes that
  // dma_exact's k-th instruction of wave w would move for this lane, store_unit(k) writes them to the same LDS place.
  // Loads issued this way are ordinary register loads, so they can be spread between other work without the compiler
  // treating every LDS read as dependent on them (which it does for copies into LDS in flight).
  template <int NW>
  __device__ static __forceinline__ u32x4 load_unit(const T* g, size_t gpitch, int w, int k, int nrows = R,
                                                    int l = lane_id()) {
    const int i = w + k * NW < NI ? w + k * NW : NI - 1;
    const int u = i * 64 + l;
    const int row = u / RU, cu = u - row * RU;
    const T* src = g;
    if (row < R && cu < PU) src = g + (size_t)(row < nrows ? row : nrows - 1) * gpitch + src_unit(row, cu) * EPU;
    return *reinterpret_cast<const u32x4*>(src);
  }
  template <int NW>
  __device__ static __forceinline__ void store_unit(T* base, int w, int k, u32x4 x, int l = lane_id()) {
    const int i = w + k * NW < NI ? w + k * NW : NI - 1;
    *reinterpret_cast<u32x4*>(base + i * 64 * EPU + l * EPU) = x;
  }
  // Copy a global tile (row r at g + r * gpitch; rows >= nrows re-read row nrows - 1, to be masked by the reader) into
  // LDS `base`; waves w, w + nw, ... share the wave instructions.
  __device__ static __forceinline__ void dma(T* base, const T* g, size_t gpitch, int w, int nw, int nrows = R) {
    const int l = lane_id();
    for (int i = w; i < NI; i += nw) {
      const int u = i * 64 + l;
      const int row = u / RU, cu = u - row * RU;
      const T* src = g;
      if (row < R && cu < PU) src = g + (size_t)(row < nrows ? row : nrows - 1) * gpitch + src_unit(row, cu) * EPU;
      __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(base + i * 64 * EPU), 16, 0, 0);
    }
  }
};

// The layout of a dense row-major [R][COLS] tile in global memory (no pad unit): the fragment readers below take it
// in place of a Tile where a chunk's tiles are read straight from memory instead of LDS.
template <typename T, int R, int COLS>
struct Dense {
  static constexpr int PITCH = COLS;
  static constexpr bool SWZ = false;
};

// Fragment (A operand rows, or B operand columns = rows of B^T) of a k-contiguous tile.
template <typename MT, typename G>
__device__ __forceinline__ Frag<MT> frag_tile(const MT* base, int row0, int k0, int l = lane_id()) {
  const int j = l >> 4;
  const MT* p = base + (row0 + (l & 15)) * G::PITCH + k0 + 4 * j;
  if constexpr (G::SWZ) {                  // the two 8-byte pieces from their swapped units
    const int r = row0 + (l & 15);
    Frag<MT> f;
    const bf16x4 a = *reinterpret_cast<const bf16x4*>(base + G::offset(r, k0 + 4 * j)),
                 b = *reinterpret_cast<const bf16x4*>(base + G::offset(r, k0 + 16 + 4 * j));
    f.v = bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    return f;
  }
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

// Wait until at most N vector-memory operations of this wave are outstanding (gfx9 s_waitcnt: vmcnt in bits 3:0 and
// 15:14, expcnt and lgkmcnt left at their maxima).  Loads retire in issue order, so this waits for everything issued
// before the last N.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// A bf16 tile of R rows copied one row per wave instruction, 4 bytes a lane (buffer_load_dword ... lds, lane l
// writes dword l of the row), so its row pitch need only be a multiple of 4 bytes: COLS + 12 elements, an odd
// number of 8-byte units.  At that pitch both the fragment reads (16 rows at one column, 8 bytes a lane) and the
// transpose reads are free of bank conflicts; a pitch of whole 16-byte units (what a 16-byte copy needs) halves the
// fragment reads (measured on gfx950 at 128 columns: 135 B/clk a CU at pitch 140, 72 at 136, 36 at 144).  The copies
// are issued through inline assembly, unseen by the compiler (see Tile::dma_exact_opaque): the caller waits.
template <int R, int COLS>
struct RowTile {
  static constexpr int PITCH = COLS + 12;
  static constexpr int ELEMS = R * PITCH;
  static constexpr bool SWZ = false;
  static constexpr int rows_per_wave(int nw) { return (R + nw - 1) / nw; }
  template <int NW>
  __device__ static __forceinline__ void dma_rows_opaque(bf16* base, const bf16* g, size_t gpitch, int w, int nrows,
                                                         int l) {
    static_assert(COLS % 2 == 0 && COLS / 2 <= 64 && R % NW == 0, "one row of at most 64 dwords a wave instruction");
    const unsigned long long ga = (unsigned long long)(const void*)g;
    const u32x4 rs = {(unsigned)__builtin_amdgcn_readfirstlane((unsigned)ga),
                      (unsigned)__builtin_amdgcn_readfirstlane((unsigned)(ga >> 32) & 0xffffu), 0x7fffffffu, 0x00020000u};
    const unsigned lds0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_void*)base);
    const bool active = COLS / 2 == 64 || l < COLS / 2;
#pragma unroll
    for (int k = 0; k < R / NW; ++k) {
      const int row = w + k * NW;
      const int off = (int)(((size_t)(row < nrows ? row : nrows - 1) * gpitch + 2 * l) * sizeof(bf16));
      const unsigned lds = lds0 + (unsigned)(row * PITCH * (int)sizeof(bf16));
      if (active)
        asm volatile("s_nop 0\n\tbuffer_load_dword %0, %1, 0 offen lds" : : "v"(off), "s"(rs), "{m0}"(lds) : "memory");
    }
  }
};

// A bf16 tile staged through registers at the same conflict-free pitch as RowTile (COLS + 12): lane l of a wave
// instruction takes 16-byte unit l % PU (PU = COLS / 8) of row l / PU of its 64 / PU rows, and writes it to LDS as two
// 8-byte halves (rows are 8-byte aligned).  Rows past nrows re-read row nrows - 1 (masked by the reader).
template <int R, int COLS>
struct RegRowTile {
  static constexpr int PITCH = COLS + 12;
  static constexpr int ELEMS = R * PITCH;
  static constexpr bool SWZ = false;
  static constexpr int PU = COLS / 8;
  static constexpr int RI = 64 / PU;
  static constexpr int NRI = R / RI;
  static constexpr int rows_per_wave(int nw) { return (NRI + nw - 1) / nw; }
  template <int NW>
  __device__ static __forceinline__ u32x4 load_row_unit(const bf16* g, size_t gpitch, int w, int k, int nrows, int l) {
    static_assert((PU & (PU - 1)) == 0 && PU <= 64 && R % RI == 0, "row units: PU a power of two");
    const int i = w + k * NW < NRI ? w + k * NW : NRI - 1;
    const int row = i * RI + l / PU, cu = l % PU;
    return *reinterpret_cast<const u32x4*>(g + (size_t)(row < nrows ? row : nrows - 1) * gpitch + cu * 8);
  }
  template <int NW>
  __device__ static __forceinline__ void store_row_unit(bf16* base, int w, int k, u32x4 x, int l) {
    const int i = w + k * NW < NRI ? w + k * NW : NRI - 1;
    unsigned* p = reinterpret_cast<unsigned*>(base + (i * RI + l / PU) * PITCH + (l % PU) * 8);
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    reinterpret_cast<u32x2*>(p)[0] = u32x2{x[0], x[1]};
    reinterpret_cast<u32x2*>(p)[1] = u32x2{x[2], x[3]};
  }
};

// ---- gfx950 LDS transpose reads (ds_read_b64_tr_b16) ---------------------------------------------------------------
// In each 16-lane group, lane s supplies the address of 4 consecutive 16-bit elements; lane i receives element i % 4 of
// the 4 elements supplied by lanes 4e + i / 4, e = 0..3 (its result element e).  So if lane s points at
// X[r0 + s / 4][c0 + 4 (s % 4)] of a row-major matrix, lane i receives X[r0 + e][c0 + i], e = 0..3: four consecutive
// rows of column c0 + i.  Addresses must be 8-byte aligned.
typedef __attribute__((address_space(3))) bf16x4* lds_bf16x4;
__device__ __forceinline__ bf16x4 read_tr(const bf16* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4)(p));
}
// Fragment whose k runs over the ROWS of a row-major bf16 matrix X[k][n] (B operand with k = row, or A operand of X^T):
// lane l (j = l / 16) takes column n0 + l % 16 and rows k0 + kmap(j, 0..7).  Two transpose reads.
__device__ __forceinline__ Frag<bf16> frag_tr(const bf16* X, int pitch, int k0, int n0, int l = lane_id()) {
  const int j = l >> 4, s = l & 15;
  const bf16* p = X + (k0 + 4 * j + (s >> 2)) * pitch + n0 + 4 * (s & 3);
  const bf16x4 lo = read_tr(p), hi = read_tr(p + 16 * pitch);
  Frag<bf16> f;
  f.v = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return f;
}
// frag_tr over a tile with swapped units (Tile with SW; k0 even): rows k0 + 4 j + s / 4 and 16 below it have the
// same parity, so both reads take the same swap
template <typename G>
__device__ __forceinline__ Frag<bf16> frag_tr_sw(const bf16* X, int k0, int n0, int l = lane_id()) {
  const int j = l >> 4, s = l & 15;
  const bf16* p = X + G::offset(k0 + 4 * j + (s >> 2), n0 + 4 * (s & 3));
  const bf16x4 lo = read_tr(p), hi = read_tr(p + 16 * G::PITCH);
  Frag<bf16> f;
  f.v = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return f;
}
// The fragment of X^T for a row-major tile X of layout G: k over X's rows k0.., the lane's column n0 + l % 16.  LDS
// transpose reads for bf16; element gathers for fp32 (no transpose read exists for 32-bit data).
template <typename MT, typename G>
__device__ __forceinline__ Frag<MT> frag_tile_tr(const MT* base, int k0, int n0) {
  if constexpr (G::SWZ) return frag_tr_sw<G>(base, k0, n0);
  else if constexpr (sizeof(MT) == 2) return frag_tr(base, G::PITCH, k0, n0);
  else return frag_tile_rows<MT, G>(base, k0, n0 + (lane_id() & 15));
}
// The accumulator layout of a 16 x 16 block of a row-major bf16 matrix X: lane l gets X[r0 + 4j + e][c0 + l % 16],
// e = 0..3, as floats.  One transpose read.
__device__ __forceinline__ f4 acc_tr(const bf16* X, int pitch, int r0, int c0) {
  const int l = lane_id(), j = l >> 4, s = l & 15;
  const bf16x4 x = read_tr(X + (r0 + 4 * j + (s >> 2)) * pitch + c0 + 4 * (s & 3));
  return f4{(float)x[0], (float)x[1], (float)x[2], (float)x[3]};
}

// Storing a wave's 64 x 16 block of bf16 results held in accumulator layout (lane l: rows 16 mi + 4 j + r, column
// l % 16) as whole 16-byte row pieces instead of 16 two-byte stores per lane: the lane's values go to a per-wave LDS
// staging area and come back by rows.  A wave's LDS accesses execute in order, so no barrier is involved.
struct ColStage {
  static constexpr int P = 24;                   // row pitch (elements): 48 bytes, 16-byte aligned rows
  static constexpr int ELEMS = 64 * P;
};
// NTL = 2 or 4 accumulator tiles (32 or 64 rows) X[0 .. NTL).
template <int NTL>
__device__ __forceinline__ void store_rows(bf16* stg, bf16* g, size_t gpitch, const f4* X) {
  static_assert(NTL == 2 || NTL == 4, "store_rows: 32 or 64 rows");
  const int l = lane_id(), j = l >> 4, n = l & 15;
#pragma unroll
  for (int mi = 0; mi < NTL; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) stg[(16 * mi + 4 * j + r) * ColStage::P + n] = (bf16)X[mi][r];
#pragma unroll
  for (int k = 0; k < NTL / 2; ++k) {            // 32 NTL units: row u / 2, columns 8 (u % 2) .. + 7
    const int u = 64 * k + l, row = u >> 1, cu = u & 1;
    *reinterpret_cast<u32x4*>(g + row * gpitch + 8 * cu) = *reinterpret_cast<const u32x4*>(stg + row * ColStage::P + 8 * cu);
  }
}
__device__ __forceinline__ void store_cols(bf16* stg, bf16* g, size_t gpitch, const f4 (&X)[4]) {
  store_rows<4>(stg, g, gpitch, X);
}

}  // namespace gdr

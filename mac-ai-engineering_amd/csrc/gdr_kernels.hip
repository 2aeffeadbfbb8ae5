// The chunked gated delta rule for MI355X (gfx950): forward, backward and the one-token decode step.
//
// Kernels (one launch each; C = 64-token chunks; MT = MFMA operand type: fp32 for fp32 inputs, bf16 for bf16 inputs;
// accumulation, the state, decays and the triangular inverse always fp32):
//   prep_kernel       one workgroup per (chunk, head, batch row), all independent.  G (in-chunk cumulative log decay),
//                     L = strictLower(diag(beta) (K K^T) * exp(G_i - G_j)), A = (I + L)^-1 by substitution on 16 x 16
//                     diagonal blocks and block products, W = A diag(beta gamma) K, U = A diag(beta) V, and
//                     M = (Q K^T) * exp(G_i - G_j) (lower with the diagonal).  Replaces the reference's gdc_prep
//                     (/root/reference/src/macai/gated_delta/_chunked.py:220-313), which keeps A and forms no W/U.
//   state_fwd_kernel  one wave per 16 value columns of a head-row, sequential over chunks, the fp32 state S in MFMA
//                     accumulators: Vn = U - W S; O = diag(gamma) Q S + M Vn; S <- exp(G_last) S + K^T diag(e) Vn.
//                     Optionally stores S_c and Vn for the backward (the recompute pass).  Float32 at key widths 64
//                     and 128 with up to two column slices a workgroup carries each slice on two waves, each holding
//                     half the state's rows (state_fwd_ks).  Replaces gdc_fwd (_chunked.py:315-659, flags 1 / 8).
//   state_bwd_kernel  the reverse pass on the same grid, dS in accumulators: dVn = M^T dO + diag(e) K dS;
//                     dS <- exp(G_last) dS + (diag(gamma) Q)^T dO - W^T dVn; stores dS_{c+1}, dVn; writes dS_0
//                     (float32: the key split too, state_bwd_ks).  Replaces gdc_bwd_state (_chunked.py:661-903).
//   chunk_bwd_kernel  one workgroup per (chunk, head, batch row): dq, dk, dv, dg, dbeta with one writer per element
//                     (no atomics), dg in the no-cancellation form, the l2norm prologue's backward fused.  Replaces
//                     gdc_bwd_chunk (_chunked.py:905-1177) and l2n_bwd (_norm.py:44-57).
//   decode_kernel     one token per sequence (T = 1): S' = e^g S + k beta (v - e^g k^T S)^T, o = S'^T q, one
//                     workgroup per head-row streaming the fp32 state once.  The math of op.py:308-313.
// Equations: _chunked.py:1-35; docs/prior_art_gated_delta.md:132-195 of the reference.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <string.h>
#include <stdarg.h>

#include <atomic>
#include <type_traits>

#include "gdr_abi.h"
#include "gdr_common.h"
#include "gdr_stage.h"
#include "gdr_lds.h"
#include "macai_gdr.h"

namespace gdr {

// ---------------------------------------------------------------------------------------------------------------------
// argument blocks (device side)
// ---------------------------------------------------------------------------------------------------------------------
struct PrepArgs {
  const void *q, *k, *v;
  const float *g, *beta;
  void* W;       // [B,H,NT,C,DK] MT   W = A diag(beta gamma) K^
  float* U;      // [B,H,NT,C,DV] fp32 U = A diag(beta) V
  void* Ke;      // [B,H,NT,C,DK] MT   diag(e) K^
  float* GL;     // [B,H,NT]      fp32 exp(G_last)
  void* Qg;      // [B,H,NT,C,DK] MT   diag(gamma) Q^
  void* M;       // [B,H,NT,C,C]  MT   M, row-major [t][s]
  void* A;       // [B,H,NT,C,C]  MT   A                         (or null)
  int B, T, H, DV, NT;
  int l2norm;
  float q_scale;
  int Hk;        // key heads of q, k ([B,T,Hk,DK]); value head h reads key head h / (H / Hk)
  const int* pack;  // packed rows (see chunk_span) or null
  int stagger;   // prep8: the first round's workgroups (two a CU) start staggered
};

struct StateFwdArgs {
  const void *W;
  const float* U;
  const void *Ke;
  const float* GL;
  const void *Qg, *M;
  const float* s0;
  void* o;
  float* sT;
  float* Sc;     // [B,H,NT,DK,DV] fp32 (the backward's <S_c, dS_{c+1}> needs it unrounded)
  void* Vn;      // [B,H,NT,C,DV]  MT
  int B, T, H, DV, NT;
  int nslice;    // workgroups per head-row
  const int* pack;  // packed rows (see chunk_span) or null
  int obf;       // o in bf16 from float32 operands (MACAI_GDR_BF16_F32); 0: o in MT
};

struct StateBwdArgs {
  const void *Ke, *Qg, *W, *M;
  const float* GL;
  const void* dO;
  const float* dsT;
  float* dSn;    // [B,H,NT,DK,DV] f32 dS_{c+1}
  void* dVn;     // [B,H,NT,C,DV]  MT
  float* ds0;    // [B,H,DK,DV]
  int B, T, H, DV, NT;
  int nslice;
  const int* pack;  // packed rows (see chunk_span) or null
};

struct ChunkBwdArgs {
  const void *q, *k, *v;
  const float *g, *beta;
  const void* dO;
  const void* A;                              // MT
  const float* Sc;                            // fp32
  const float* dSn;                           // fp32
  const void *Vn, *dVn;                       // MT
  void *dq, *dk, *dv;                         // dq, dk per VALUE head [B,T,H,DK] (the caller sums a group)
  float *dg, *dbeta;
  int B, T, H, DV, NT;
  int l2norm;
  float q_scale;
  int Hk;                                     // key heads of q, k; value head h reads key head h / (H / Hk)
  const int* pack;                            // packed rows (see chunk_span) or null
  int stagger;                                // chunk_bwd8: the first round's workgroups (one a CU) start staggered
};

// Packed rows (several sequences in one row, cu_seqlens): `pack` holds, for the NT chunks of all sequences, each
// chunk's first token and its sequence's end, then each sequence's first chunk ([t0 x NT | end x NT | c0 x (B + 1)]).
// Token tensors are then [1, T, ...] and per-chunk tensors [1, H, NT, ...]; B counts sequences (the state passes run
// B x H head-rows, each over its sequence's chunks; states are [B, H, DK, DV]).  Without it, chunk c of batch row b
// spans tokens 64 c .. min(64 c + 64, T) of that row.
// A read, through the scalar cache, of memory that no kernel here writes, at a workgroup-uniform address.  Its wait is
// on the LDS / scalar counter, so it never waits for the workgroup's outstanding global stores or copies.
template <typename T>
__device__ __forceinline__ T ld_const(const T* p, size_t i) {
  return ((const __attribute__((address_space(4))) T*)p)[i];
}
// (SCALAR: the table through the scalar cache, for a wave whose waits must not cover its copies in flight.)
template <bool SCALAR = false>
__device__ __forceinline__ void chunk_span(const int* pack, int NT, int c, int T, int& t0, int& tend) {
  if (pack) {
    t0 = SCALAR ? ld_const(pack, c) : pack[c];
    tend = SCALAR ? ld_const(pack, NT + c) : pack[NT + c];
  } else {
    t0 = c * C;
    tend = T;
  }
}
__device__ __forceinline__ void seq_chunks(const int* pack, int NT, int seq, int& cb, int& ce) {
  if (pack) {
    cb = pack[2 * NT + seq];
    ce = pack[2 * NT + seq + 1];
  } else {
    cb = 0;
    ce = NT;
  }
}

struct DecodeArgs {
  const void *q, *k, *v;
  const float *g, *beta, *s_in;
  void* o;
  float* s_out;
  int B, H;
  int l2norm;
  float q_scale;
  int Hk;        // key heads of q, k; value head h reads key head h / (H / Hk)
};

template <typename MT>
__device__ __forceinline__ Frag<MT> cvt(const Frag<float>& x, float s = 1.0f) {
  Frag<MT> f;
#pragma unroll
  for (int r = 0; r < 8; ++r) f.set(r, x.v[r] * s);
  return f;
}

// ---------------------------------------------------------------------------------------------------------------------
// prep: G, L, A = (I + L)^-1, W, U, M per chunk
// ---------------------------------------------------------------------------------------------------------------------
// 8 waves (two a SIMD, hiding each other's latencies): wave w owns row block w % 4 of the 16 x 16 tiles and every
// other column block of it from w / 4 on.
template <typename IT, typename MT, int DK>
__global__ void __launch_bounds__(512) prep_kernel(PrepArgs a) {
  // Key features are staged DKS at a time, so the tiles fit LDS at every key width: the products over the key features
  // accumulate across the passes, and W is formed a pass of columns at a time.  float32 tiles of up to 192 columns
  // fit in one pass (256: two of 128; 224: seven of 32).
  constexpr int DKS = (DK <= 192 || sizeof(MT) == 2) ? DK : (DK % 128 == 0 ? 128 : 32);
  static_assert(DK % DKS == 0 && DKS % 32 == 0, "prep key-column passes");
  constexpr int NPASS = DK / DKS;
  constexpr int KP = DKS + 8;  // pitch of [C][DKS] tiles (elements)
  constexpr int CP = C + 8;    // pitch of [*][C] MT tiles
  constexpr int FP = C + 4;    // pitch of fp32 [C][C] tiles
  constexpr int QSZ = (C * KP > DKS * CP) ? C * KP : DKS * CP;
  constexpr int KSZ = (C * KP > C * CP) ? C * KP : C * CP;
  __shared__ __attribute__((aligned(16))) MT sK[KSZ];    // K^ rows (a pass of columns); then (beta V)^T blocks
  __shared__ __attribute__((aligned(16))) MT sQ[QSZ];    // Q^ rows (a pass); then (beta gamma K^)^T (a pass)
  __shared__ __attribute__((aligned(16))) float sL[C * FP];
  __shared__ __attribute__((aligned(16))) float sA[C * FP];
  __shared__ ChunkScalars cs;
  __shared__ float rk[C], rq[C];

  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int H = a.H, DV = a.DV, NT = a.NT;
  int t0, T;                               // the chunk's first token; T: its sequence's end (the bound for its rows)
  chunk_span(a.pack, NT, c, a.T, t0, T);
  const int l = lane_id(), w = wave_id(), j = l >> 4;
  const size_t qk_base = ((size_t)b * a.T * a.Hk + h / (H / a.Hk)) * DK, qk_pitch = (size_t)a.Hk * DK;
  const size_t v_base = ((size_t)b * a.T * H + h) * DV, v_pitch = (size_t)H * DV;
  const size_t s_base = (size_t)b * a.T * H + h;
  const size_t bhc = ((size_t)b * H + h) * NT + c;
  const IT* q = (const IT*)a.q + qk_base;
  const IT* k = (const IT*)a.k + qk_base;
  const IT* v = (const IT*)a.v + v_base;

  const int rb = w & 3, half = w >> 2;       // row block; which column blocks (every other one from half)
  if (w == 0) chunk_scalars(cs, a.g, a.beta, s_base, H, t0, T);
  if (a.l2norm) {                          // k's norms on waves 0-3, q's on 4-7
    if (w < 4) row_rnorms<IT, DK>(rk, (const IT*)a.k, qk_base, qk_pitch, t0, T, 4, w);
    else row_rnorms<IT, DK>(rq, (const IT*)a.q, qk_base, qk_pitch, t0, T, 4, w - 4);
  } else if (threadIdx.x < C) {
    rk[threadIdx.x] = 1.f;
    rq[threadIdx.x] = 1.f;
  }
  __syncthreads();
  if (threadIdx.x == 0) a.GL[bhc] = cs.gam[C - 1];
  const float qs = a.q_scale;

  // K K^T and Q K^T on the lower 16 x 16 tiles (wave w: row block rb, column blocks half, half + 2), accumulated over
  // the passes of key columns.
  // Each pass stages K^ and Q^ rows of its columns into LDS and writes diag(e) K^ and diag(gamma) Q^ out.
  f4 kk[4], qk[4];
#pragma unroll
  for (int ni = 0; ni < 4; ++ni) kk[ni] = qk[ni] = f4{0.f, 0.f, 0.f, 0.f};
  for (int ps = 0; ps < NPASS; ++ps) {
    const int cb = ps * DKS;               // the pass's first key column
    if (ps) __syncthreads();               // the previous pass's products are done with the tiles
    MT* Ke = (MT*)a.Ke + bhc * C * DK + cb;
    MT* Qg = (MT*)a.Qg + bhc * C * DK + cb;
    // A thread's (row, 8 columns) pieces of the pass: every load issued first, unconditionally (a row past the end
    // reads row T - 1, the chunk having t0 < T) and masked on the row's multiplier after -- in a per-row branch each
    // load was waited for alone.
    constexpr int PR = DKS / 8, NIT = (C * PR + 511) / 512;   // 512 threads (the launch's)
    float lk[NIT][8], lq[NIT][8];
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int i = (int)threadIdx.x + 512 * it;
      if (i < C * PR) {
        const int r = i / PR, c8 = (i - r * PR) * 8, t = (t0 + r < T) ? t0 + r : T - 1;
        load8(k + (size_t)t * qk_pitch + cb + c8, lk[it]);
        load8(q + (size_t)t * qk_pitch + cb + c8, lq[it]);
      }
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int i = (int)threadIdx.x + 512 * it;
      if (i < C * PR) {
        const int r = i / PR, c8 = (i - r * PR) * 8;
        const bool in = t0 + r < T;
        const float mk = in ? rk[r] : 0.f, mq = in ? rq[r] * qs : 0.f;
        float x[8], y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          y[e] = lk[it][e] * mk;
          x[e] = y[e] * cs.e[r];
        }
        store8(sK + r * KP + c8, y);
        store8(Ke + r * DK + c8, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          y[e] = lq[it][e] * mq;
          x[e] = y[e] * cs.gam[r];
        }
        store8(sQ + r * KP + c8, y);
        store8(Qg + r * DK + c8, x);
      }
    }
    __syncthreads();
    const int mi = rb;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      if (ni <= mi && (ni & 1) == half) {
#pragma unroll
        for (int p = 0; p < DKS / 32; ++p) {
          Frag<MT> bk = frag_k_raw(sK, KP, 16 * ni, 32 * p);
          Frag<MT> ak = frag_k_raw(sK, KP, 16 * mi, 32 * p);
          mma(kk[ni], ak, bk);
          mma(qk[ni], frag_k_raw(sQ, KP, 16 * mi, 32 * p), bk);
        }
      }
    }
  }
  // L (strictly lower, fp32) into LDS; M out
  {
    const int mi = rb;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
      if ((ni & 1) != half) continue;
      const int col = 16 * ni + (l & 15);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mi + 4 * j + r;
        const float gm = (row >= col) ? cs.decay(row, col) : 0.f;   // mask before the exponent
        sL[row * FP + col] = (row > col) ? cs.beta[row] * kk[ni][r] * gm : 0.f;
        ((MT*)a.M)[bhc * C * C + row * C + col] = from_f<MT>((row >= col) ? qk[ni][r] * gm : 0.f);
      }
    }
  }
  __syncthreads();

  // (beta gamma K^)^T of key columns [cb, cb + DKS) into LDS for W, from the raw rows (one rounding)
  auto stage_kT = [&](int cb) {
    for (int i = threadIdx.x; i < C * (DKS / 8); i += blockDim.x) {
      const int r = i % C, c8 = (i / C) * 8, t = t0 + r;
      float x[8];
      if (t < T) load8(k + (size_t)t * qk_pitch + cb + c8, x);
      else
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = 0.f;
      const float sb = rk[r] * cs.beta[r] * cs.gam[r];
#pragma unroll
      for (int e = 0; e < 8; ++e) sQ[(c8 + e) * CP + r] = from_f<MT>(x[e] * sb);
    }
  };
  stage_kT(0);

  // A = (I + L)^-1.  Diagonal 16 x 16 blocks by forward substitution: wave 0, lane = (block l/16, column l%16).
  if (w == 0) {
    const int bb = l >> 4, cc = l & 15;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float sacc = (i == cc) ? 1.f : 0.f;
      const float* Lr = sL + (16 * bb + i) * FP + 16 * bb;
#pragma unroll
      for (int m = 0; m < i; ++m) sacc = fmaf(-Lr[m], x[m], sacc);
      x[i] = sacc;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sA[(16 * bb + i) * FP + 16 * bb + cc] = x[i];
  }
  for (int i = threadIdx.x; i < C * C; i += blockDim.x) {
    const int row = i / C, col = i % C;
    if ((col >> 4) > (row >> 4)) sA[row * FP + col] = 0.f;
  }
  __syncthreads();
  // blocks below the diagonal, one block-distance at a time: A_ij = -A_ii sum_{m=j}^{i-1} L_im A_mj (fp32 MFMA)
  for (int dist = 1; dist < 4; ++dist) {
    if (w < 4 - dist) {
      const int bi = w + dist, bj = w;
      f4 t = {0.f, 0.f, 0.f, 0.f};
      for (int m = bj; m < bi; ++m) {
#pragma unroll
        for (int kk2 = 0; kk2 < 16; kk2 += 4)
          t = __builtin_amdgcn_mfma_f32_16x16x4f32(sL[(16 * bi + (l & 15)) * FP + 16 * m + kk2 + j],
                                                   sA[(16 * m + kk2 + j) * FP + 16 * bj + (l & 15)], t, 0, 0, 0);
      }
      f4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 4; ++r)
        o = __builtin_amdgcn_mfma_f32_16x16x4f32(sA[(16 * bi + (l & 15)) * FP + 16 * bi + 4 * j + r], t[r], o, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) sA[(16 * bi + 4 * j + r) * FP + 16 * bj + (l & 15)] = -o[r];
    }
    __syncthreads();
  }

  // W = A (beta gamma K^): wave w owns row block rb, column blocks half, half + 2, ...; A is lower triangular, so
  // k-blocks above the row block are zero
  {
    Frag<MT> af[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) af[p] = cvt<MT>(frag_k_f32(sA, FP, 16 * rb, 32 * p));
    const int np = (16 * rb + 15) / 32 + 1;
    MT* Wc = (MT*)a.W + bhc * C * DK;
    for (int ps = 0; ps < NPASS; ++ps) {
      if (ps) {                            // the next pass of columns of (beta gamma K^)^T
        __syncthreads();
        stage_kT(ps * DKS);
        __syncthreads();
      }
      for (int ni = half; ni < DKS / 16; ni += 2) {
        f4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int p = 0; p < np; ++p) mma(acc, af[p], frag_k_raw(sQ, CP, 16 * ni, 32 * p));
#pragma unroll
        for (int r = 0; r < 4; ++r) Wc[(16 * rb + 4 * j + r) * DK + ps * DKS + 16 * ni + (l & 15)] = from_f<MT>(acc[r]);
      }
    }
    // U = A (beta V), 64 value columns at a time staged transposed in sK
    float* Uc = a.U + bhc * C * DV;
    for (int vb = 0; vb < DV; vb += 64) {
      const int nv = (DV - vb < 64) ? DV - vb : 64;
      __syncthreads();
      stage_rows_T<MT, IT>(sK, CP, v + vb, v_pitch, t0, T, nv, [&](int r) { return cs.beta[r]; });
      __syncthreads();
      for (int ni = half; ni < nv / 16; ni += 2) {
        f4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int p = 0; p < np; ++p) mma(acc, af[p], frag_k_raw(sK, CP, 16 * ni, 32 * p));
#pragma unroll
        for (int r = 0; r < 4; ++r) Uc[(16 * rb + 4 * j + r) * DV + vb + 16 * ni + (l & 15)] = acc[r];
      }
    }
  }
  if (a.A) {
    MT* Ag = (MT*)a.A + bhc * C * C;
    for (int i = threadIdx.x; i < C * C; i += blockDim.x) {
      const int row = i / C, col = i % C;
      Ag[row * C + col] = from_f<MT>(sA[row * FP + col]);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// prep for bf16 operands: 8 waves, the chunk's raw q, k, v in LDS
// ---------------------------------------------------------------------------------------------------------------------
// One workgroup of 8 waves per (chunk, head, batch row), two workgroups per CU (under 80 KB of LDS: A reuses q's tile,
// W is staged in L's), so one's copies and latencies overlap the other's work.  The raw q, k and v rows are copied into
// padded LDS tiles (asynchronous; the chunk scalars are computed meanwhile), so every product reads raw bf16 operands
// and the prologue's scales are applied in fp32 to the products: L and M from q k^T and k k^T, W = (A diag(beta gamma
// rk)) k and U = (A diag(beta)) v, formed transposed (tokens as the MFMA columns) with k and v read by LDS transpose
// reads.  The inverse is the same substitution + block products as prep_kernel.  Ke, Qg, M, A and W leave as whole
// rows; U (fp32) as the accumulators' 4-column quads.  VB = value columns per pass (DV is a multiple of it).
template <int DK, int VB>
__global__ void __launch_bounds__(512) prep8_kernel(PrepArgs a) {
  using MT = bf16;
  constexpr int NW = 8, KP = DK + 8, CP = C + 8, FP = C + 4;
  constexpr int NBD = DK / 16, NBV = VB / 16;
  using GQ = Tile<MT, C, DK>;
  using GV = Tile<MT, C, VB>;
  static_assert(GQ::PITCH == KP && NW == 8 && NBD <= NW && NBV <= NW, "prep8 tiling");
  constexpr int VP = GV::PITCH;
  constexpr int QA = (GQ::ELEMS * 2 > C * FP * 4) ? GQ::ELEMS * 2 : C * FP * 4;   // bytes: q's tile, then A (fp32)
  constexpr int LW = (C * FP * 4 > C * KP * 2) ? C * FP * 4 : C * KP * 2;          // bytes: L (fp32), then W staged
  __shared__ __attribute__((aligned(16))) unsigned char qa[QA];
  __shared__ __attribute__((aligned(16))) MT tk[GQ::ELEMS];
  __shared__ __attribute__((aligned(16))) MT tv[GV::ELEMS];
  __shared__ __attribute__((aligned(16))) unsigned char lw[LW];
  __shared__ __attribute__((aligned(16))) MT sM[C * CP];                            // M staged
  __shared__ ChunkScalars cs;
  __shared__ __attribute__((aligned(16))) float rk[C], rq[C], fW[C], fU[C];

  // The first round of workgroups (a.stagger of them, two a CU) starts in three groups 6.4K cycles apart, as in
  // chunk_bwd8: their loads then do not all hit the memory system at once, and the offsets carry into the later
  // rounds.  Measured on the long prefill's 16 rounds: 2-3% off the kernel; neutral at two rounds.
  if (a.stagger) {
    const unsigned flat = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    if (flat < (unsigned)a.stagger)
      for (int i = 0, n = (int)(flat % 3u) * 50; i < n; ++i) __builtin_amdgcn_s_sleep(2);   // 128 cycles each
  }
  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int H = a.H, DV = a.DV, NT = a.NT;
  int t0, T;                               // the chunk's first token; T: its sequence's end (the bound for its rows)
  chunk_span(a.pack, NT, c, a.T, t0, T);
  const int nrows = (T - t0 < C) ? T - t0 : C;
  const int l = lane_id(), w = wave_id(), j = l >> 4, n = l & 15;
  const size_t qk_base = ((size_t)b * a.T * a.Hk + h / (H / a.Hk)) * DK, qk_pitch = (size_t)a.Hk * DK;
  const size_t v_base = ((size_t)b * a.T * H + h) * DV, v_pitch = (size_t)H * DV;
  const size_t s_base = (size_t)b * a.T * H + h;
  const size_t bhc = ((size_t)b * H + h) * NT + c;
  const MT* q = (const MT*)a.q + qk_base;
  const MT* k = (const MT*)a.k + qk_base;
  const MT* v = (const MT*)a.v + v_base;
  const float qs = a.q_scale;
  MT* const tq = reinterpret_cast<MT*>(qa);
  float* const sA = reinterpret_cast<float*>(qa);   // q's tile is consumed by then
  float* const sL = reinterpret_cast<float*>(lw);
  MT* const stW = reinterpret_cast<MT*>(lw);        // L is consumed by then

  // ---- 0: g and beta read, then the q and k tiles copied, then v's, which is read only from phase 4 on: the waves
  // wait for q and k (a partial wait; copies retire in issue order) and v lands during phases 1a and 1b.  Until then
  // the barriers order LDS only (a workgroup fence would wait for v's copy).  The row norms come from the tiles.
  float gv = 0.f, bv = 0.f;
  if (w == 0) {
    const size_t o = s_base + (size_t)(t0 + l < T ? t0 + l : T - 1) * H;
    gv = a.g[o];
    bv = a.beta[o];
  }
  GQ::template dma_exact<NW>(tq, q + (size_t)t0 * qk_pitch, qk_pitch, w, nrows);
  GQ::template dma_exact<NW>(tk, k + (size_t)t0 * qk_pitch, qk_pitch, w, nrows);
  __builtin_amdgcn_sched_barrier(0);
  GV::template dma_exact<NW>(tv, v + (size_t)t0 * v_pitch, v_pitch, w, nrows);
  __builtin_amdgcn_sched_barrier(0);
  wait_vmcnt<GV::per_wave(NW)>();          // g, beta, q and k have landed
  if (w == 0) {
    asm volatile("" : "+v"(gv), "+v"(bv));  // no arithmetic on g ahead of the copies (it would wait for the load)
    chunk_scalars_from(cs, t0 + l < T ? gv : 0.f, t0 + l < T ? bv : 0.f, t0, T);
  }
  lds_barrier();
  if (a.l2norm) {
    if (w < 4) row_rnorms_lds<DK>(rq, tq, KP, nrows, 4, w);
    else row_rnorms_lds<DK>(rk, tk, KP, nrows, 4, w - 4);
  } else if (threadIdx.x < C) {
    rk[threadIdx.x] = 1.f;
    rq[threadIdx.x] = 1.f;
  }
  if (nrows < C) {                         // rows past the end: zeros in q and k (v's once it has landed)
    constexpr int UQ = KP / 8;
    const int nz = C - nrows;
    for (int i = threadIdx.x; i < nz * 2 * UQ; i += blockDim.x) {
      const int row = nrows + i % nz, u = i / nz;
      *reinterpret_cast<bf16x8*>(u < UQ ? tq + row * KP + 8 * u : tk + row * KP + 8 * (u - UQ)) = bf16x8{};
    }
  }
  lds_barrier();
  if (threadIdx.x < C) {                   // read from phase 3 on, after several barriers
    const int s = threadIdx.x;
    fW[s] = cs.beta[s] * cs.gam[s] * rk[s];
    fU[s] = cs.beta[s];
  }
  if (threadIdx.x == 0) a.GL[bhc] = cs.gam[C - 1];

  // ---- 1a: diag(e) K^ and diag(gamma) Q^ rows out (16 bytes a lane)
  {
    constexpr int UQ = DK / 8;
    MT* Ke = (MT*)a.Ke + bhc * C * DK;
    MT* Qg = (MT*)a.Qg + bhc * C * DK;
    for (int i = threadIdx.x; i < C * UQ; i += blockDim.x) {
      const int t = i / UQ, u = i - t * UQ;
      const float fk = rk[t] * cs.e[t], fq = rq[t] * qs * cs.gam[t];
      const bf16x8 xk = *reinterpret_cast<const bf16x8*>(tk + t * KP + 8 * u);
      const bf16x8 xq = *reinterpret_cast<const bf16x8*>(tq + t * KP + 8 * u);
      bf16x8 ok, oq;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ok[e] = (bf16)((float)xk[e] * fk);
        oq[e] = (bf16)((float)xq[e] * fq);
      }
      *reinterpret_cast<bf16x8*>(Ke + t * DK + 8 * u) = ok;
      *reinterpret_cast<bf16x8*>(Qg + t * DK + 8 * u) = oq;
    }
  }
  // ---- 1b: k k^T and q k^T on this wave's tiles (column block cb, row tiles 2 hh, 2 hh + 1): L into LDS, M staged
  {
    const int cb = w & 3, hh = w >> 2;
    f4 KK[2], QK[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) KK[i] = QK[i] = f4{0.f, 0.f, 0.f, 0.f};
    // tiles above the diagonal (mi < cb) are computed too and masked below: no wave-dependent branch, so each
    // k-block's fragments are read one stage ahead of its products
    Frag<MT> st[2][5];
    auto load = [&](int p, Frag<MT>(&f)[5]) {
      f[0] = frag_tile<MT, GQ>(tk, 16 * cb, 32 * p);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        f[1 + 2 * i] = frag_tile<MT, GQ>(tk, 16 * (2 * hh + i), 32 * p);
        f[2 + 2 * i] = frag_tile<MT, GQ>(tq, 16 * (2 * hh + i), 32 * p);
      }
    };
    load(0, st[0]);
#pragma unroll
    for (int p = 0; p < DK / 32; ++p) {
      if (p + 1 < DK / 32) load(p + 1, st[(p + 1) & 1]);
      const Frag<MT>(&f)[5] = st[p & 1];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        mma(KK[i], f[1 + 2 * i], f[0]);
        mma(QK[i], f[2 + 2 * i], f[0]);
      }
    }
    const int s = 16 * cb + n;
    const float rks = rk[s];
    const double Gs = cs.G[s];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r0 = 16 * (2 * hh + i) + 4 * j;
      const f4 rq4 = *reinterpret_cast<const f4*>(rq + r0), rk4 = *reinterpret_cast<const f4*>(rk + r0);
      const f4 b4 = *reinterpret_cast<const f4*>(cs.beta + r0);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = r0 + r;
        // mask before the exponent; the hardware exp2 (a bf16 kernel: its ~1e-6 relative error is far below the
        // operands'; 2-3% off the kernel against the library expf)
        const float gm = (row >= s) ? __builtin_amdgcn_exp2f((float)(cs.G[row] - Gs) * 1.4426950408889634f) : 0.f;
        sL[row * FP + s] = (row > s) ? b4[r] * (KK[i][r] * (rk4[r] * rks)) * gm : 0.f;
        sM[row * CP + s] = (bf16)((row >= s) ? QK[i][r] * (rq4[r] * qs * rks) * gm : 0.f);
      }
    }
  }
  wait_dma();                              // v's tile has landed (this wave's part of it)
  __syncthreads();
  if (nrows < C) {                         // v's rows past the end: zeros (read in phase 4, after several barriers)
    constexpr int UV = VP / 8;
    const int nz = C - nrows;
    for (int i = threadIdx.x; i < nz * UV; i += blockDim.x)
      *reinterpret_cast<bf16x8*>(tv + (nrows + i % nz) * VP + 8 * (i / nz)) = bf16x8{};
  }
  // ---- 1c: M out; the diagonal 16 x 16 blocks of A = (I + L)^-1 by forward substitution (wave 0, lane = (block l / 16,
  // column l % 16), column form: the same fmaf sequence per element as the row form), zeros above the diagonal blocks
  {
    MT* Mg = (MT*)a.M + bhc * C * C;
    for (int i = threadIdx.x; i < C * (C / 8); i += blockDim.x) {
      const int t = i >> 3, u = i & 7;
      *reinterpret_cast<bf16x8*>(Mg + t * C + 8 * u) = *reinterpret_cast<const bf16x8*>(sM + t * CP + 8 * u);
    }
  }
  if (w == 0) {
    const int bb = l >> 4, cc = l & 15;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = (i == cc) ? 1.f : 0.f;
#pragma unroll
    for (int m = 0; m < 16; ++m) {
      const float* Lc = sL + (16 * bb) * FP + 16 * bb + m;
#pragma unroll
      for (int i = m + 1; i < 16; ++i) x[i] = fmaf(-Lc[i * FP], x[m], x[i]);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sA[(16 * bb + i) * FP + 16 * bb + cc] = x[i];
  } else {
    for (int i = threadIdx.x - 64; i < C * C; i += blockDim.x - 64) {
      const int row = i / C, col = i % C;
      if ((col >> 4) > (row >> 4)) sA[row * FP + col] = 0.f;
    }
  }
  __syncthreads();
  // ---- 2: blocks below the diagonal, one block-distance at a time: A_ij = -A_ii sum_{m=j}^{i-1} L_im A_mj (fp32 MFMA)
  for (int dist = 1; dist < 4; ++dist) {
    if (w < 4 - dist) {
      const int bi = w + dist, bj = w;
      f4 t = {0.f, 0.f, 0.f, 0.f};
      for (int m = bj; m < bi; ++m) {
#pragma unroll
        for (int kk = 0; kk < 16; kk += 4)
          t = __builtin_amdgcn_mfma_f32_16x16x4f32(sL[(16 * bi + (l & 15)) * FP + 16 * m + kk + j],
                                                   sA[(16 * m + kk + j) * FP + 16 * bj + (l & 15)], t, 0, 0, 0);
      }
      f4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int r = 0; r < 4; ++r)
        o = __builtin_amdgcn_mfma_f32_16x16x4f32(sA[(16 * bi + (l & 15)) * FP + 16 * bi + 4 * j + r], t[r], o, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < 4; ++r) sA[(16 * bi + 4 * j + r) * FP + 16 * bj + (l & 15)] = -o[r];
    }
    __syncthreads();
  }

  // ---- 3: A out; W^T = k^T (A diag(beta gamma rk))^T staged and written
  if (a.A) {
    MT* Ag = (MT*)a.A + bhc * C * C;
    const int t = threadIdx.x >> 3, u = threadIdx.x & 7;     // 512 threads = 64 rows x 8 units
    const f4 lo = *reinterpret_cast<const f4*>(sA + t * FP + 8 * u), hi = *reinterpret_cast<const f4*>(sA + t * FP + 8 * u + 4);
    *reinterpret_cast<bf16x8*>(Ag + t * C + 8 * u) =
        bf16x8{(bf16)lo[0], (bf16)lo[1], (bf16)lo[2], (bf16)lo[3], (bf16)hi[0], (bf16)hi[1], (bf16)hi[2], (bf16)hi[3]};
  }
  // B operand (A diag(f))^T, k = s: lane's token t = 16 ti + l % 16, slots s = 32 p + kmap(j, .), as a hi + lo pair of
  // bf16 fragments (two products for one).  A diag(f) is fp32; rounded once to bf16 it put ~2^-9 relative error into
  // every W and U (U is stored fp32 because Vn = U - W S cancels), which doubled the bf16 path's dg and dk against
  // float64.  With the pair, W is the bf16 rounding of the fp32 product and U carries only fp32 error.  Wave w takes
  // token tile ti = w % 4 and every other feature block from w / 4 on, so it splits only its own tile's two fragments
  // (once for W's blocks, once for all of U's).
  const int ti = w & 3, np = (16 * ti + 15) / 32 + 1;     // k-blocks p < np: the tokens s <= the tile's last row
  auto fragAf = [&](int p, const float* f, Frag<MT>& hi, Frag<MT>& lo) {
    const int t = 16 * ti + n, s0 = 32 * p + 4 * j;
    const f4 a0 = *reinterpret_cast<const f4*>(sA + t * FP + s0), a1 = *reinterpret_cast<const f4*>(sA + t * FP + s0 + 16);
    const f4 f0 = *reinterpret_cast<const f4*>(f + s0), f1 = *reinterpret_cast<const f4*>(f + s0 + 16);
    Frag<float> x;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x.set(e, a0[e] * f0[e]);
      x.set(e + 4, a1[e] * f1[e]);
    }
    frag_split(x, hi, lo);
  };
  {
    Frag<MT> hi[2], lo[2];
#pragma unroll
    for (int p = 0; p < 2; ++p)
      if (p < np) fragAf(p, fW, hi[p], lo[p]);
#pragma unroll
    for (int db = w >> 2; db < NBD; db += 2) {
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (p < np) {
          const Frag<MT> kT = frag_tr(tk, KP, 32 * p, 16 * db);
          mma(acc, kT, hi[p]);
          mma(acc, kT, lo[p]);
        }
      const int t = 16 * ti + n;
      *reinterpret_cast<bf16x4*>(stW + t * KP + 16 * db + 4 * j) = bf16x4{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
    }
  }
  __syncthreads();
  {
    constexpr int UQ = DK / 8;
    MT* Wg = (MT*)a.W + bhc * C * DK;
    for (int i = threadIdx.x; i < C * UQ; i += blockDim.x) {
      const int t = i / UQ, u = i - t * UQ;
      *reinterpret_cast<bf16x8*>(Wg + t * DK + 8 * u) = *reinterpret_cast<const bf16x8*>(stW + t * KP + 8 * u);
    }
  }
  // ---- 4: U^T = v^T (A diag(beta))^T, VB value columns per pass, written from the accumulators (4 fp32 columns a lane)
  float* Ug = a.U + bhc * C * DV;
  Frag<MT> uhi[2], ulo[2];
#pragma unroll
  for (int p = 0; p < 2; ++p)
    if (p < np) fragAf(p, fU, uhi[p], ulo[p]);
  for (int vb = 0; vb < DV; vb += VB) {
    if (vb > 0) {                          // the next block of v, once every wave is done with this one
      __syncthreads();
      GV::dma(tv, v + (size_t)t0 * v_pitch + vb, v_pitch, w, NW, nrows);
      wait_dma();
      __syncthreads();
      if (nrows < C) {
        constexpr int UV = VP / 8;
        for (int i = threadIdx.x; i < (C - nrows) * UV; i += blockDim.x)
          *reinterpret_cast<bf16x8*>(tv + (nrows + i / UV) * VP + 8 * (i % UV)) = bf16x8{};
        __syncthreads();
      }
    }
#pragma unroll
    for (int vk = w >> 2; vk < NBV; vk += 2) {
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (p < np) {
          const Frag<MT> vT = frag_tr(tv, VP, 32 * p, 16 * vk);
          mma(acc, vT, uhi[p]);
          mma(acc, vT, ulo[p]);
        }
      *reinterpret_cast<f4*>(Ug + (size_t)(16 * ti + n) * DV + vb + 16 * vk + 4 * j) = acc;
    }
  }
}

// XCD-aware map of a flat workgroup id to (head-row, column slice): the slices of one head-row share an XCD (and its
// L2), since consecutive workgroup ids go to consecutive XCDs.  Returns false for the padding workgroups.
__device__ __forceinline__ bool state_map(int nslice, int HR, int& hr, int& slice, int f) {
  const int xcd = f & 7, kx = f >> 3;
  hr = (kx / nslice) * 8 + xcd;
  slice = kx % nslice;
  return hr < HR;
}

// The state's 16-column slice of a wave into accumulator tiles (rows 16 di + 4 j + r, column col); zeros for NULL.  One
// uniform branch, so all the loads of the slice are in flight together.
template <int ND>
__device__ __forceinline__ void load_state(f4 (&S)[ND], const float* src, size_t base, int DV, int col) {
  const int j = lane_id() >> 4;
  if (src) {
#pragma unroll
    for (int di = 0; di < ND; ++di)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[di][r] = src[base + (size_t)(16 * di + 4 * j + r) * DV + col];
  } else {
#pragma unroll
    for (int di = 0; di < ND; ++di) S[di] = f4{0.f, 0.f, 0.f, 0.f};
  }
}

// double-buffer the chunk stages when two fit in LDS
constexpr int LDS_BYTES = 160 * 1024 - 2048;
template <int STAGE_BYTES, int EXTRA_BYTES = 0>
struct Buffers {
  static constexpr int N = (2 * STAGE_BYTES + EXTRA_BYTES <= LDS_BYTES) ? 2 : 1;
};

// The L2 prefetch of a sequential pass's loader wave.  The loader copies the next chunk into LDS while this one
// computes, and the chain waits whenever that copy's HBM latency exceeds a chunk's compute; so the loader also touches
// the chunk after the next one, a period ahead: one dword a 128-byte line, copied into an LDS sink of its own
// (TOUCH_SINK bytes) that nothing reads, so that its copy a period later finds the lines in L2.  The lines are those
// of the chunk's per-chunk tiles (tiles[k] its tile of tensor k, `ends` the cumulative line counts, NK tiles) -- a
// head-row's value-column slices read the same tiles, so the workgroup touches lines [lo, hi] only, its share -- and
// the first line of each of 64 rows of its own columns of a token-major tensor (row r at rows + min(r, nrows - 1) *
// pitch bytes).  It issues exactly TOUCH_LOADS loads, after every copy already issued: loads retire in issue order,
// so wait_vmcnt<TOUCH_LOADS>() after it leaves those copies landed.
constexpr int TOUCH_SINK = 256, TOUCH_NTL = 2, TOUCH_LOADS = TOUCH_NTL + 1;
template <int NK>
__device__ __forceinline__ void touch_chunk(const char* const (&tiles)[NK], const int (&ends)[NK], int lo, int hi,
                                            const char* rows, size_t pitch, int nrows) {
  __shared__ unsigned sink[TOUCH_SINK / 4];
  const int l = lane_id();
  lds_void* const s = (lds_void*)sink;
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < TOUCH_NTL; ++i) {
    const int li = min(lo + 64 * i + l, hi);
    const char* p = tiles[0] + (size_t)li * 128;
#pragma unroll
    for (int k = 1; k < NK; ++k)
      if (li >= ends[k - 1]) p = tiles[k] + (size_t)(li - ends[k - 1]) * 128;
    __builtin_amdgcn_global_load_lds((const void*)p, s, 4, 0, 0);
  }
  __builtin_amdgcn_global_load_lds((const void*)(rows + (size_t)min(l, nrows - 1) * pitch), s, 4, 0, 0);
  __builtin_amdgcn_sched_barrier(0);
}
// This workgroup's share [lo, hi] of `lines` lines split over `parts` workgroups.
__device__ __forceinline__ void touch_share(int lines, int parts, int part, int& lo, int& hi) {
  const int per = (lines + parts - 1) / parts;
  lo = part * per;
  hi = min(lo + per, lines) - 1;
}

// ---------------------------------------------------------------------------------------------------------------------
// the forward state pass (+ output), sequential over chunks.  Per chunk the workgroup streams W, diag(e) K^ and, for
// the output, diag(gamma) Q^ and M into a swizzled LDS stage by asynchronous copies -- the next chunk's copies are in
// flight while this chunk's MFMAs run -- and each wave keeps its 16 columns of S in accumulators.  The barriers order
// LDS only (lds_barrier): the loader waits for its copies itself, and no wave waits for its global stores.
// ---------------------------------------------------------------------------------------------------------------------
template <typename MT, int DK, bool OUT, bool STORE, int NW, int KS = 1>
struct StateFwdLds {
  using GW = Tile<MT, C, DK>;    // W, diag(e) K^, diag(gamma) Q^     [t][d]
  using GM = Tile<MT, C, C>;     // M                                  [t][s]
  static constexpr int O_KE = GW::ELEMS, O_Q = O_KE + GW::ELEMS, O_M = O_Q + (OUT ? GW::ELEMS : 0);
  static constexpr int SZ = O_M + (OUT ? GM::ELEMS : 0);
  // bf16 Vn leaves through per-wave row staging (store mode)
  static constexpr int STG = (STORE && sizeof(MT) == 2) ? NW * ColStage::ELEMS : 0;
  // KS = 2 (the key-split float32 pass): a slot per compute wave for its partial W S product (64 x 16) and, for the
  // output, its half of S as fragments
  static constexpr int XS = OUT ? (DK / 64) * 8 * 64 : 0, XW = XS + 16 * 64;
  static constexpr int EX = KS == 2 ? 2 * NW * XW : 0;
  // DIRECT: one stage of the chunk's tiles does not fit LDS (fp32 at DK = 256); the compute waves then read their
  // fragments from global memory (L2) and the loader wave has nothing to do
  static constexpr bool DIRECT = (SZ + STG + EX) * (int)sizeof(MT) > LDS_BYTES;
  static constexpr int NBUF = DIRECT ? 0 : Buffers<SZ * (int)sizeof(MT), (STG + EX) * (int)sizeof(MT)>::N;
  static constexpr int O_STG = NBUF * SZ, O_EX = O_STG + STG;
  static constexpr int ELEMS = (O_EX + EX) > 16 ? O_EX + EX : 16;
  // whether the key-split form (this struct with KS = 2) serves the pass: float32 operands, key widths 64 and 128
  // (whole 32-row fragments in each half), both halves' slots and a stage in LDS, and at most 5 waves (two column
  // slices): at 9 waves a wave has 168 registers and the pass spills
  static constexpr bool KS_OK = KS == 2 && sizeof(MT) == 4 && (DK == 64 || DK == 128) && !DIRECT && NW <= 2;
};

// The key-split float32 pass (the compute waves of state_fwd_body with KS = 2).  The 16x16x4 float32 MFMA takes a
// SIMD 32 cycles, so a wave that carries a 16-column slice alone is bound by its matrix core: two waves (on two SIMDs)
// carry each slice, wave 2 s + h holding rows [h DK / 2, (h + 1) DK / 2) of the slice's state.  Per chunk each forms
// its half of W S, the pair exchanges the halves through LDS (one barrier) and both take Vn = U - (P_0 + P_1)
// (the same bits in both waves: the sum is commutative), then each updates its own rows of S, and with the output
// each forms the output's row blocks 2 h, 2 h + 1 from the whole S (the partner's half from LDS) and Vn.  Per wave
// that is 208-224 MFMAs a chunk at DK = 128 against 432 for one wave.  The single-wave form sums the two halves of
// W S the same way, so both give the same bits.
template <int DK, int NW, bool OUT, bool STORE>
__device__ __forceinline__ void state_fwd_ks(const StateFwdArgs& a, float* lds, int hr, int slice, int cb, int ce,
                                             size_t crow, int tb) {
  using MT = float;
  using L = StateFwdLds<MT, DK, OUT, STORE, NW, 2>;
  using GW = typename L::GW;
  using GM = typename L::GM;
  constexpr int ND = DK / 16, NH = ND / 2, PH = NH / 2;   // state tiles; a wave's tiles and its 32-row k-blocks
  constexpr int O_KE = L::O_KE, O_Q = L::O_Q, O_M = L::O_M, SZ = L::SZ, NBUF = L::NBUF;
  const int T = a.T, H = a.H, DV = a.DV, NT = a.NT;
  const int h = hr % H;
  const int l = lane_id(), w = wave_id(), j = l >> 4;
  const int cw = w >> 1, kh = w & 1;       // the wave's column slice, and its half of the state's rows
  const int v0 = (slice * NW + cw) * 16;
  const int col = v0 + (l & 15);
  const int r0 = kh * NH * 16;             // the wave's first state row
  float* const xme = lds + L::O_EX + (2 * cw + kh) * L::XW;             // this wave's exchange slot
  const float* const xpa = lds + L::O_EX + (2 * cw + (kh ^ 1)) * L::XW;  // its partner's
  const size_t o_base = ((size_t)tb * T * H + h) * DV, o_pitch = (size_t)H * DV;
  auto loadU = [&](int c, f4* U) {
    const float* Uc = a.U + (crow * NT + c) * C * DV + (size_t)(4 * j) * DV + col;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) U[mi][r] = Uc[(16 * mi + r) * DV];
  };

  f4 S[NH];
  load_state(S, a.s0, (size_t)hr * DK * DV + (size_t)r0 * DV, DV, col);
  f4 Un[4];
  float gln = 0.f;
  if (cb < ce) {
    loadU(cb, Un);
    gln = a.GL[crow * NT + cb];
    if (NBUF == 2) lds_barrier();        // the first chunk is in LDS
  }
  for (int c = cb; c < ce; ++c) {
    const size_t bhc = crow * NT + c;
    const int buf = (NBUF == 2) ? ((c - cb) & 1) : 0;
    f4 U[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) U[mi] = Un[mi];
    const float gl = gln;
    if (c + 1 < ce) {
      loadU(c + 1, Un);
      gln = a.GL[bhc + 1];
    }
    if constexpr (STORE) {                 // S_c: this wave's rows
      float* Scc = a.Sc + bhc * DK * DV + (size_t)(r0 + 4 * j) * DV + col;
#pragma unroll
      for (int di = 0; di < NH; ++di)
#pragma unroll
        for (int r = 0; r < 4; ++r) Scc[(16 * di + r) * DV] = S[di][r];
    }
    if (NBUF == 1) lds_barrier();        // chunk c is in LDS
    const MT* st = lds + buf * SZ;
    const MT* tW = st;
    const MT* tK = st + O_KE;
    // this wave's half of S as B fragments; the output needs the partner's too
    Frag<MT> Sf[PH];
#pragma unroll
    for (int p = 0; p < PH; ++p) {
      Sf[p] = frag_acc<MT>(S[2 * p], S[2 * p + 1]);
      if constexpr (OUT) {
        *reinterpret_cast<f4*>(xme + ((2 * p) * 64 + l) * 4) = f4{Sf[p].v[0], Sf[p].v[1], Sf[p].v[2], Sf[p].v[3]};
        *reinterpret_cast<f4*>(xme + ((2 * p + 1) * 64 + l) * 4) = f4{Sf[p].v[4], Sf[p].v[5], Sf[p].v[6], Sf[p].v[7]};
      }
    }
    // this wave's half of W S: k-blocks kh PH .. kh PH + PH - 1
    f4 P[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) P[mi] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < PH; ++p)
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) mma(P[mi], frag_tile<MT, GW>(tW, 16 * mi, 32 * (kh * PH + p)), Sf[p]);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) *reinterpret_cast<f4*>(xme + L::XS + (mi * 64 + l) * 4) = P[mi];
    lds_barrier();                         // the pair's halves are in LDS
    f4 Vn[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) Vn[mi] = U[mi] - (P[mi] + *reinterpret_cast<const f4*>(xpa + L::XS + (mi * 64 + l) * 4));
    Frag<MT> Vf[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) Vf[p] = frag_acc<MT>(Vn[2 * p], Vn[2 * p + 1]);
    if (STORE && kh == 0) {                // Vn (both waves hold it)
      float* Vnc = (float*)a.Vn + bhc * C * DV + (size_t)(4 * j) * DV + col;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) Vnc[(16 * mi + r) * DV] = Vn[mi][r];
    }
    // this wave's rows of S <- exp(G_last) S + (diag(e) K)^T Vn
#pragma unroll
    for (int di = 0; di < NH; ++di) {
      S[di] = S[di] * gl;
#pragma unroll
      for (int p = 0; p < 2; ++p) mma(S[di], frag_tile_tr<MT, GW>(tK, 32 * p, r0 + 16 * di), Vf[p]);
    }
    if constexpr (OUT) {
      // rows 16 mi of O^T = S^T (diag(gamma) Q)^T + Vn^T M^T for mi = 2 kh, 2 kh + 1, from the whole S (fragments of
      // rows 0 .. DK / 2 - 1 in S0, the rest in S1)
      const MT* tQ = st + O_Q;
      const MT* tM = st + O_M;
      Frag<MT> S0[PH], S1[PH];
#pragma unroll
      for (int p = 0; p < PH; ++p) {
        const f4 x = *reinterpret_cast<const f4*>(xpa + ((2 * p) * 64 + l) * 4);
        const f4 y = *reinterpret_cast<const f4*>(xpa + ((2 * p + 1) * 64 + l) * 4);
        Frag<MT> q;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          q.v[r] = x[r];
          q.v[r + 4] = y[r];
        }
        S0[p] = kh ? q : Sf[p];
        S1[p] = kh ? Sf[p] : q;
      }
      f4 pO[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) pO[m] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < ND / 2; ++p)
#pragma unroll
        for (int m = 0; m < 2; ++m)
          mma(pO[m], p < PH ? S0[p % PH] : S1[p % PH], frag_tile<MT, GW>(tQ, 16 * (2 * kh + m), 32 * p));
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int m = 0; m < 2; ++m)
          if (32 * p <= 16 * (2 * kh + m) + 15) mma(pO[m], Vf[p], frag_tile<MT, GM>(tM, 16 * (2 * kh + m), 32 * p));
      int t0, tend;
      chunk_span(a.pack, NT, c, T, t0, tend);
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const int t = t0 + 16 * (2 * kh + m) + (l & 15);
        const size_t at = o_base + (size_t)t * o_pitch + v0 + 4 * j;
        if (t < tend) {
          if (a.obf) store4<bf16>((bf16*)a.o + at, pO[m]);
          else store4<MT>((MT*)a.o + at, pO[m]);
        }
      }
    }
    lds_barrier();                         // end of chunk c: the next chunk is in, this buffer and the slots are free
  }
  if (a.sT) {
#pragma unroll
    for (int di = 0; di < NH; ++di)
#pragma unroll
      for (int r = 0; r < 4; ++r) a.sT[(size_t)hr * DK * DV + (r0 + 16 * di + 4 * j + r) * DV + col] = S[di][r];
  }
}

// The pass of workgroup f of the launch (see state_map), with `lds` the workgroup's LDS (StateFwdLds::ELEMS elements).
// MAP (with neither OUT nor STORE): the chunk map of each sequence instead of its states.  A sequence's pass is affine
// in its starting state, S_end = A S_0 + B, so it runs on DK + DV columns: the first DK start from the identity with U
// taken as zero (they end as A, DK x DK), the other DV from zero with the real U (they end as B); sT receives
// [A | B] per head-row, row pitch DK + DV.
template <typename MT, int DK, int NW, bool OUT, bool STORE, bool MAP = false, int KS = 1>
__device__ __forceinline__ void state_fwd_body(const StateFwdArgs& a, MT* lds, int f) {
  static_assert(!MAP || (!OUT && !STORE), "the map pass writes only the maps");
  static_assert(KS == 1 || (!MAP && StateFwdLds<MT, DK, OUT, STORE, NW, KS>::KS_OK), "the key-split pass");
  using L = StateFwdLds<MT, DK, OUT, STORE, NW, KS>;
  using GW = typename L::GW;
  using GM = typename L::GM;
  constexpr int ND = DK / 16;
  constexpr int O_KE = L::O_KE, O_Q = L::O_Q, O_M = L::O_M, SZ = L::SZ, NBUF = L::NBUF;
  constexpr bool DIRECT = L::DIRECT;
  // the layouts the fragment readers see: the padded LDS tiles, or the dense global ones
  using FW = std::conditional_t<DIRECT, Dense<MT, C, DK>, GW>;
  using FM = std::conditional_t<DIRECT, Dense<MT, C, C>, GM>;

  const int T = a.T, H = a.H, DV = a.DV, NT = a.NT;
  int hr, slice;
  if (!state_map(a.nslice, a.B * H, hr, slice, f)) return;
  const int b = hr / H, h = hr % H;
  const int l = lane_id(), w = wave_id(), j = l >> 4;
  int cb, ce;                              // this head-row's chunks (its sequence's, for packed rows)
  seq_chunks(a.pack, NT, b, cb, ce);
  const size_t crow = a.pack ? (size_t)h : (size_t)hr;   // row of the per-chunk tensors [*, H, NT, ...]
  const int tb = a.pack ? 0 : b;           // batch row of the token tensors

  if (w == KS * NW) {
    if constexpr (DIRECT) return;          // no copies: the compute waves pass no barrier in this mode
    // the loader wave: every asynchronous copy of the chunk tiles, one chunk ahead of the compute waves, so that their
    // issue (a CU's load path takes ~1K cycles for a chunk's tiles) never stalls the MFMA chain.  With KS = 2 it also
    // passes the compute waves' mid-chunk barrier (their exchange of halves), before waiting for its copies.
    int offW[GW::per_wave(1)], offM[GM::per_wave(1)];
    GW::template plan<1>(offW, 0, DK);
    if (OUT) GM::template plan<1>(offM, 0, C);
    auto issue = [&](int c, int buf) {
      MT* st = lds + buf * SZ;
      const size_t bhc = crow * NT + c;
      GW::template dma_planned<1>(st, (const MT*)a.W + bhc * C * DK, offW, 0);
      GW::template dma_planned<1>(st + O_KE, (const MT*)a.Ke + bhc * C * DK, offW, 0);
      if (OUT) {
        GW::template dma_planned<1>(st + O_Q, (const MT*)a.Qg + bhc * C * DK, offW, 0);
        GM::template dma_planned<1>(st + O_M, (const MT*)a.M + bhc * C * C, offM, 0);
      }
    };
    if (NBUF == 2) {
      if (cb < ce) {
        issue(cb, 0);
        wait_dma();
        lds_barrier();
      }
      for (int c = cb; c < ce; ++c) {
        if (c + 1 < ce) issue(c + 1, (c + 1 - cb) & 1);
        if constexpr (KS == 2) lds_barrier();
        wait_dma();
        lds_barrier();
      }
    } else {
      for (int c = cb; c < ce; ++c) {
        issue(c, 0);
        wait_dma();
        lds_barrier();   // chunk c is in LDS
        if constexpr (KS == 2) lds_barrier();
        lds_barrier();   // the compute waves are done with it
      }
    }
    return;                // the compute waves pass no barrier after their loop
  }
  if constexpr (KS == 2) {
    state_fwd_ks<DK, NW, OUT, STORE>(a, lds, hr, slice, cb, ce, crow, tb);
    return;
  }

  const int v0 = (slice * NW + w) * 16;
  const int col = v0 + (l & 15);
  const int DVt = MAP ? DV + DK : DV;      // the pass's columns (the map pass: A's DK, then B's DV)
  const bool ident = MAP && v0 < DK;       // a map column of A: identity start, no U (uniform across the wave)
  const size_t o_base = ((size_t)tb * T * H + h) * DV, o_pitch = (size_t)H * DV;
  auto loadU = [&](int c, f4* U) {
    if (ident) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) U[mi] = f4{0.f, 0.f, 0.f, 0.f};
      return;
    }
    const float* Uc = a.U + (crow * NT + c) * C * DV + (size_t)(4 * j) * DV + (MAP ? col - DK : col);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) U[mi][r] = Uc[(16 * mi + r) * DV];
  };
  // results go out as soon as they exist, after the next chunk's U loads are issued (vmcnt is in order, so waiting on
  // those loads never waits on the stores)
  // O^T tiles: lane l holds O[16 mi + l % 16][v0 + 4 j + 0..3], four adjacent outputs of one token (one 8- or
  // 16-byte store each)
  auto store_o = [&](int c, const f4 (&Ot)[4]) {
    int t0, tend;
    chunk_span(a.pack, NT, c, T, t0, tend);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const int t = t0 + 16 * mi + (l & 15);
      const size_t at = o_base + (size_t)t * o_pitch + v0 + 4 * j;
      if (t < tend) {
        if (sizeof(MT) == 4 && a.obf) store4<bf16>((bf16*)a.o + at, Ot[mi]);
        else store4<MT>((MT*)a.o + at, Ot[mi]);
      }
    }
  };
  auto store_sc = [&](int c, const f4 (&X)[ND]) {
    float* Scc = a.Sc + (crow * NT + c) * DK * DV + (size_t)(4 * j) * DV + col;
#pragma unroll
    for (int di = 0; di < ND; ++di)
#pragma unroll
      for (int r = 0; r < 4; ++r) Scc[(16 * di + r) * DV] = X[di][r];
  };
  auto store_vn = [&](int c, const f4 (&X)[4]) {
    if constexpr (sizeof(MT) == 2) {
      store_cols(lds + L::O_STG + w * ColStage::ELEMS, (MT*)a.Vn + (crow * NT + c) * C * DV + v0, DV, X);
    } else {
      MT* Vnc = (MT*)a.Vn + (crow * NT + c) * C * DV + (size_t)(4 * j) * DV + col;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) Vnc[(16 * mi + r) * DV] = from_f<MT>(X[mi][r]);
    }
  };

  f4 S[ND];
  if constexpr (MAP) {
#pragma unroll
    for (int di = 0; di < ND; ++di)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[di][r] = (ident && 16 * di + 4 * j + r == col) ? 1.f : 0.f;
  } else {
    load_state(S, a.s0, (size_t)hr * DK * DV, DV, col);
  }

  f4 Un[4];
  float gln = 0.f;
  if (cb < ce) {
    loadU(cb, Un);
    gln = a.GL[crow * NT + cb];
    if (NBUF == 2) lds_barrier();        // the first chunk is in LDS
  }
  for (int c = cb; c < ce; ++c) {
    const size_t bhc = crow * NT + c;
    const int buf = (NBUF == 2) ? ((c - cb) & 1) : 0;
    f4 U[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) U[mi] = Un[mi];
    const float gl = gln;
    if (c + 1 < ce) {
      loadU(c + 1, Un);
      gln = a.GL[bhc + 1];
    }
    if (STORE) store_sc(c, S);
    if (NBUF == 1) lds_barrier();        // chunk c is in LDS
    const MT* st = lds + buf * SZ;
    // the chunk's tiles: W, diag(e) K^, diag(gamma) Q^, M
    const MT* tW = DIRECT ? (const MT*)a.W + bhc * C * DK : st;
    const MT* tK = DIRECT ? (const MT*)a.Ke + bhc * C * DK : st + O_KE;
    const MT* tQ = DIRECT ? (const MT*)a.Qg + bhc * C * DK : st + O_Q;
    const MT* tM = DIRECT ? (const MT*)a.M + bhc * C * C : st + O_M;

    // The output pass (one wave per SIMD, registers to spare) reads every fragment that does not depend on S first, so
    // the LDS latency overlaps the conversions and the MFMAs, and runs the products k-block by k-block across their
    // tiles (independent accumulators between dependent ones).  The store pass, which shares a launch with the reverse
    // pass at two waves per SIMD, keeps the register-lean order (fragments next to their MFMAs).
    constexpr bool EARLY = OUT && NW <= 4;   // 9 waves (NW = 8) leave 168 registers a wave: lean order there
    Frag<MT> fw[4][ND / 2], fk[ND][2];
    if constexpr (EARLY) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int p = 0; p < ND / 2; ++p) fw[mi][p] = frag_tile<MT, FW>(tW, 16 * mi, 32 * p);
#pragma unroll
      for (int di = 0; di < ND; ++di)
#pragma unroll
        for (int p = 0; p < 2; ++p) fk[di][p] = frag_tile_tr<MT, FW>(tK, 32 * p, 16 * di);
    }
    // S as the B operand (k = state rows)
    Frag<MT> Sf[ND / 2];
#pragma unroll
    for (int p = 0; p < ND / 2; ++p) Sf[p] = frag_acc<MT>(S[2 * p], S[2 * p + 1]);
    // Vn = U - W S.  Float32 at key widths 64 and 128 sums the state's two row halves apart and then adds them, the
    // key-split pass's order (state_fwd_ks), so the two forms give the same bits.
    constexpr bool HALVES = sizeof(MT) == 4 && !MAP && (DK == 64 || DK == 128);
    f4 Vn[4], Vh[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) Vn[mi] = Vh[mi] = f4{0.f, 0.f, 0.f, 0.f};
    if constexpr (EARLY) {
#pragma unroll
      for (int p = 0; p < ND / 2; ++p)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) mma((HALVES && p >= ND / 4) ? Vh[mi] : Vn[mi], fw[mi][p], Sf[p]);
    } else {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int p = 0; p < ND / 2; ++p)
          mma((HALVES && p >= ND / 4) ? Vh[mi] : Vn[mi], frag_tile<MT, FW>(tW, 16 * mi, 32 * p), Sf[p]);
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) Vn[mi] = U[mi] - (HALVES ? Vn[mi] + Vh[mi] : Vn[mi]);
    Frag<MT> Vf[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) Vf[p] = frag_acc<MT>(Vn[2 * p], Vn[2 * p + 1]);
    if (STORE) store_vn(c, Vn);
    // S <- exp(G_last) S + (diag(e) K)^T Vn   (the chain to the next chunk; the rest below is off it)
    f4 Sn[ND];
#pragma unroll
    for (int di = 0; di < ND; ++di) Sn[di] = S[di] * gl;
    if constexpr (EARLY) {
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int di = 0; di < ND; ++di) mma(Sn[di], fk[di][p], Vf[p]);
    } else {
#pragma unroll
      for (int di = 0; di < ND; ++di)
#pragma unroll
        for (int p = 0; p < 2; ++p) mma(Sn[di], frag_tile_tr<MT, FW>(tK, 32 * p, 16 * di), Vf[p]);
    }
    if (OUT) {
      // O = diag(gamma) Q S + M Vn (M lower triangular: k-blocks past the row block are zero)
      Frag<MT> fq[4][ND / 2], fm[4][2];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int p = 0; p < ND / 2; ++p) fq[mi][p] = frag_tile<MT, FW>(tQ, 16 * mi, 32 * p);
#pragma unroll
        for (int p = 0; p < 2; ++p)
          if (32 * p <= 16 * mi + 15) fm[mi][p] = frag_tile<MT, FM>(tM, 16 * mi, 32 * p);
      }
      // O^T = S^T (diag(gamma) Q)^T + Vn^T M^T: the same fragments with A and B swapped
      f4 pO[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) pO[mi] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < ND / 2; ++p)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) mma(pO[mi], Sf[p], fq[mi][p]);
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
          if (32 * p <= 16 * mi + 15) mma(pO[mi], Vf[p], fm[mi][p]);
      store_o(c, pO);
    }
#pragma unroll
    for (int di = 0; di < ND; ++di) S[di] = Sn[di];
    if constexpr (!DIRECT) lds_barrier();   // end of chunk c: the next chunk is in, this buffer may be refilled
  }
  if (a.sT) {
#pragma unroll
    for (int di = 0; di < ND; ++di)
#pragma unroll
      for (int r = 0; r < 4; ++r) a.sT[(size_t)hr * DK * DVt + (16 * di + 4 * j + r) * DVt + col] = S[di][r];
  }
}

template <typename MT, int DK, int NW, bool OUT, bool STORE, bool MAP = false, int KS = 1>
__global__ void __launch_bounds__(64 * (KS * NW + 1)) state_fwd_kernel(StateFwdArgs a) {
  __shared__ __attribute__((aligned(1024))) MT lds[StateFwdLds<MT, DK, OUT, STORE, NW, KS>::ELEMS];
  state_fwd_body<MT, DK, NW, OUT, STORE, MAP, KS>(a, lds, blockIdx.x);
}

// state_scan_kernel for DK <= 128 (see above).  A step is A_s [DK x DK] times the state slice [DK x 16] on fp32 MFMAs
// (16x16x4): wave w forms row tiles w, w + 4 of the new slice, A's fragments from the LDS stage, the slice's from LDS
// in fragment order (Sf[q][g][j][r] = S[16 q + 4 g + r][c0 + j], which is also where each row tile's accumulators go),
// B_s's columns as the accumulators' start.  The products' k order: instruction (q, r) sums k = 16 q + 4 g + r over the
// lane groups g.
template <int DK>
__device__ __forceinline__ void state_scan_staged(const float* maps, const float* s0, float* starts, int nseg, int H,
                                                  int DV) {
  using GA = Tile<float, DK, DK>;          // A_s rows at a padded pitch (DK + 4 floats)
  constexpr int NW = 4, NRT = DK / 16, TPW = (NRT + NW - 1) / NW;   // row tiles, per wave
  __shared__ __attribute__((aligned(16))) float Sf[DK * 16];
  __shared__ __attribute__((aligned(16))) float As[2][GA::ELEMS];
  const int h = blockIdx.y, r = blockIdx.z, c0 = blockIdx.x * 16;
  const int DVt = DK + DV;
  const int l = lane_id(), w = wave_id(), g = l >> 4, j = l & 15;
  auto sf_index = [](int d, int c) { return ((((d >> 4) * 4 + ((d & 15) >> 2)) * 16 + c) << 2) + (d & 3); };
  auto map_of = [&](int sg) { return maps + (((size_t)r * nseg + sg) * H + h) * DK * DVt; };
  f4 bn[TPW];                              // the next step's B_s[16 t + 4 g + 0..3][c0 + j] of this lane's row tiles
  auto prefetch = [&](int sg) {            // A_sg into stage sg & 1 (asynchronous) and its B columns into bn
    GA::template dma_exact_opaque<NW>(As[sg & 1], map_of(sg), DVt, w, DK, l);
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const int t = min(w + NW * u, NRT - 1);
      const float* Bc = map_of(sg) + (size_t)(16 * t + 4 * g) * DVt + DK + c0 + j;
#pragma unroll
      for (int e = 0; e < 4; ++e) bn[u][e] = Bc[(size_t)e * DVt];
    }
  };
  for (int i = threadIdx.x; i < DK * 16; i += 256) {
    const int d = i / 16, c = i % 16;
    Sf[sf_index(d, c)] = s0 ? s0[((size_t)r * H + h) * DK * DV + (size_t)d * DV + c0 + c] : 0.f;
  }
  if (nseg > 1) prefetch(0);
  __syncthreads();
  for (int sg = 0; sg < nseg; ++sg) {
    const size_t seg = (size_t)r * nseg + sg;
    float* out = starts + (seg * H + h) * DK * DV;
    for (int i = threadIdx.x; i < DK * 16; i += 256) out[(size_t)(i / 16) * DV + c0 + i % 16] = Sf[sf_index(i / 16, i % 16)];
    if (sg + 1 == nseg) break;
    f4 acc[TPW];
    wait_vmcnt<0>();                       // A_sg and B_sg have landed (and this step's stores are out)
#pragma unroll
    for (int u = 0; u < TPW; ++u) acc[u] = bn[u];
    lds_barrier();                         // A_sg visible; every wave is past step sg - 1's reads of stage (sg + 1) & 1
    if (sg + 2 < nseg) prefetch(sg + 1);   // A_{sg+1} lands while this step computes
    const float* A = As[sg & 1];
    f4 sfr[NRT];                           // the slice as B fragments: S[16 q + 4 g + e][c0 + j]
#pragma unroll
    for (int q = 0; q < NRT; ++q) sfr[q] = *reinterpret_cast<const f4*>(Sf + ((q * 4 + g) * 16 + j) * 4);
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const int t = w + NW * u;
      if (t < NRT) {
        const float* Ar = A + GA::offset(16 * t + j, 4 * g);   // A[16 t + j][16 q + 4 g + e] at Ar + 16 q + e
#pragma unroll
        for (int q = 0; q < NRT; ++q) {
          const f4 a = *reinterpret_cast<const f4*>(Ar + 16 * q);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], sfr[q][e], acc[u], 0, 0, 0);
        }
      }
    }
    lds_barrier();                         // every lane has read this step's slice
#pragma unroll
    for (int u = 0; u < TPW; ++u) {
      const int t = w + NW * u;
      if (t < NRT) *reinterpret_cast<f4*>(Sf + ((t * 4 + g) * 16 + j) * 4) = acc[u];
    }
    lds_barrier();
  }
}

// The sequential composition of the segment maps of a row: starts[s] = the state entering segment s, starts[0] = s0
// (zeros when null), starts[s + 1] = A_s starts[s] + B_s, maps[s] = [A_s | B_s] as the map pass writes them.  A
// workgroup takes 16 value columns of a (row, head); the state slice [DK x 16] sits in LDS, and each step a lane forms
// 8 columns of one state row.  The maps do not depend on the chain, so for DK <= 128 the next step's A (DK x DK fp32,
// 64 KiB at 128) is copied into LDS (two stages, asynchronous, unseen by the compiler and waited for explicitly) and its
// B columns into registers while this step computes: a step is then its FMAs only, not a 64 KiB read from memory
// (10 us a step at config 3 before).  Wider keys read A's rows from memory, 16-byte loads all in flight.
template <int DK>
__global__ void __launch_bounds__(256) state_scan_kernel(const float* maps, const float* s0, float* starts, int nseg,
                                                         int H, int DV) {
  if constexpr (DK <= 128) {
    state_scan_staged<DK>(maps, s0, starts, nseg, H, DV);
  } else {
    __shared__ __attribute__((aligned(16))) float Sl[DK * 16];
    const int h = blockIdx.y, r = blockIdx.z, c0 = blockIdx.x * 16;
    const int DVt = DK + DV;
    for (int i = threadIdx.x; i < DK * 16; i += 256) {
      const int d = i / 16, c = i % 16;
      Sl[i] = s0 ? s0[((size_t)r * H + h) * DK * DV + (size_t)d * DV + c0 + c] : 0.f;
    }
    __syncthreads();
    for (int sg = 0; sg < nseg; ++sg) {
      const size_t seg = (size_t)r * nseg + sg;
      float* out = starts + (seg * H + h) * DK * DV;
      for (int i = threadIdx.x; i < DK * 16; i += 256) out[(size_t)(i / 16) * DV + c0 + i % 16] = Sl[i];
      if (sg + 1 == nseg) break;
      const float* Mp = maps + (seg * H + h) * DK * DVt;
      float acc[(2 * DK + 255) / 256][8];
#pragma unroll
      for (int u = 0; u < (2 * DK + 255) / 256; ++u) {
        const int pr = threadIdx.x + 256 * u, d = pr / 2, cg = (pr % 2) * 8;
        if (pr >= 2 * DK) break;
        const float* Ar = Mp + (size_t)d * DVt;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[u][i] = Ar[DK + c0 + cg + i];           // B_s
#pragma unroll 8
        for (int k4 = 0; k4 < DK; k4 += 4) {
          const f4 a = *reinterpret_cast<const f4*>(Ar + k4);                  // A_s[d][k4 .. k4 + 3]
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) {
            const f4 s_lo = *reinterpret_cast<const f4*>(Sl + (k4 + kk) * 16 + cg);
            const f4 s_hi = *reinterpret_cast<const f4*>(Sl + (k4 + kk) * 16 + cg + 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              acc[u][i] = fmaf(a[kk], s_lo[i], acc[u][i]);
              acc[u][4 + i] = fmaf(a[kk], s_hi[i], acc[u][4 + i]);
            }
          }
        }
      }
      __syncthreads();                       // every lane has read this step's state
#pragma unroll
      for (int u = 0; u < (2 * DK + 255) / 256; ++u) {
        const int pr = threadIdx.x + 256 * u, d = pr / 2, cg = (pr % 2) * 8;
        if (pr >= 2 * DK) break;
#pragma unroll
        for (int i = 0; i < 8; ++i) Sl[d * 16 + cg + i] = acc[u][i];
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// The forward state pass with the output, the chain and the output on separate waves (bf16, NW <= 2 column slices per
// workgroup).  A chain wave runs only what the next chunk's state depends on -- Vn = U - W S and
// S <- exp(G_last) S + (diag(e) K)^T Vn -- and hands S and Vn, as the bf16 MFMA fragments it formed, to its output
// wave through LDS.  The output wave forms O = diag(gamma) Q S + M Vn for that chunk one chunk later, from the same
// fragments with the same products in the same order as state_fwd_body (so the same bits).  With STORE the pass also
// writes the backward's S_c (fp32, by the chain wave, whose stores drain under its products) and Vn (bf16, by the
// output wave from the hand-off: the rounding the store pass writes).  The loader wave copies W and diag(e) K^ one
// chunk ahead of the chain and diag(gamma) Q^ and M in the chunk the chain computes, for the output wave's use one
// chunk later: each of the three LDS rings (W, Ke | Qg, M | hand-off) is two stages deep, and one barrier a chunk
// orders them.
// ---------------------------------------------------------------------------------------------------------------------
template <int DK, int NW, bool STORE>
struct StateOutLds {
  // W, Qg and M are read as fragments, whose reads conflict at a pitch of whole 16-byte units: their odd rows hold
  // 64-byte halves swapped (Tile's SW; Ke shares W's layout), -5% on the pass at config 1
  using GW = Tile<bf16, C, DK, (DK >= 64)>;   // W, diag(e) K^, diag(gamma) Q^     [t][d]
  using GM = Tile<bf16, C, C, true>;          // M                                  [t][s]
  static constexpr int ND = DK / 16;
  static constexpr int O_KE = GW::ELEMS, WK = 2 * GW::ELEMS;          // a [W | Ke] stage
  static constexpr int O_M = GW::ELEMS, QM = GW::ELEMS + GM::ELEMS;   // a [Qg | M] stage
  static constexpr int HO = (ND / 2 + 2) * 64 * 8;                    // one chain wave's S and Vn fragments
  static constexpr int O_QM = 2 * WK, O_HO = O_QM + 2 * QM, O_STG = O_HO + 2 * NW * HO;
  static constexpr int ELEMS = O_STG + (STORE ? NW * ColStage::ELEMS : 0);   // the output waves' Vn staging
  static_assert(ELEMS * 2 + (STORE ? 0 : TOUCH_SINK) <= LDS_BYTES, "state_out LDS");
};

template <int DK, int NW, bool STORE>
__global__ void __launch_bounds__(64 * (2 * NW + 1)) state_out_kernel(StateFwdArgs a) {
  using MT = bf16;
  using L = StateOutLds<DK, NW, STORE>;
  using GW = typename L::GW;
  using GM = typename L::GM;
  constexpr int ND = DK / 16;
  __shared__ __attribute__((aligned(1024))) MT lds[L::ELEMS];

  const int T = a.T, H = a.H, DV = a.DV, NT = a.NT;
  int hr, slice;
  if (!state_map(a.nslice, a.B * H, hr, slice, blockIdx.x)) return;
  const int b = hr / H, h = hr % H;
  const int l = lane_id(), w = wave_id(), j = l >> 4;
  int cb, ce;                              // this head-row's chunks (its sequence's, for packed rows)
  seq_chunks(a.pack, NT, b, cb, ce);
  const int nc = ce - cb;
  const size_t crow = a.pack ? (size_t)h : (size_t)hr;   // row of the per-chunk tensors [*, H, NT, ...]
  const int tb = a.pack ? 0 : b;           // batch row of the token tensors
  // barriers: B_0 before the first chunk, B_{i+1} at the end of the chain's chunk cb + i; every wave passes all nc + 1

  if (w == 2 * NW) {                       // the loader wave
    int offW[GW::per_wave(1)], offM[GM::per_wave(1)];
    GW::template plan<1>(offW, 0, DK);
    GM::template plan<1>(offM, 0, C);
    auto wk = [&](int c, int s) {
      MT* st = lds + s * L::WK;
      const size_t bhc = crow * NT + c;
      GW::template dma_planned<1>(st, (const MT*)a.W + bhc * C * DK, offW, 0);
      GW::template dma_planned<1>(st + L::O_KE, (const MT*)a.Ke + bhc * C * DK, offW, 0);
    };
    auto qm = [&](int c, int s) {
      MT* st = lds + L::O_QM + s * L::QM;
      const size_t bhc = crow * NT + c;
      GW::template dma_planned<1>(st, (const MT*)a.Qg + bhc * C * DK, offW, 0);
      GM::template dma_planned<1>(st + L::O_M, (const MT*)a.M + bhc * C * C, offM, 0);
    };
    // Without the state stores the pass moves little per chunk and the chain waits on each copy's HBM latency (the
    // long single-row prefill: 1.7 us a chunk), so the loader also touches chunk c + 2's tiles and the workgroup's U
    // columns into L2 while chunk c + 1 is copied (touch_chunk).  With them the pass is bound by its bytes, and the
    // touch only slowed the kernels after it.
    constexpr bool TOUCH = !STORE;
    constexpr int LK = C * DK * 2 / 128;
    constexpr int ENDS[4] = {LK, 2 * LK, 3 * LK, 3 * LK + C * C * 2 / 128};
    int lo, hi;
    touch_share(ENDS[3], a.nslice, slice, lo, hi);
    auto touch = [&](int c) {
      const size_t bhc = crow * NT + c, tk = bhc * C * DK * 2;
      const char* const tiles[4] = {(const char*)a.W + tk, (const char*)a.Ke + tk, (const char*)a.Qg + tk,
                                    (const char*)a.M + bhc * C * C * 2};
      touch_chunk<4>(tiles, ENDS, lo, hi, (const char*)(a.U + bhc * C * DV + slice * NW * 16), DV * sizeof(float), C);
      wait_vmcnt<TOUCH_LOADS>();
    };
    if (nc > 0) wk(cb, 0);
    if (TOUCH && nc > 1) touch(cb + 1);
    else wait_dma();
    lds_barrier();                         // B_0: the first [W | Ke] stage is in
    for (int i = 0; i < nc; ++i) {
      if (i + 1 < nc) wk(cb + i + 1, (i + 1) & 1);
      qm(cb + i, i & 1);
      if (TOUCH && i + 2 < nc) touch(cb + i + 2);
      else wait_dma();
      lds_barrier();                       // B_{i+1}
    }
    return;
  }

  const bool chain = w < NW;
  const int cw = chain ? w : w - NW;       // the column slice's chain wave
  const int v0 = (slice * NW + cw) * 16;
  const int col = v0 + (l & 15);
  MT* const ho = lds + L::O_HO + cw * 2 * L::HO;   // the slice's two hand-off stages
  auto ho_frag = [&](int s, int u) { return ho + s * L::HO + (u * 64 + l) * 8; };

  if (chain) {
    auto loadU = [&](int c, f4* U) {
      const float* Uc = a.U + (crow * NT + c) * C * DV + (size_t)(4 * j) * DV + col;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) U[mi][r] = Uc[(16 * mi + r) * DV];
    };
    f4 S[ND];
    load_state(S, a.s0, (size_t)hr * DK * DV, DV, col);
    f4 Un[4];
    float gln = 0.f;
    if (nc > 0) {
      loadU(cb, Un);
      gln = a.GL[crow * NT + cb];
    }
    lds_barrier();                         // B_0
    for (int i = 0; i < nc; ++i) {
      const int c = cb + i, s = i & 1;
      f4 U[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) U[mi] = Un[mi];
      const float gl = gln;
      if (i + 1 < nc) {
        loadU(c + 1, Un);
        gln = a.GL[crow * NT + c + 1];
      }
      const MT* st = lds + s * L::WK;
      // every fragment that does not depend on S first, then the products k-block by k-block across their tiles
      Frag<MT> fw[4][ND / 2], fk[ND][2];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int p = 0; p < ND / 2; ++p) fw[mi][p] = frag_tile<MT, GW>(st, 16 * mi, 32 * p);
#pragma unroll
      for (int di = 0; di < ND; ++di)
#pragma unroll
        for (int p = 0; p < 2; ++p) fk[di][p] = frag_tile_tr<MT, GW>(st + L::O_KE, 32 * p, 16 * di);
      // S as the B operand (k = state rows), handed off
      Frag<MT> Sf[ND / 2];
#pragma unroll
      for (int p = 0; p < ND / 2; ++p) {
        Sf[p] = frag_acc<MT>(S[2 * p], S[2 * p + 1]);
        *reinterpret_cast<bf16x8*>(ho_frag(s, p)) = Sf[p].v;
      }
      if constexpr (STORE) {               // S_c in fp32
        float* Scc = a.Sc + (crow * NT + c) * DK * DV + (size_t)(4 * j) * DV + col;
#pragma unroll
        for (int di = 0; di < ND; ++di)
#pragma unroll
          for (int r = 0; r < 4; ++r) Scc[(16 * di + r) * DV] = S[di][r];
      }
      // Vn = U - W S
      f4 Vn[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) Vn[mi] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < ND / 2; ++p)
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) mma(Vn[mi], fw[mi][p], Sf[p]);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) Vn[mi] = U[mi] - Vn[mi];
      Frag<MT> Vf[2];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        Vf[p] = frag_acc<MT>(Vn[2 * p], Vn[2 * p + 1]);
        *reinterpret_cast<bf16x8*>(ho_frag(s, ND / 2 + p)) = Vf[p].v;
      }
      // S <- exp(G_last) S + (diag(e) K)^T Vn
#pragma unroll
      for (int di = 0; di < ND; ++di) S[di] = S[di] * gl;
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int di = 0; di < ND; ++di) mma(S[di], fk[di][p], Vf[p]);
      lds_barrier();                       // B_{i+1}: this chunk's hand-off is visible, its [W | Ke] stage free
    }
    if (a.sT) {
#pragma unroll
      for (int di = 0; di < ND; ++di)
#pragma unroll
        for (int r = 0; r < 4; ++r) a.sT[(size_t)hr * DK * DV + (16 * di + 4 * j + r) * DV + col] = S[di][r];
    }
    return;
  }

  // the output wave: chunk cb + i after B_{i+1}
  const size_t o_base = ((size_t)tb * T * H + h) * DV, o_pitch = (size_t)H * DV;
  lds_barrier();                           // B_0
  for (int i = 0; i < nc; ++i) {
    lds_barrier();                         // B_{i+1}
    const int c = cb + i, s = i & 1;
    const MT* st = lds + L::O_QM + s * L::QM;
    Frag<MT> Sf[ND / 2], Vf[2];
#pragma unroll
    for (int p = 0; p < ND / 2; ++p) Sf[p].v = *reinterpret_cast<const bf16x8*>(ho_frag(s, p));
#pragma unroll
    for (int p = 0; p < 2; ++p) Vf[p].v = *reinterpret_cast<const bf16x8*>(ho_frag(s, ND / 2 + p));
    // O = diag(gamma) Q S + M Vn (M lower triangular: k-blocks past the row block are zero), formed as
    // O^T = S^T (diag(gamma) Q)^T + Vn^T M^T: lane l holds O[16 mi + l % 16][v0 + 4 j + 0..3]
    Frag<MT> fq[4][ND / 2], fm[4][2];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
      for (int p = 0; p < ND / 2; ++p) fq[mi][p] = frag_tile<MT, GW>(st, 16 * mi, 32 * p);
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (32 * p <= 16 * mi + 15) fm[mi][p] = frag_tile<MT, GM>(st + L::O_M, 16 * mi, 32 * p);
    }
    f4 pO[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) pO[mi] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < ND / 2; ++p)
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) mma(pO[mi], Sf[p], fq[mi][p]);
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
        if (32 * p <= 16 * mi + 15) mma(pO[mi], Vf[p], fm[mi][p]);
    int t0, tend;
    chunk_span(a.pack, NT, c, T, t0, tend);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      const int t = t0 + 16 * mi + (l & 15);
      if (t < tend) store4<MT>((MT*)a.o + o_base + (size_t)t * o_pitch + v0 + 4 * j, pO[mi]);
    }
    if constexpr (STORE) {                 // Vn in accumulator layout (exact: they are bf16 values)
      f4 Y[4];
#pragma unroll
      for (int p = 0; p < 2; ++p)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          Y[2 * p][r] = (float)Vf[p].v[r];
          Y[2 * p + 1][r] = (float)Vf[p].v[r + 4];
        }
      store_cols(lds + L::O_STG + cw * ColStage::ELEMS, (MT*)a.Vn + (crow * NT + c) * C * DV + v0, DV, Y);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// the reverse state pass: streams diag(e) K^, diag(gamma) Q^, W, M and the workgroup's dO columns per chunk
// ---------------------------------------------------------------------------------------------------------------------
template <typename MT, int DK, int NW, int KS = 1>
struct StateBwdLds {
  using GK = Tile<MT, C, DK>;        // diag(e) K^, diag(gamma) Q^, W    [t][d]
  using GM = Tile<MT, C, C>;         // M                                [t][s]
  using GO = Tile<MT, C, 16 * NW>;   // dO columns                       [t][v]
  static constexpr int O_Q = GK::ELEMS, O_W = O_Q + GK::ELEMS, O_M = O_W + GK::ELEMS, O_O = O_M + GM::ELEMS;
  static constexpr int SZ = O_O + GO::ELEMS;
  static constexpr int STG = sizeof(MT) == 2 ? NW * ColStage::ELEMS : 0;   // bf16 dVn leaves through row staging
  static constexpr int SCAL = 32 / (int)sizeof(MT);   // per stage: the chunk's G_last (bits), t0, tend, as 4 ints
  // KS = 2 (the key-split float32 pass): a slot per compute wave for its partial dVn (64 x 16)
  static constexpr int XW = 16 * 64, EX = KS == 2 ? 2 * NW * XW : 0;
  // DIRECT: one stage does not fit LDS (fp32 at DK = 256): the compute waves read the tiles from global memory
  static constexpr bool DIRECT = (SZ + STG + SCAL + EX) * (int)sizeof(MT) + TOUCH_SINK > LDS_BYTES;
  static constexpr int NBUF =
      DIRECT ? 0 : Buffers<SZ * (int)sizeof(MT), (STG + SCAL + EX) * (int)sizeof(MT) + TOUCH_SINK>::N;
  static constexpr int O_STG = NBUF * SZ, O_SCAL = O_STG + STG, O_EX = O_SCAL + SCAL;
  static constexpr int ELEMS = O_EX + EX;
  // see StateFwdLds::KS_OK
  static constexpr bool KS_OK = KS == 2 && sizeof(MT) == 4 && (DK == 64 || DK == 128) && !DIRECT && NW <= 2;
};

// The key-split float32 reverse pass (the compute waves of state_bwd_body with KS = 2; see state_fwd_ks): wave
// 2 s + h holds rows [h DK / 2, (h + 1) DK / 2) of its slice's dS.  Per chunk each forms its half of diag(e) K^ dS
// (with M^T dO for row blocks 2 h, 2 h + 1), the pair exchanges the halves through LDS and both take dVn as their sum,
// then each updates its own rows of dS.  Per wave 208-224 MFMAs a chunk at DK = 128 against 432 for one wave.
template <int DK, int NW>
__device__ __forceinline__ void state_bwd_ks(const StateBwdArgs& a, float* lds, int hr, int slice, int cb, int ce,
                                             size_t crow, int tb) {
  using MT = float;
  using L = StateBwdLds<MT, DK, NW, 2>;
  using GK = typename L::GK;
  using GM = typename L::GM;
  using GO = typename L::GO;
  constexpr int ND = DK / 16, NH = ND / 2, PH = NH / 2;
  constexpr int O_Q = L::O_Q, O_W = L::O_W, O_M = L::O_M, O_O = L::O_O, SZ = L::SZ, NBUF = L::NBUF;
  const int DV = a.DV, NT = a.NT;
  const int l = lane_id(), w = wave_id(), j = l >> 4;
  const int cw = w >> 1, kh = w & 1;       // the wave's column slice, and its half of the state's rows
  const int vg = slice * NW * 16;          // the workgroup's first value column
  const int col = vg + cw * 16 + (l & 15);
  const int r0 = kh * NH * 16;             // the wave's first state row
  float* const xme = lds + L::O_EX + (2 * cw + kh) * L::XW;
  const float* const xpa = lds + L::O_EX + (2 * cw + (kh ^ 1)) * L::XW;
  (void)tb;

  f4 dS[NH];
  load_state(dS, a.dsT, (size_t)hr * DK * DV + (size_t)r0 * DV, DV, col);
  if (cb < ce && NBUF == 2) lds_barrier();   // the last chunk is in LDS
  for (int c = ce - 1, it = 0; c >= cb; --c, ++it) {
    const int buf = (NBUF == 2) ? (it & 1) : 0;
    const size_t bhc = crow * NT + c;
    // the row pitch, opaque to the compiler here: otherwise it keeps the 32 store addresses of dSn and dVn (64-bit
    // each) live across the loop, which spills at 5 waves' 256 registers
    int dv = DV;
    asm volatile("" : "+s"(dv));
    {                                      // dS_{c+1}: this wave's rows
      float* dSc = a.dSn + bhc * DK * dv + (size_t)(r0 + 4 * j) * dv + col;
#pragma unroll
      for (int di = 0; di < NH; ++di)
#pragma unroll
        for (int r = 0; r < 4; ++r) dSc[(16 * di + r) * dv] = dS[di][r];
    }
    if (NBUF == 1) lds_barrier();        // chunk c is in LDS
    const int* sc = (const int*)(lds + L::O_SCAL) + 4 * buf;
    const float gl = __int_as_float(sc[0]);
    const int t0 = sc[1], tend = sc[2];
    const MT* st = lds + buf * SZ;
    const MT* tK = st;
    const MT* tQ = st + O_Q;
    const MT* tW = st + O_W;
    const MT* tM = st + O_M;
    Frag<MT> Of[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      Of[p] = frag_tile_rows<MT, GO>(st + O_O, 32 * p, cw * 16 + (l & 15));
      if (t0 + C > tend)                   // rows past the sequence end hold copies of its last row: zero them
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (t0 + 32 * p + kmap(j, e) >= tend) Of[p].set(e, 0.f);
    }
    Frag<MT> Sf[PH];
#pragma unroll
    for (int p = 0; p < PH; ++p) Sf[p] = frag_acc<MT>(dS[2 * p], dS[2 * p + 1]);
    // this wave's half of dVn
    f4 P[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < PH; ++p) mma(acc, frag_tile<MT, GK>(tK, 16 * mi, 32 * (kh * PH + p)), Sf[p]);
      if ((mi >> 1) == kh)
#pragma unroll
        for (int p = 0; p < 2; ++p)
          if (32 * p + 31 >= 16 * mi) mma(acc, frag_tile_tr<MT, GM>(tM, 32 * p, 16 * mi), Of[p]);
      P[mi] = acc;
      *reinterpret_cast<f4*>(xme + (mi * 64 + l) * 4) = acc;
    }
    lds_barrier();                         // the pair's halves are in LDS
    f4 dV[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) dV[mi] = P[mi] + *reinterpret_cast<const f4*>(xpa + (mi * 64 + l) * 4);
    Frag<MT> Vf[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) Vf[p] = frag_acc<MT>(dV[2 * p], dV[2 * p + 1], -1.f);
    if (kh == 0) {                         // dVn (both waves hold it)
      float* dVc = (float*)a.dVn + bhc * C * dv + (size_t)(4 * j) * dv + col;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) dVc[(16 * mi + r) * dv] = dV[mi][r];
    }
    // this wave's rows of dS <- exp(G_last) dS + (diag(gamma) Q^)^T dO - W^T dVn, one row block at a time (the
    // scheduling barrier keeps the next block's 32 gathered fragment values from being loaded early: 5 waves on 4
    // SIMDs leave 256 registers a wave)
#pragma unroll
    for (int di = 0; di < NH; ++di) {
      f4 acc = dS[di] * gl;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        mma(acc, frag_tile_tr<MT, GK>(tW, 32 * p, r0 + 16 * di), Vf[p]);
        mma(acc, frag_tile_tr<MT, GK>(tQ, 32 * p, r0 + 16 * di), Of[p]);
      }
      dS[di] = acc;
      __builtin_amdgcn_sched_barrier(0);
    }
    lds_barrier();                         // end of chunk c
  }
#pragma unroll
  for (int di = 0; di < NH; ++di)
#pragma unroll
    for (int r = 0; r < 4; ++r) a.ds0[(size_t)hr * DK * DV + (r0 + 16 * di + 4 * j + r) * DV + col] = dS[di][r];
}

template <typename MT, int DK, int NW, int KS = 1>
__device__ __forceinline__ void state_bwd_body(const StateBwdArgs& a, MT* lds, int f) {
  static_assert(KS == 1 || StateBwdLds<MT, DK, NW, KS>::KS_OK, "the key-split pass");
  using L = StateBwdLds<MT, DK, NW, KS>;
  using GK = typename L::GK;
  using GM = typename L::GM;
  using GO = typename L::GO;
  constexpr int ND = DK / 16;
  constexpr int O_Q = L::O_Q, O_W = L::O_W, O_M = L::O_M, O_O = L::O_O, SZ = L::SZ, NBUF = L::NBUF;
  constexpr bool DIRECT = L::DIRECT;
  using FK = std::conditional_t<DIRECT, Dense<MT, C, DK>, GK>;
  using FM = std::conditional_t<DIRECT, Dense<MT, C, C>, GM>;

  const int T = a.T, H = a.H, DV = a.DV, NT = a.NT;
  int hr, slice;
  if (!state_map(a.nslice, a.B * H, hr, slice, f)) return;
  const int b = hr / H, h = hr % H;
  const int l = lane_id(), w = wave_id(), j = l >> 4;
  const int vg = slice * NW * 16;            // the workgroup's first value column
  int cb, ce;                                // this head-row's chunks (its sequence's, for packed rows)
  seq_chunks(a.pack, NT, b, cb, ce);
  const size_t crow = a.pack ? (size_t)h : (size_t)hr;   // row of the per-chunk tensors [*, H, NT, ...]
  const int tb = a.pack ? 0 : b;             // batch row of the token tensors
  const size_t o_base = ((size_t)tb * T * H + h) * DV, o_pitch = (size_t)H * DV;

  if (w == KS * NW) {
    if constexpr (DIRECT) return;          // no copies: the compute waves pass no barrier in this mode
    // the loader wave (see state_fwd_kernel), walking the chunks backwards
    int offK[GK::per_wave(1)], offM[GM::per_wave(1)], offO[GO::per_wave(1)];
    GK::template plan<1>(offK, 0, DK);
    GM::template plan<1>(offM, 0, C);
    GO::template plan<1>(offO, 0, (int)o_pitch);
    auto issue = [&](int c, int buf) {
      MT* st = lds + buf * SZ;
      const size_t bhc = crow * NT + c;
      int t0, tend;
      chunk_span<true>(a.pack, NT, c, T, t0, tend);
      const MT* og = (const MT*)a.dO + o_base + (size_t)t0 * o_pitch + vg;
      if constexpr (KS == 2) {             // addresses formed per copy: the planned offsets (59 registers at DK = 128)
        GK::dma(st, (const MT*)a.Ke + bhc * C * DK, DK, 0, 1);   // spill at 5 waves' 256 registers a wave
        GK::dma(st + O_Q, (const MT*)a.Qg + bhc * C * DK, DK, 0, 1);
        GK::dma(st + O_W, (const MT*)a.W + bhc * C * DK, DK, 0, 1);
        GM::dma(st + O_M, (const MT*)a.M + bhc * C * C, C, 0, 1);
        GO::dma(st + O_O, og, o_pitch, 0, 1, tend - t0);
      } else {
        GK::template dma_planned<1>(st, (const MT*)a.Ke + bhc * C * DK, offK, 0);
        GK::template dma_planned<1>(st + O_Q, (const MT*)a.Qg + bhc * C * DK, offK, 0);
        GK::template dma_planned<1>(st + O_W, (const MT*)a.W + bhc * C * DK, offK, 0);
        GM::template dma_planned<1>(st + O_M, (const MT*)a.M + bhc * C * C, offM, 0);
        if (t0 + C <= tend) GO::template dma_planned<1>(st + O_O, og, offO, 0);
        else GO::dma(st + O_O, og, o_pitch, 0, 1, tend - t0);   // a partial chunk: rows clamped to the sequence
      }
      if (l == 0) {                        // the chunk's scalars beside its stage (the compute waves load nothing)
        int* sc = (int*)(lds + L::O_SCAL) + 4 * buf;
        sc[0] = __float_as_int(ld_const(a.GL, bhc));
        sc[1] = t0;
        sc[2] = tend;
      }
    };
    // the L2 prefetch of chunk c - 2 (touch_chunk) while chunk c - 1 is copied
    constexpr int LK = C * DK * (int)sizeof(MT) / 128;
    constexpr int ENDS[4] = {LK, 2 * LK, 3 * LK, 3 * LK + C * C * (int)sizeof(MT) / 128};
    int lo, hi;
    touch_share(ENDS[3], a.nslice, slice, lo, hi);
    auto touch = [&](int c) {
      const size_t bhc = crow * NT + c, tk = bhc * C * DK * sizeof(MT);
      int t0, tend;
      chunk_span<true>(a.pack, NT, c, T, t0, tend);
      const char* const tiles[4] = {(const char*)a.Ke + tk, (const char*)a.Qg + tk, (const char*)a.W + tk,
                                    (const char*)a.M + bhc * C * C * sizeof(MT)};
      touch_chunk<4>(tiles, ENDS, lo, hi, (const char*)((const MT*)a.dO + o_base + (size_t)t0 * o_pitch + vg),
                     o_pitch * sizeof(MT), tend - t0);
      wait_vmcnt<TOUCH_LOADS>();
    };
    if (NBUF == 2) {
      if (cb < ce) {
        issue(ce - 1, 0);
        if (ce - 2 >= cb) touch(ce - 2);
        else wait_dma();
        lds_barrier();
      }
      for (int c = ce - 1, it = 0; c >= cb; --c, ++it) {
        if (c > cb) issue(c - 1, (it + 1) & 1);
        if constexpr (KS == 2) lds_barrier();   // the compute waves' exchange of halves
        if (c - 2 >= cb) touch(c - 2);
        else wait_dma();
        lds_barrier();
      }
    } else {
      for (int c = ce - 1; c >= cb; --c) {
        issue(c, 0);
        wait_dma();
        lds_barrier();
        if constexpr (KS == 2) lds_barrier();
        lds_barrier();
      }
    }
    return;
  }
  if constexpr (KS == 2) {
    state_bwd_ks<DK, NW>(a, lds, hr, slice, cb, ce, crow, tb);
    return;
  }
  const int col = vg + w * 16 + (l & 15);
  // dS_{c+1} and dVn go out as soon as they exist
  auto store_ds = [&](int c, const f4 (&X)[ND]) {
    float* dSc = a.dSn + (crow * NT + c) * DK * DV + (size_t)(4 * j) * DV + col;
#pragma unroll
    for (int di = 0; di < ND; ++di)
#pragma unroll
      for (int r = 0; r < 4; ++r) dSc[(16 * di + r) * DV] = X[di][r];
  };
  auto store_dv = [&](int c, const f4 (&X)[4]) {
    if constexpr (sizeof(MT) == 2) {
      store_cols(lds + L::O_STG + w * ColStage::ELEMS, (MT*)a.dVn + (crow * NT + c) * C * DV + vg + 16 * w, DV, X);
    } else {
      MT* dVc = (MT*)a.dVn + (crow * NT + c) * C * DV + (size_t)(4 * j) * DV + col;
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) dVc[(16 * mi + r) * DV] = from_f<MT>(X[mi][r]);
    }
  };

  f4 dS[ND];
  load_state(dS, a.dsT, (size_t)hr * DK * DV, DV, col);

  if (cb < ce && NBUF == 2) lds_barrier();   // the last chunk is in LDS
  // The loop issues no global loads: a wait for one would also wait for the chunk's stores issued before it.
  for (int c = ce - 1, it = 0; c >= cb; --c, ++it) {
    const int buf = (NBUF == 2) ? (it & 1) : 0;
    store_ds(c, dS);
    if (NBUF == 1) lds_barrier();        // chunk c is in LDS
    float gl;
    int t0, tend;
    if constexpr (DIRECT) {
      gl = a.GL[crow * NT + c];
      chunk_span(a.pack, NT, c, T, t0, tend);
    } else {
      const int* sc = (const int*)(lds + L::O_SCAL) + 4 * buf;
      gl = __int_as_float(sc[0]);
      t0 = sc[1];
      tend = sc[2];
    }
    const MT* st = lds + buf * SZ;
    // the chunk's tiles: diag(e) K^, diag(gamma) Q^, W, M
    const size_t bhc = crow * NT + c;
    const MT* tK = DIRECT ? (const MT*)a.Ke + bhc * C * DK : st;
    const MT* tQ = DIRECT ? (const MT*)a.Qg + bhc * C * DK : st + O_Q;
    const MT* tW = DIRECT ? (const MT*)a.W + bhc * C * DK : st + O_W;
    const MT* tM = DIRECT ? (const MT*)a.M + bhc * C * C : st + O_M;

    Frag<MT> Of[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      if constexpr (DIRECT)    // dO rows of the lane's column straight from memory (zeros past the sequence end)
        Of[p] = frag_rows<MT, MT>((const MT*)a.dO + o_base, o_pitch, t0, tend, 32 * p, col, One());
      else if constexpr (sizeof(MT) == 2) Of[p] = frag_tr(st + O_O, GO::PITCH, 32 * p, w * 16);
      else Of[p] = frag_tile_rows<MT, GO>(st + O_O, 32 * p, w * 16 + (l & 15));
      if (!DIRECT && t0 + C > tend)   // rows past the sequence end hold copies of its last row: zero them
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (t0 + 32 * p + kmap(j, e) >= tend) Of[p].set(e, 0.f);
    }
    Frag<MT> Sf[ND / 2];
#pragma unroll
    for (int p = 0; p < ND / 2; ++p) Sf[p] = frag_acc<MT>(dS[2 * p], dS[2 * p + 1]);
    // dVn = M^T dO + diag(e) K^ dS   (M^T upper triangular: k-blocks before the row block are zero).  Float32 at key
    // widths 64 and 128 sums in the key-split pass's order (state_bwd_ks): the two row halves of dS apart, M^T dO
    // with the first half for row blocks 0, 1 and with the second for 2, 3, then the halves added.
    constexpr bool HALVES = sizeof(MT) == 4 && (DK == 64 || DK == 128);
    f4 dV[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      Frag<MT> fk[ND / 2];
#pragma unroll
      for (int p = 0; p < ND / 2; ++p) fk[p] = frag_tile<MT, FK>(tK, 16 * mi, 32 * p);
      f4 acc = {0.f, 0.f, 0.f, 0.f}, acch = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < ND / 2; ++p) mma((HALVES && p >= ND / 4) ? acch : acc, fk[p], Sf[p]);
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (32 * p + 31 >= 16 * mi)
          mma((HALVES && mi >= 2) ? acch : acc, frag_tile_tr<MT, FM>(tM, 32 * p, 16 * mi), Of[p]);
      dV[mi] = HALVES ? acc + acch : acc;
    }
    Frag<MT> Vf[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) Vf[p] = frag_acc<MT>(dV[2 * p], dV[2 * p + 1], -1.f);
    store_dv(c, dV);
    // dS <- exp(G_last) dS + (diag(gamma) Q^)^T dO - W^T dVn
    f4 dSn[ND];
#pragma unroll
    for (int di = 0; di < ND; ++di) {
      Frag<MT> fw[2], fq[2];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        fw[p] = frag_tile_tr<MT, FK>(tW, 32 * p, 16 * di);
        fq[p] = frag_tile_tr<MT, FK>(tQ, 32 * p, 16 * di);
      }
      f4 acc = dS[di] * gl;
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        mma(acc, fw[p], Vf[p]);
        mma(acc, fq[p], Of[p]);
      }
      dSn[di] = acc;
    }
#pragma unroll
    for (int di = 0; di < ND; ++di) dS[di] = dSn[di];
    if constexpr (!DIRECT) lds_barrier();   // end of chunk c
  }
#pragma unroll
  for (int di = 0; di < ND; ++di)
#pragma unroll
    for (int r = 0; r < 4; ++r) a.ds0[(size_t)hr * DK * DV + (16 * di + 4 * j + r) * DV + col] = dS[di][r];
}

template <typename MT, int DK, int NW, int KS = 1>
__global__ void __launch_bounds__(64 * (KS * NW + 1)) state_bwd_kernel(StateBwdArgs a) {
  __shared__ __attribute__((aligned(1024))) MT lds[StateBwdLds<MT, DK, NW, KS>::ELEMS];
  state_bwd_body<MT, DK, NW, KS>(a, lds, blockIdx.x);
}

// The backward's recompute pass (storing S_c, Vn) and its reverse pass in one launch: they read prep's outputs and
// not each other's, so workgroups [0, nfwd) run the first and the rest the second, side by side on the CUs, with no
// stream synchronisation between them.
template <typename MT, int DK, int NW, int KS = 1>
__global__ void __launch_bounds__(64 * (KS * NW + 1)) state_pair_kernel(StateFwdArgs af, StateBwdArgs ab, int nfwd) {
  constexpr int EF = StateFwdLds<MT, DK, false, true, NW, KS>::ELEMS, EB = StateBwdLds<MT, DK, NW, KS>::ELEMS;
  __shared__ __attribute__((aligned(1024))) MT lds[EF > EB ? EF : EB];
  if ((int)blockIdx.x < nfwd) state_fwd_body<MT, DK, NW, false, true, false, KS>(af, lds, blockIdx.x);
  else state_bwd_body<MT, DK, NW, KS>(ab, lds, blockIdx.x - nfwd);
}

// ---------------------------------------------------------------------------------------------------------------------
// the per-chunk backward: dq, dk, dv, dg, dbeta
// ---------------------------------------------------------------------------------------------------------------------
enum { P_QD = 0, P_E, P_KX, P_R1, P_R2, P_VY, P_DQ, P_DK, NPART };

template <typename MT>
__device__ __forceinline__ Frag<MT> zero_frag() {
  Frag<MT> o;
#pragma unroll
  for (int r = 0; r < 8; ++r) o.set(r, 0.f);
  return o;
}

// The fp32 per-chunk backward (bf16 operands take chunk_bwd8_kernel): one workgroup of NW = cb32_waves(DK) waves per
// (chunk, head, batch row), fragments read straight from global memory (fp32 tiles do not fit LDS).  The prologue's
// row scales (q^ = q rq DK^-1/2, k^ = k rk) are applied to the products' rows and columns, and folded into the stored
// dM and Z, so the raw inputs are the MFMA operands.  Wave w owns key-column blocks w, w + NW, ... of the [C x DK]
// products and value-column blocks w, w + NW, ..., and of the [C x C] ones column block w % 4, row tiles
// TPW (w / 4) .. TPW (w / 4) + TPW - 1 (TPW = 16 / NW: all four with 4 waves, two with 8).  8 waves (two a SIMD) hide
// each other's global-load latency; at key widths above 128 the fp32 tiles leave LDS for 4 only.
constexpr int cb32_waves(int DK) { return DK <= 128 ? 8 : 4; }
// IT: the type of q, k, v and of dq, dk, dv in memory (bf16 with MACAI_GDR_BF16_F32: read exactly, the gradients
// rounded once from float32); dO and the per-chunk operands are MT.
template <typename MT, int DK, int DVT, typename IT = MT>
__global__ void __launch_bounds__(64 * cb32_waves(DK)) chunk_bwd_kernel(ChunkBwdArgs a) {
  static_assert(sizeof(MT) == 4, "bf16 operands take chunk_bwd8_kernel");
  const int DV = DVT ? DVT : a.DV;        // DVT = 0: the value width at run time (a multiple of 32)
  constexpr int KP = DK + 8, CP = C + 8;
  constexpr int NW = cb32_waves(DK);
  constexpr int RH = NW / 4, TPW = 4 / RH;   // row groups of the C x C tiles, row tiles a wave owns there
  constexpr int NBD = DK / 16;            // 16-column blocks of the key width
  constexpr int NBW = (NBD + NW - 1) / NW;   // most blocks a wave owns
  __shared__ __attribute__((aligned(16))) MT sdW[C * KP];   // dW = -dVn S_c^T
  __shared__ __attribute__((aligned(16))) MT sdMk[C * CP];  // dM diag(rk):            [t][s] = dM[t][s] rk_s
  __shared__ __attribute__((aligned(16))) MT sdMq[C * CP];  // dM^T diag(rq DK^-1/2):  [t][s] = dM[s][t] rq_s qs
  __shared__ __attribute__((aligned(16))) MT sZk[C * CP];   // Z diag(rk), Z = diag(beta) P + (diag(beta) P)^T
  __shared__ __attribute__((aligned(16))) MT sdA[C * CP];   // dA
  __shared__ ChunkScalars cs;
  __shared__ float rk[C], rq[C];
  __shared__ float part[NPART][NW][C];
  __shared__ float partS[NW];
  __shared__ float colR1[RH][C], colR2b[RH][C];

  const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int H = a.H, NT = a.NT;
  int t0, T;                               // the chunk's first token; T: its sequence's end (the bound for its rows)
  chunk_span(a.pack, NT, c, a.T, t0, T);
  const int nrows = (T - t0 < C) ? T - t0 : C;
  const int l = lane_id(), w = wave_id(), j = l >> 4;
  const size_t qk_base = ((size_t)b * a.T * a.Hk + h / (H / a.Hk)) * DK, qk_pitch = (size_t)a.Hk * DK;
  const size_t dqk_base = ((size_t)b * a.T * H + h) * DK, dqk_pitch = (size_t)H * DK;   // dq, dk: value heads
  const size_t v_base = ((size_t)b * a.T * H + h) * DV, v_pitch = (size_t)H * DV;
  const size_t s_base = (size_t)b * a.T * H + h;
  const size_t bhc = ((size_t)b * H + h) * NT + c;
  const IT* q = (const IT*)a.q + qk_base;
  const IT* k = (const IT*)a.k + qk_base;
  const IT* v = (const IT*)a.v + v_base;
  const MT* dO = (const MT*)a.dO + v_base;
  const float* Scc = a.Sc + bhc * DK * DV;
  const float* dSc = a.dSn + bhc * DK * DV;
  const MT* Vnc = (const MT*)a.Vn + bhc * C * DV;
  const MT* dVc = (const MT*)a.dVn + bhc * C * DV;
  const MT* Ac = (const MT*)a.A + bhc * C * C;
  const float qs = a.q_scale;

  if (w == 0) chunk_scalars(cs, a.g, a.beta, s_base, H, t0, T);
  if (a.l2norm) {
    if constexpr (NW == 8) {               // k's norms on waves 0-3, q's on 4-7 (the same sums as on one wave set)
      if (w < 4) row_rnorms<IT, DK>(rk, (const IT*)a.k, qk_base, qk_pitch, t0, T, 4, w);
      else row_rnorms<IT, DK>(rq, (const IT*)a.q, qk_base, qk_pitch, t0, T, 4, w - 4);
    } else {
      row_rnorms<IT, DK>(rk, (const IT*)a.k, qk_base, qk_pitch, t0, T, 4);
      row_rnorms<IT, DK>(rq, (const IT*)a.q, qk_base, qk_pitch, t0, T, 4);
    }
  } else if (threadIdx.x < C) {
    rk[threadIdx.x] = (int)threadIdx.x < nrows ? 1.f : 0.f;
    rq[threadIdx.x] = (int)threadIdx.x < nrows ? 1.f : 0.f;
  }
  __syncthreads();

  // operand accessors: raw rows (zero past the sequence end)
  auto fq = [&](int row0, int k0) { return frag_k_seq<MT, IT>(q, qk_pitch, t0, T, row0, k0, One()); };
  auto fk = [&](int row0, int k0) { return frag_k_seq<MT, IT>(k, qk_pitch, t0, T, row0, k0, One()); };
  // key widths up to 128: the row fragments' loads issued together (frag_rows_eager); 256 keeps frag_rows (it spills)
  constexpr bool EAGER = DK <= 128;
  auto fqrows = [&](int krow0, int col) {
    if constexpr (EAGER) return frag_rows_eager<MT, IT>(q, qk_pitch, t0, T, krow0, col, One());
    else return frag_rows<MT, IT>(q, qk_pitch, t0, T, krow0, col, One());
  };
  auto fkrows = [&](int krow0, int col) {
    if constexpr (EAGER) return frag_rows_eager<MT, IT>(k, qk_pitch, t0, T, krow0, col, One());
    else return frag_rows<MT, IT>(k, qk_pitch, t0, T, krow0, col, One());
  };
  auto fO = [&](int row0, int k0) { return frag_k_seq<MT, MT>(dO, v_pitch, t0, T, row0, k0, One()); };
  auto fVn = [&](int row0, int k0) { return frag_k<MT, MT>(Vnc, DV, row0, k0); };
  auto fdVn = [&](int row0, int k0) { return frag_k<MT, MT>(dVc, DV, row0, k0); };
  auto fdVnrows = [&](int krow0, int col) {
    if constexpr (EAGER) return frag_rows_eager<MT, MT>(dVc, DV, 0, C, krow0, col, One());
    else return frag_rows<MT, MT>(dVc, DV, 0, C, krow0, col, One());
  };
  // A^T rows row0.. (A operand): column row0 + l % 16 of A, k over A's rows
  auto fAt = [&](int row0, int k0) {
    if constexpr (EAGER) return frag_rows_eager<MT, MT>(Ac, C, 0, C, k0, row0 + (l & 15), One());
    else return frag_rows<MT, MT>(Ac, C, 0, C, k0, row0 + (l & 15), One());
  };
  // raw q / k at (chunk row, key column) times the row's inverse norm: the unit-norm direction (zero past the end).
  // EAGER: the load unconditional (a row past the end reads the last row) and the mask on the multiplier, so the
  // compiler cannot sink the load into a per-row branch and wait for it there (rows past the end only ever feed
  // their own masked partial sums).
  auto xq = [&](int row, int d) -> float {
    if constexpr (EAGER) {
      const float x = to_f(q[(size_t)(t0 + row < T ? t0 + row : T - 1) * qk_pitch + d]);
      return x * ((t0 + row < T) ? rq[row] : 0.f);
    } else {
      return (t0 + row < T) ? to_f(q[(size_t)(t0 + row) * qk_pitch + d]) * rq[row] : 0.f;
    }
  };
  auto xk = [&](int row, int d) -> float {
    if constexpr (EAGER) {
      const float x = to_f(k[(size_t)(t0 + row < T ? t0 + row : T - 1) * qk_pitch + d]);
      return x * ((t0 + row < T) ? rk[row] : 0.f);
    } else {
      return (t0 + row < T) ? to_f(k[(size_t)(t0 + row) * qk_pitch + d]) * rk[row] : 0.f;
    }
  };

  // ---- B: products with the chunk states; wave w owns key-column blocks w, w + NW, ...
  f4 dQ[NBW][4], dK[NBW][4];
  float pQD[4][4], pE[4][4], pKX[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) pQD[mi][r] = pE[mi][r] = pKX[mi][r] = 0.f;
  float sds = 0.f;
#pragma unroll
  for (int ib = 0; ib < NBW; ++ib) {
    const int nb = w + NW * ib;
    if (nb >= NBD) break;
    const int d0 = 16 * nb, d = d0 + (l & 15);
    f4 aO[4], aV[4], aD[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) aO[mi] = aV[mi] = aD[mi] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < DV / 32; ++kb) {
      const Frag<float> s32 = frag_k_f32(Scc, DV, d0, 32 * kb);
      const Frag<MT> bS = cvt<MT>(s32);
      const Frag<MT> bD = frag_k<MT, float>(dSc, DV, d0, 32 * kb);
#pragma unroll
      for (int r = 0; r < 8; ++r) sds = fmaf(s32.v[r], bD.get(r), sds);
      Frag<MT> fo[4], fv[4], fd[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        fo[mi] = fO(16 * mi, 32 * kb);
        fv[mi] = fVn(16 * mi, 32 * kb);
        fd[mi] = fdVn(16 * mi, 32 * kb);
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        mma(aO[mi], fo[mi], bS);
        mma(aV[mi], fv[mi], bD);
        mma(aD[mi], fd[mi], bS);
      }
    }
    float kv[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mi + 4 * j + r;
        const float qv = xq(row, d) * qs;
        kv[mi][r] = xk(row, d);
        const float oq = aO[mi][r] * cs.gam[row];
        dQ[ib][mi][r] = oq;
        pQD[mi][r] = fmaf(qv, oq, pQD[mi][r]);
        const float ve = aV[mi][r] * cs.e[row];
        dK[ib][mi][r] = ve;
        pE[mi][r] = fmaf(kv[mi][r], ve, pE[mi][r]);
        sdW[row * KP + d] = from_f<MT>(-aD[mi][r]);
      }
    // X = A^T dW = -A^T (dVn S_c^T)   (A^T upper triangular)
    Frag<MT> xf[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) xf[p] = frag_acc<MT>(aD[2 * p], aD[2 * p + 1], -1.f);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
      f4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (32 * p + 31 >= 16 * mi) mma(x, fAt(16 * mi, 32 * p), xf[p]);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mi + 4 * j + r;
        dK[ib][mi][r] = fmaf(cs.beta[row] * cs.gam[row], x[r], dK[ib][mi][r]);
        pKX[mi][r] = fmaf(kv[mi][r], x[r], pKX[mi][r]);
      }
    }
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float s1 = group16_sum(pQD[mi][r]), s2 = group16_sum(pE[mi][r]), s3 = group16_sum(pKX[mi][r]);
      if ((l & 15) == 0) {
        const int row = 16 * mi + 4 * j + r;
        part[P_QD][w][row] = s1;
        part[P_E][w][row] = s2;
        part[P_KX][w][row] = s3;
      }
    }
  sds = across_groups_sum(group16_sum(sds));
  if (l == 0) partS[w] = sds;
  __syncthreads();

  // ---- C: the C x C products; wave w owns column block cb = w % 4, row tiles mi = TPW hh + i (hh = w / 4)
  const int cb = w & 3, hh = w >> 2, s = 16 * cb + (l & 15);
  f4 QK[TPW], KK[TPW], dOV[TPW], Ta[TPW], Tb[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) QK[i] = KK[i] = dOV[i] = Ta[i] = Tb[i] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int p = 0; p < DK / 32; ++p) {
    const Frag<MT> bk = fk(16 * cb, 32 * p);
    Frag<MT> fa[TPW], fb[TPW], fw[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int mi = TPW * hh + i;
      fa[i] = fq(16 * mi, 32 * p);
      fb[i] = fk(16 * mi, 32 * p);
      fw[i] = frag_k_raw(sdW, KP, 16 * mi, 32 * p);
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      mma(QK[i], fa[i], bk);
      mma(KK[i], fb[i], bk);
      mma(Ta[i], fw[i], bk);
    }
  }
#pragma unroll
  for (int kb = 0; kb < DV / 32; ++kb) {
    const Frag<MT> bvn = fVn(16 * cb, 32 * kb);
    const Frag<MT> bv = frag_k_seq<MT, IT>(v, v_pitch, t0, T, 16 * cb, 32 * kb, One());
    Frag<MT> fo[TPW], fd[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int mi = TPW * hh + i;
      fo[i] = fO(16 * mi, 32 * kb);
      fd[i] = fdVn(16 * mi, 32 * kb);
    }
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      mma(dOV[i], fo[i], bvn);
      mma(Tb[i], fd[i], bv);
    }
  }
  float gm[TPW][4], KG[TPW][4];
  {
    float cR1 = 0.f;
    float pR1[TPW][4];
    const float bs = cs.beta[s], bgs = cs.beta[s] * cs.gam[s], rks = rk[s];
#pragma unroll
    for (int i = 0; i < TPW; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * (TPW * hh + i) + 4 * j + r;
        gm[i][r] = (row >= s) ? cs.decay(row, s) : 0.f;
        const float Mv = QK[i][r] * (rq[row] * qs * rks) * gm[i][r];
        const float dMv = dOV[i][r] * gm[i][r];
        sdMk[row * CP + s] = from_f<MT>(dMv * rks);
        sdMq[s * CP + row] = from_f<MT>(dMv * (rq[row] * qs));
        const float r1 = (row > s) ? dOV[i][r] * Mv : 0.f;
        pR1[i][r] = r1;
        cR1 += r1;
        sdA[row * CP + s] = from_f<MT>((row > s) ? fmaf(Ta[i][r] * rks, bgs, Tb[i][r] * bs) : 0.f);
        KG[i][r] = (row > s) ? KK[i][r] * (rk[row] * rks) * gm[i][r] : 0.f;
      }
    cR1 = across_groups_sum(cR1);
    if (j == 0) colR1[hh][s] = cR1;
#pragma unroll
    for (int i = 0; i < TPW; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float t = group16_sum(pR1[i][r]);
        if ((l & 15) == 0) part[P_R1][w][16 * (TPW * hh + i) + 4 * j + r] = t;
      }
  }
  __syncthreads();
  // T1 = dA A^T (column block cb of T1, all four row tiles: each wave of the column block forms it), then dL =
  // strictLower(-A^T T1) on this wave's row tiles
  f4 T1[4], dL[TPW];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi) {
    T1[mi] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < 2; ++p)
      if (32 * p <= 16 * mi + 15 && 32 * p <= 16 * cb + 15)
        mma(T1[mi], frag_k_raw(sdA, CP, 16 * mi, 32 * p), frag_k<MT, MT>(Ac, C, 16 * cb, 32 * p));
  }
  Frag<MT> T1f[2];
#pragma unroll
  for (int p = 0; p < 2; ++p) T1f[p] = frag_acc<MT>(T1[2 * p], T1[2 * p + 1]);
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int mi = TPW * hh + i;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < 2; ++p)
      if (32 * p + 31 >= 16 * mi) mma(acc, fAt(16 * mi, 32 * p), T1f[p]);
    dL[i] = acc;
  }
  {
    float cR2 = 0.f;
    float pR2[TPW][4];
    const float rks = rk[s];
#pragma unroll
    for (int i = 0; i < TPW; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * (TPW * hh + i) + 4 * j + r;
        const float dl = (row > s) ? -dL[i][r] : 0.f;
        const float r2 = dl * KG[i][r];
        pR2[i][r] = r2;
        cR2 = fmaf(cs.beta[row], r2, cR2);
        const float z = cs.beta[row] * dl * gm[i][r];    // Z[row][s] = Z[s][row] = beta_row P[row][s]
        if (row > s) {
          sZk[row * CP + s] = from_f<MT>(z * rks);
          sZk[s * CP + row] = from_f<MT>(z * rk[row]);
        } else if (row == s) {
          sZk[row * CP + s] = from_f<MT>(0.f);
        }
      }
    cR2 = across_groups_sum(cR2);
    if (j == 0) colR2b[hh][s] = cR2;
#pragma unroll
    for (int i = 0; i < TPW; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float t = group16_sum(pR2[i][r]);
        if ((l & 15) == 0) part[P_R2][w][16 * (TPW * hh + i) + 4 * j + r] = t;
      }
  }
  __syncthreads();

  // ---- D: dQ^ += (dM diag(rk)) K; dK^ += (dM^T diag(rq qs)) Q + (Z diag(rk)) K   (own key-column blocks)
  float pDQ[4][4], pDK[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) pDQ[mi][r] = pDK[mi][r] = 0.f;
#pragma unroll
  for (int ib = 0; ib < NBW; ++ib) {
    const int nb = w + NW * ib;
    if (nb >= NBD) break;
    const int d = 16 * nb + (l & 15);
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const Frag<MT> bK = fkrows(32 * p, d);
      const Frag<MT> bQ = fqrows(32 * p, d);
      Frag<MT> fm[4], fmt[4], fz[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        fm[mi] = frag_k_raw(sdMk, CP, 16 * mi, 32 * p);
        fmt[mi] = frag_k_raw(sdMq, CP, 16 * mi, 32 * p);
        fz[mi] = frag_k_raw(sZk, CP, 16 * mi, 32 * p);
      }
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        if (32 * p <= 16 * mi + 15) mma(dQ[ib][mi], fm[mi], bK);
        if (32 * p + 31 >= 16 * mi) mma(dK[ib][mi], fmt[mi], bQ);
        mma(dK[ib][mi], fz[mi], bK);
      }
    }
    if (a.l2norm) {
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * mi + 4 * j + r;
          pDQ[mi][r] = fmaf(xq(row, d), dQ[ib][mi][r], pDQ[mi][r]);
          pDK[mi][r] = fmaf(xk(row, d), dK[ib][mi][r], pDK[mi][r]);
        }
    }
  }
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float s1 = group16_sum(pDQ[mi][r]), s2 = group16_sum(pDK[mi][r]);
      if ((l & 15) == 0) {
        part[P_DQ][w][16 * mi + 4 * j + r] = s1;
        part[P_DK][w][16 * mi + 4 * j + r] = s2;
      }
    }

  // ---- E: Y = A^T dVn, dV = diag(beta) Y; v . Y row sums  (value-column blocks w, w + NW, ...)
  {
    float pVY[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) pVY[mi][r] = 0.f;
    for (int vb = w; vb < DV / 16; vb += NW) {
      const int vc = 16 * vb + (l & 15);
      Frag<MT> bdv[2];
#pragma unroll
      for (int p = 0; p < 2; ++p) bdv[p] = fdVnrows(32 * p, vc);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) {
        f4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int p = 0; p < 2; ++p)
          if (32 * p + 31 >= 16 * mi) mma(y, fAt(16 * mi, 32 * p), bdv[p]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int row = 16 * mi + 4 * j + r, t = t0 + row;
          // EAGER: loaded outside the branch (the last row past the end)
          const float vv = EAGER ? to_f(v[(size_t)(t < T ? t : T - 1) * v_pitch + vc]) : 0.f;
          if (t < T) {
            ((IT*)a.dv)[v_base + (size_t)t * v_pitch + vc] = from_f<IT>(cs.beta[row] * y[r]);
            pVY[mi][r] = fmaf(EAGER ? vv : to_f(v[(size_t)t * v_pitch + vc]), y[r], pVY[mi][r]);
          }
        }
      }
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float t = group16_sum(pVY[mi][r]);
        if ((l & 15) == 0) part[P_VY][w][16 * mi + 4 * j + r] = t;
      }
  }
  __syncthreads();

  // ---- F: dbeta and dg (wave 0, lane = chunk row), fixed-order sums of the per-wave partials
  if (w == 0) {
    const int r = l, t = t0 + r;
    auto sumw = [&](int pi) {              // over every wave, in wave order
      float x = part[pi][0][r];
#pragma unroll
      for (int u = 1; u < NW; ++u) x += part[pi][u][r];
      return x;
    };
    const int g0 = 4 * ((r >> 4) / TPW);   // the four waves whose C x C row tiles hold row r
    auto sumc = [&](int pi) { return ((part[pi][g0][r] + part[pi][g0 + 1][r]) + part[pi][g0 + 2][r]) + part[pi][g0 + 3][r]; };
    float cr1 = colR1[0][r], cr2 = colR2b[0][r];
#pragma unroll
    for (int u = 1; u < RH; ++u) {
      cr1 += colR1[u][r];
      cr2 += colR2b[u][r];
    }
    const float kx = sumw(P_KX), qd = sumw(P_QD), E = sumw(P_E), r1 = sumc(P_R1), r2 = sumc(P_R2), vy = sumw(P_VY);
    const float gmr = cs.gam[r], bt = cs.beta[r];
    const float db = fmaf(gmr, kx, vy) + r2;
    float dG = qd + bt * gmr * kx + (r1 - cr1) + (bt * r2 - cr2);
    if (r == C - 1) {
      float ss = partS[0];
#pragma unroll
      for (int u = 1; u < NW; ++u) ss += partS[u];
      dG += cs.gam[C - 1] * ss;
    }
    // dg_t = sum_{s >= t} dG_s + sum_{r < t} E_r; the exclusive prefix by a shift, not incl - E: E on the last valid
    // row is O(1) while the earlier ones carry exp(G_last - G_r) and can be ~1e-9 of it
    const float rev = __shfl(dG, C - 1 - r, 64);
    const float suf = __shfl(wave_incl_scan(rev), C - 1 - r, 64);
    float Esh = wave_shift_up1(E);
    if (r == 0) Esh = 0.f;
    const float pre = wave_incl_scan(Esh);
    if (t < T) {
      a.dg[s_base + (size_t)t * H] = suf + pre;
      a.dbeta[s_base + (size_t)t * H] = db;
    }
  }

  // ---- G: the prologue's backward, dq and dk out (own key-column blocks)
#pragma unroll
  for (int ib = 0; ib < NBW; ++ib) {
    const int nb = w + NW * ib;
    if (nb >= NBD) break;
    const int d = 16 * nb + (l & 15);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = 16 * mi + 4 * j + r, t = t0 + row;
        if (t >= T) continue;
        float gq = dQ[ib][mi][r], gk = dK[ib][mi][r];
        if (a.l2norm) {
          float dq_dot = part[P_DQ][0][row], dk_dot = part[P_DK][0][row];
#pragma unroll
          for (int u = 1; u < NW; ++u) {
            dq_dot += part[P_DQ][u][row];
            dk_dot += part[P_DK][u][row];
          }
          gq = qs * rq[row] * fmaf(-xq(row, d), dq_dot, gq);
          gk = rk[row] * fmaf(-xk(row, d), dk_dot, gk);
        } else {
          gq = qs * gq;
        }
        ((IT*)a.dq)[dqk_base + (size_t)t * dqk_pitch + d] = from_f<IT>(gq);
        ((IT*)a.dk)[dqk_base + (size_t)t * dqk_pitch + d] = from_f<IT>(gk);
      }
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// the per-chunk backward for bf16 operands: 8 waves, every operand in LDS
// ---------------------------------------------------------------------------------------------------------------------
// One workgroup of 8 waves (two per SIMD) per (chunk, head, batch row).  The chunk's raw q, k, dO and Vn, dVn, A
// are copied into padded LDS tiles at the start (asynchronous; rows past the sequence end are zeroed), and v replaces
// dO once dO is consumed.  The [C x D] products are formed transposed, as [D x C] with the chunk's tokens as the MFMA
// columns, so that in their epilogues a lane holds one token and 4 consecutive features: per-token scalars are lane
// values and the feature quads are 8-byte LDS accesses.  Contractions over chunk rows read their operand with LDS
// transpose reads.  The prologue's row scales (q^ = q rq DK^-1/2, k^ = k rk) are applied to products and folded into
// the stored dM and Z, so the raw inputs are the MFMA operands.  Wave w owns key block w and value block w (16
// features each) of the [D x C] products, and column block w % 4, row tiles 2 (w / 4) and 2 (w / 4) + 1 of the [C x C]
// ones.  dq, dk and dv are staged in LDS and written as whole rows.  With DK = DV the workgroups are persistent
// (chunk_bwd8xn_kernel, one a CU), each running a strided run of chunk-heads, the next one's reads issued while the
// current one computes.
// The workgroup's LDS, as pointers to its arrays (declared in the kernels by CB8_LDS).  The three value tiles and dW's
// tile are four arrays of one size (R1, R2, R3, R7; dW's tile is a value tile's size when DK = DV), so that a workgroup
// running a sequence of chunk-heads can take the next one's tiles into arrays the current one has finished with: dVn
// always in R3, while dO (then v), Vn (then dv) and dW rotate over R1, R2, R7 (chunk_bwd8xn_kernel).
struct Cb8Lds {
  bf16 *R1, *R2, *R3, *R7;
  bf16* tiles2;                            // q, k, A
  bf16 *sMkT, *sMqT, *sAZ;                 // [s][t] = dM[t][s] rk_s; [s][t] = dM[t][s] rq_t qs; dA^T, then Z rk
  ChunkScalars* cs;
  float *rk, *rq;
  float (*part)[8][C];
  float (*colp)[2][C];
  float* partS;
  float (*rowdot)[C];                      // the prologue's row dots of dq and dk, summed over key blocks
};
#define CB8_LDS(DK, DV)                                                                                              \
  constexpr int CB8_KP = (DK) + 12, CB8_CP = C + 4;                                                                  \
  constexpr int CB8_VE = RowTile<C, (DV)>::ELEMS > C * CB8_KP ? RowTile<C, (DV)>::ELEMS : C * CB8_KP;              \
  __shared__ __attribute__((aligned(16))) bf16 cb8_R1[CB8_VE];                                                       \
  __shared__ __attribute__((aligned(16))) bf16 cb8_R2[CB8_VE];                                                       \
  __shared__ __attribute__((aligned(16))) bf16 cb8_R3[RowTile<C, (DV)>::ELEMS];                                      \
  __shared__ __attribute__((aligned(16))) bf16 cb8_R7[CB8_VE];                                                       \
  __shared__ __attribute__((aligned(16))) bf16 cb8_t2[2 * RegRowTile<C, (DK)>::ELEMS + Tile<bf16, C, C>::ELEMS];    \
  __shared__ __attribute__((aligned(16))) bf16 cb8_mk[C * CB8_CP];                                                   \
  __shared__ __attribute__((aligned(16))) bf16 cb8_mq[C * CB8_CP];                                                   \
  __shared__ __attribute__((aligned(16))) bf16 cb8_az[C * CB8_CP];                                                   \
  __shared__ ChunkScalars cb8_cs;                                                                                    \
  __shared__ __attribute__((aligned(16))) float cb8_rk[C], cb8_rq[C];                                                \
  __shared__ float cb8_part[NPART][8][C];                                                                            \
  __shared__ float cb8_partS[8];                                                                                     \
  /* colp and rowdot live in the partial rows that P_R1 and P_R2 leave unused (those take column blocks 0-3) */     \
  const Cb8Lds L{cb8_R1, cb8_R2, cb8_R3, cb8_R7, cb8_t2, cb8_mk, cb8_mq, cb8_az, &cb8_cs, cb8_rk, cb8_rq, cb8_part,   \
                 reinterpret_cast<float(*)[2][C]>(&cb8_part[P_R1][4][0]), cb8_partS,                                 \
                 reinterpret_cast<float(*)[C]>(&cb8_part[P_R2][4][0])};

// A chunk-head's place in a flat order of (chunk, head, batch row), chunks fastest
__device__ __forceinline__ void cb8_unit(int u, int NT, int H, int& c, int& h, int& b) {
  c = u % NT;
  h = (u / NT) % H;
  b = u / (NT * H);
}

// The first round of workgroups (a.stagger of them, one a CU) starts in three groups 6.4K cycles apart.  Launched
// together, every CU issues its block's 233 KB of reads at once and waits on the memory system's backpressure, and
// the later rounds keep that lockstep (each CU's next workgroup starts when its last one ends); staggered, a third
// of the CUs load while the rest compute, and the offsets carry into the later rounds.  Measured at 4 rounds with
// the inputs out of the caches: 2.5-4% off the kernel (2 groups or 4 groups, and other offsets, gained less); in
// the training step, whose chunk states are still in the Infinity Cache, 0.4 us of its 111.
__device__ __forceinline__ void cb8_stagger(int stagger, unsigned flat) {
  if (stagger && flat < (unsigned)stagger)
    for (int i = 0, n = (int)(flat % 3u) * 50; i < n; ++i) __builtin_amdgcn_s_sleep(2);   // 128 cycles each
}

// One chunk-head (unit: its place in the flat (chunk, head, batch row) order), its dO / v, Vn / dv and dW tiles in
// the arrays tO, tVn, sdW (dVn's in R3).  first: its global reads are issued here; otherwise the previous chunk-head of
// the workgroup issued them (its tiles into these arrays, its chunk states into s32 / sD, its g and beta into gv, bv).
// next >= 0 (DK = DV): the chunk-head this workgroup runs after this one, whose reads are issued here while this one
// computes: its dO into sdW once dW is consumed (after C), its chunk states into s32 / sD (dead after the state
// products) a value block at a time in T1, dL and D, its Vn into tO and its dVn, g and beta in G.  The copies into
// LDS are issued unseen by the compiler (dma_exact_opaque), so the arrays may be chosen at run time, and each is
// waited for explicitly.
template <int DK, int DV>
__device__ __forceinline__ void chunk_bwd8_body(const ChunkBwdArgs& a, const Cb8Lds& L, int unit, int next, bool first,
                                                bf16* const tO, bf16* const tVn, bf16* const sdW,
                                                Frag<float> (&s32)[DV / 32], Frag<float> (&sD)[DV / 32], float& gv,
                                                float& bv) {
  int c, h, b;
  cb8_unit(unit, a.NT, a.H, c, h, b);
  using MT = bf16;
  constexpr int NW = 8;
  constexpr int NBD = DK / 16, NBV = DV / 16;   // feature blocks (<= NW)
  // CQ: the C x C tiles formed here (8-byte stores, any pitch) at 136 bytes a row, where both their fragment and
  // their transpose reads are free of LDS bank conflicts (at 144, A's pitch, fragment reads run at half rate)
  constexpr int KP = DK + 12, CP = C + 8, CQ = C + 4;
  using GQ = RegRowTile<C, DK>;            // q, k: through registers at a conflict-free pitch
  using GV = RowTile<C, DV>;               // dO (then v), Vn (then dv), dVn: row copies at a conflict-free pitch
  using GA = Tile<MT, C, C>;
  static_assert(GQ::PITCH == KP && GA::PITCH == CP && NBD <= NW && NBV <= NW, "chunk_bwd8 tiling");
  constexpr int VP = GV::PITCH;
  MT* const tiles2 = L.tiles2;
  MT* const sMkT = L.sMkT;
  MT* const sMqT = L.sMqT;
  MT* const sAZ = L.sAZ;
  ChunkScalars& cs = *L.cs;
  float* const rk = L.rk;
  float* const rq = L.rq;
  float(*const part)[8][C] = L.part;
  float(*const colp)[2][C] = L.colp;
  float* const partS = L.partS;
  float(*const rowdot)[C] = L.rowdot;
  const int H = a.H, NT = a.NT;
  int t0, T;                               // the chunk's first token; T: its sequence's end (the bound for its rows)
  chunk_span<true>(a.pack, NT, c, a.T, t0, T);   // through the scalar cache: no wait on copies in flight
  const int nrows = (T - t0 < C) ? T - t0 : C;
  // The lane and wave numbers pass through empty assembly: a workgroup running several chunk-heads then forms each
  // one's lane-dependent offsets afresh instead of keeping the previous one's live across it (which spills).
  int l = lane_id(), w = __builtin_amdgcn_readfirstlane(wave_id());
  asm volatile("" : "+v"(l));
  asm volatile("" : "+s"(w));
  const int j = l >> 4, n = l & 15, tid = 64 * w + l;
  const size_t qk_base = ((size_t)b * a.T * a.Hk + h / (H / a.Hk)) * DK, qk_pitch = (size_t)a.Hk * DK;
  const size_t dqk_base = ((size_t)b * a.T * H + h) * DK, dqk_pitch = (size_t)H * DK;   // dq, dk: value heads
  const size_t v_base = ((size_t)b * a.T * H + h) * DV, v_pitch = (size_t)H * DV;
  const size_t s_base = (size_t)b * a.T * H + h;
  const size_t bhc = ((size_t)b * H + h) * NT + c;
  const MT* q = (const MT*)a.q + qk_base;
  const MT* k = (const MT*)a.k + qk_base;
  const MT* v = (const MT*)a.v + v_base;
  const MT* dO = (const MT*)a.dO + v_base;
  const float* Scc = a.Sc + bhc * DK * DV;
  const float* dSc = a.dSn + bhc * DK * DV;
  const MT* Vnc = (const MT*)a.Vn + bhc * C * DV;
  const MT* dVc = (const MT*)a.dVn + bhc * C * DV;
  const MT* Ac = (const MT*)a.A + bhc * C * C;
  const float qs = a.q_scale;
  MT* const tq = tiles2;
  MT* const tk = tiles2 + GQ::ELEMS;
  MT* const tA = tiles2 + 2 * GQ::ELEMS;
  MT* const tdV = L.R3;
  const int cb = w & 3, hh = w >> 2;       // [C x C] column block and row half
  constexpr int NSTATE = 4 * (DV / 32);   // state loads a wave issues: two 16-byte loads a fragment
  constexpr bool HOLDS_STATES = NBD == NW;  // every wave holds a key block of the states (else waves w < NBD)
  const bool holds = HOLDS_STATES || w < NBD;

  // ---- 0: global reads in two groups.  Group 1 is what the state products of B consume: the dO, Vn, dVn tiles and
  // the chunk states (into registers), issued in that order.  Loads retire in issue order, so once at most the state
  // loads are outstanding the tiles have landed: B starts then, and each value block's states are waited for at their
  // first use, so the tail of group 1 (the states are 128 of its 176 KiB) overlaps the first stages.  Group 2 -- the v
  // fragments and the q, k, A tiles -- lands while B runs.  Every read is unconditional (rows past the end re-read the
  // last row and are masked later).
  // (gv, bv: this lane's g and beta, used by wave 0; s32, sD: S_c and dS_{c+1} rows of key block w, A operands with
  // k = value features)
  if (first) {
    {
      const size_t o = s_base + (size_t)(t0 + l < T ? t0 + l : T - 1) * H;
      gv = a.g[o];
      bv = a.beta[o];
    }
    GV::template dma_rows_opaque<NW>(tO, dO + (size_t)t0 * v_pitch, v_pitch, w, nrows, l);
    GV::template dma_rows_opaque<NW>(tVn, Vnc, DV, w, C, l);
    GV::template dma_rows_opaque<NW>(tdV, dVc, DV, w, C, l);
    __builtin_amdgcn_sched_barrier(0);    // the state loads stay behind the copies (the partial wait below counts on it)
    if (holds) {
#pragma unroll
      for (int kb = 0; kb < DV / 32; ++kb) {
        s32[kb] = frag_k_f32(Scc, DV, 16 * w, 32 * kb, l);
        sD[kb] = frag_k_f32(dSc, DV, 16 * w, 32 * kb, l);
      }
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<NSTATE>();                // g, beta and the tiles have landed; the states may still be in flight
    } else {
      wait_dma();
    }
  } else {
    wait_dma();                            // issued by the previous chunk-head (and its global stores)
  }
  // Group 2 -- the v fragments and the q, k, A tile units -- goes through registers. Its loads are spread over the
  // state products' stages below: an issue stalls while the memory system is saturated, so issuing them all here
  // would hold the products back. The tile units are written to LDS after the products.
  constexpr int NQ = GQ::rows_per_wave(NW), NA = GA::per_wave(NW);
  constexpr int NG2 = DV / 32 + 2 * NQ + NA;                   // load slots: v fragments, q units, k units, A units
  Frag<MT> vf[DV / 32];                   // v rows of column block cb (B operand of dVn V^T)
  u32x4 uq[NQ], uk[NQ], ua[NA];
  const int tv = t0 + 16 * cb + n;        // this lane's v row
  const MT* const pv = v + (size_t)(tv < T ? tv : T - 1) * v_pitch + 4 * j;
  auto issue_g2 = [&](int sl) {
    if (sl < DV / 32) {
      const bf16x4 lo = *reinterpret_cast<const bf16x4*>(pv + 32 * sl), hi = *reinterpret_cast<const bf16x4*>(pv + 32 * sl + 16);
      vf[sl].v = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    } else if (sl < DV / 32 + NQ) {
      uq[sl - DV / 32] = GQ::template load_row_unit<NW>(q + (size_t)t0 * qk_pitch, qk_pitch, w, sl - DV / 32, nrows, l);
    } else if (sl < DV / 32 + 2 * NQ) {
      uk[sl - DV / 32 - NQ] = GQ::template load_row_unit<NW>(k + (size_t)t0 * qk_pitch, qk_pitch, w, sl - DV / 32 - NQ, nrows,
                                                             l);
    } else if (sl < NG2) {
      ua[sl - DV / 32 - 2 * NQ] = GA::template load_unit<NW>(Ac, C, w, sl - DV / 32 - 2 * NQ, C, l);
    }
  };
  if (w == 0) chunk_scalars_from(cs, t0 + l < T ? gv : 0.f, t0 + l < T ? bv : 0.f, t0, T, l);
  // the chunk states in their MFMA forms, value block by value block at its first stage, as hi + lo bf16 pairs where
  // one rounding shows: dS_{c+1} (the e k . (Vn dS^T) terms of dg sum 64 rows of it) and S_c in S_c dO^T (gamma
  // q . (S_c dO^T) in dg and dq cancels when the state is large against the output's gradient: with N(0, 1) starting
  // states the oracle's rounding model put 3 of 90 random draws over 1e-2 on dg with S_c rounded once, 1 with the
  // pair; in dW = -S_c dVn^T its one rounding changes nothing there); and the last-row dg term <S_c, dS_{c+1}> from
  // the fp32 values, in value-block order
  Frag<MT> fS[DV / 32], fSl[DV / 32], dHi[DV / 32], dLo[DV / 32];
  float sds = 0.f;
  auto states = [&](int kb) {
    frag_split<MT>(s32[kb], fS[kb], fSl[kb]);
    frag_split<MT>(sD[kb], dHi[kb], dLo[kb]);
#pragma unroll
    for (int r = 0; r < 8; ++r) sds = fmaf(s32[kb].v[r], sD[kb].v[r], sds);
  };
  lds_barrier();                         // the group-1 tiles and the chunk scalars visible
  if (nrows < C) {                         // rows past the end: zeros in dO
    constexpr int UV = VP / 4;             // 8-byte units (rows are 8-byte aligned)
    const int nz = C - nrows;
    for (int i = tid; i < nz * UV; i += 64 * NW)
      *reinterpret_cast<bf16x4*>(tO + (nrows + i % nz) * VP + 4 * (i / nz)) = bf16x4{};
    lds_barrier();
  }

  // ---- B: products with the chunk states, transposed: [key block w] x [token tiles]
  //   dQ^T = gamma * (S_c dO^T),  dK^T = e * (dS Vn^T),  dW^T = -(S_c dVn^T),  X^T = dW^T A,  dK^T += beta gamma X^T
  f4 dQt[4], dKt[4];
  f4 aO[4], aV[4], aD[4];
  constexpr int NS = 2 * (DV / 32), PER = (NG2 + NS - 1) / NS;   // stages; group-2 loads issued per stage
  if (holds) {
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) aO[ti] = aV[ti] = aD[ti] = f4{0.f, 0.f, 0.f, 0.f};
    // stage sg = (value block kb = sg / 2, token tiles 2 (sg % 2) and 2 (sg % 2) + 1): its dO, Vn, dVn fragments are
    // read one stage ahead of its products
    Frag<MT> st[2][6];
    auto load = [&](int sg, Frag<MT>(&f)[6]) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ti = 2 * (sg & 1) + u;
        f[3 * u] = frag_tile<MT, GV>(tO, 16 * ti, 32 * (sg >> 1));
        f[3 * u + 1] = frag_tile<MT, GV>(tVn, 16 * ti, 32 * (sg >> 1));
        f[3 * u + 2] = frag_tile<MT, GV>(tdV, 16 * ti, 32 * (sg >> 1));
      }
    };
    load(0, st[0]);
#pragma unroll
    for (int sg = 0; sg < NS; ++sg) {
      if ((sg & 1) == 0) states(sg >> 1);
#pragma unroll
      for (int p = 0; p < PER; ++p) issue_g2(PER * sg + p);
      if (sg + 1 < NS) load(sg + 1, st[(sg + 1) & 1]);
      const int kb = sg >> 1;
      const Frag<MT>(&f)[6] = st[sg & 1];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int ti = 2 * (sg & 1) + u;
        mma(aO[ti], fS[kb], f[3 * u]);
        mma(aO[ti], fSl[kb], f[3 * u]);
        mma(aV[ti], dHi[kb], f[3 * u + 1]);
        mma(aV[ti], dLo[kb], f[3 * u + 1]);
        mma(aD[ti], fS[kb], f[3 * u + 2]);
      }
    }
  } else {
#pragma unroll
    for (int sl = 0; sl < NG2; ++sl) issue_g2(sl);
  }
  wait_dma();                              // group 2 is in registers
#pragma unroll
  for (int u = 0; u < NQ; ++u) {
    GQ::template store_row_unit<NW>(tq, w, u, uq[u], l);
    GQ::template store_row_unit<NW>(tk, w, u, uk[u], l);
  }
#pragma unroll
  for (int u = 0; u < NA; ++u) GA::template store_unit<NW>(tA, w, u, ua[u], l);
  lds_barrier();                         // group 2 visible
  if (tv >= T) {                           // v rows past the end
#pragma unroll
    for (int kb = 0; kb < DV / 32; ++kb) vf[kb].v = bf16x8{};
  }
  if (nrows < C) {                         // rows past the end: zeros in q and k (the norms read rows < nrows only)
    constexpr int UQ = KP / 4;             // 8-byte units (rows are 8-byte aligned)
    const int nz = C - nrows;
    for (int i = tid; i < nz * 2 * UQ; i += 64 * NW) {
      const int row = nrows + i % nz, u = i / nz;
      *reinterpret_cast<bf16x4*>(u < UQ ? tq + row * KP + 4 * u : tk + row * KP + 4 * (u - UQ)) = bf16x4{};
    }
  }
  if (a.l2norm) {                          // the row norms from the tiles (rows past the end: 0)
    if (w < 4) row_rnorms_lds<DK>(rq, tq, KP, nrows, 4, w, l);
    else row_rnorms_lds<DK>(rk, tk, KP, nrows, 4, w - 4, l);
  } else if (tid < C) {
    rk[tid] = tid < nrows ? 1.f : 0.f;
    rq[tid] = tid < nrows ? 1.f : 0.f;
  }
  lds_barrier();                         // norms visible
  if (w < NBD) {
    const int d0 = 16 * w + 4 * j;        // this lane's 4 key features
    float pQD[4], pE[4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int t = 16 * ti + n;
      const f4 q4 = load4(tq + t * KP + d0), k4 = load4(tk + t * KP + d0);
      dQt[ti] = aO[ti] * cs.gam[t];
      dKt[ti] = aV[ti] * cs.e[t];
      pQD[ti] = (rq[t] * qs) * (((q4[0] * dQt[ti][0] + q4[1] * dQt[ti][1]) + q4[2] * dQt[ti][2]) + q4[3] * dQt[ti][3]);
      pE[ti] = rk[t] * (((k4[0] * dKt[ti][0] + k4[1] * dKt[ti][1]) + k4[2] * dKt[ti][2]) + k4[3] * dKt[ti][3]);
      *reinterpret_cast<bf16x4*>(sdW + t * KP + d0) =
          bf16x4{(bf16)(-aD[ti][0]), (bf16)(-aD[ti][1]), (bf16)(-aD[ti][2]), (bf16)(-aD[ti][3])};
    }
    // X^T = dW^T A (this wave's own dW^T columns, just written): A is lower triangular
    Frag<MT> fW[2];
    Frag<MT> fx[4][2];                     // A's nonzero blocks, all read before the products
#pragma unroll
    for (int p = 0; p < 2; ++p) fW[p] = frag_tr(sdW, KP, 32 * p, 16 * w, l);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (32 * p + 31 >= 16 * ti) fx[ti][p] = frag_tr(tA, CP, 32 * p, 16 * ti, l);
    float pKX[4];
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      f4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (32 * p + 31 >= 16 * ti) mma(x, fW[p], fx[ti][p]);
      const int t = 16 * ti + n;
      const f4 k4 = load4(tk + t * KP + d0);
      dKt[ti] += (cs.beta[t] * cs.gam[t]) * x;
      pKX[ti] = rk[t] * (((k4[0] * x[0] + k4[1] * x[1]) + k4[2] * x[2]) + k4[3] * x[3]);
    }
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const float s1 = across_groups_sum(pQD[ti]), s2 = across_groups_sum(pE[ti]), s3 = across_groups_sum(pKX[ti]);
      if (j == 0) {
        part[P_QD][w][16 * ti + n] = s1;
        part[P_E][w][16 * ti + n] = s2;
        part[P_KX][w][16 * ti + n] = s3;
      }
    }
    sds = across_groups_sum(group16_sum(sds));
    if (l == 0) partS[w] = sds;
  }
  lds_barrier();

  // ---- C: the C x C products on this wave's row tiles mi = 2 hh, 2 hh + 1 of column block cb.  Tiles above the
  // diagonal are computed too (their results are masked to zero below): no wave-dependent branch splits the loop, so the
  // fragment reads of stage s + 1 are issued before the products of stage s.
  float KG[2][4], gmv[2][4];
  {
    f4 QK[2], KK[2], Ta[2], dOV[2], Tb[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) QK[i] = KK[i] = Ta[i] = dOV[i] = Tb[i] = f4{0.f, 0.f, 0.f, 0.f};
    // stage s < NP: key features 32 s (B = k rows of block cb; A = q, k, dW rows of the two tiles);
    // stage NP + kb: value features 32 kb (B = Vn rows of block cb; A = dO rows; A = dVn rows against v)
    constexpr int NP = DK / 32, NS = NP + DV / 32;
    Frag<MT> st[2][7];
    auto load = [&](int sg, Frag<MT>(&f)[7]) {
      if (sg < NP) {
        f[0] = frag_tile<MT, GQ>(tk, 16 * cb, 32 * sg, l);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int mi = 2 * hh + i;
          f[1 + 3 * i] = frag_tile<MT, GQ>(tq, 16 * mi, 32 * sg, l);
          f[2 + 3 * i] = frag_tile<MT, GQ>(tk, 16 * mi, 32 * sg, l);
          f[3 + 3 * i] = frag_k_raw(sdW, KP, 16 * mi, 32 * sg, l);
        }
      } else {
        const int kb = sg - NP;
        f[0] = frag_tile<MT, GV>(tVn, 16 * cb, 32 * kb, l);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int mi = 2 * hh + i;
          f[1 + 2 * i] = frag_tile<MT, GV>(tO, 16 * mi, 32 * kb, l);
          f[2 + 2 * i] = frag_tile<MT, GV>(tdV, 16 * mi, 32 * kb, l);
        }
      }
    };
    load(0, st[0]);
#pragma unroll
    for (int sg = 0; sg < NS; ++sg) {
      if (sg + 1 < NS) load(sg + 1, st[(sg + 1) & 1]);
      const Frag<MT>(&f)[7] = st[sg & 1];
      if (sg < NP) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          mma(QK[i], f[1 + 3 * i], f[0]);
          mma(KK[i], f[2 + 3 * i], f[0]);
          mma(Ta[i], f[3 + 3 * i], f[0]);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          mma(dOV[i], f[1 + 2 * i], f[0]);
          mma(Tb[i], f[2 + 2 * i], vf[sg - NP]);
        }
      }
    }
    const int s = 16 * cb + n;
    const float bs = cs.beta[s], bgs = bs * cs.gam[s], rks = rk[s];
    const double Gs = cs.G[s];
    float pR1[8], cR1 = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int r0 = 16 * (2 * hh + i) + 4 * j;   // this lane's 4 rows
      const f4 rq4 = *reinterpret_cast<const f4*>(rq + r0), rk4 = *reinterpret_cast<const f4*>(rk + r0);
      float mk[4], mq[4], da[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = r0 + r;
        // the decay by the hardware exp2 (a bf16 kernel: its ~1e-6 relative error is far below the operands')
        const float gm = (row >= s) ? __builtin_amdgcn_exp2f((float)(cs.G[row] - Gs) * 1.4426950408889634f) : 0.f;
        gmv[i][r] = gm;
        const float Mv = QK[i][r] * (rq4[r] * qs * rks) * gm;
        const float dMv = dOV[i][r] * gm;
        mk[r] = dMv * rks;
        mq[r] = dMv * (rq4[r] * qs);
        const float r1 = (row > s) ? dOV[i][r] * Mv : 0.f;
        pR1[4 * i + r] = r1;
        cR1 += r1;
        da[r] = (row > s) ? fmaf(Ta[i][r] * rks, bgs, Tb[i][r] * bs) : 0.f;
        KG[i][r] = (row > s) ? KK[i][r] * (rk4[r] * rks) * gm : 0.f;
      }
      *reinterpret_cast<bf16x4*>(sMkT + s * CQ + r0) = bf16x4{(bf16)mk[0], (bf16)mk[1], (bf16)mk[2], (bf16)mk[3]};
      *reinterpret_cast<bf16x4*>(sMqT + s * CQ + r0) = bf16x4{(bf16)mq[0], (bf16)mq[1], (bf16)mq[2], (bf16)mq[3]};
      *reinterpret_cast<bf16x4*>(sAZ + s * CQ + r0) = bf16x4{(bf16)da[0], (bf16)da[1], (bf16)da[2], (bf16)da[3]};
    }
    const float rs = group16_sum8(pR1, l);            // row (l % 16) / 2 of the 8: tile i = idx / 4, r = idx % 4
    if ((n & 1) == 0) {
      const int idx = n >> 1;
      part[P_R1][cb][16 * (2 * hh + (idx >> 2)) + 4 * j + (idx & 3)] = rs;
    }
    cR1 = across_groups_sum(cR1);
    if (j == 0) colp[0][hh][s] = cR1;
  }
  lds_barrier();
  // dO is consumed: v takes its tile (needed from E on).  The copies are hidden from the compiler (dma_exact_opaque), so
  // it does not make the LDS reads of the next phases wait for them; the waits below are explicit.
  GV::template dma_rows_opaque<NW>(tO, v + (size_t)t0 * v_pitch, v_pitch, w, nrows, l);
  // The next chunk-head's reads, spread over the phases up to G: a wave's vector-memory issue stalls while the memory
  // system is saturated, so issued at once they would hold this chunk-head's compute back.  Its dO goes into dW's
  // array (consumed by C) now, its chunk states into s32 / sD (dead since B) a value block at a time in T1, dL and D,
  // its Vn and dVn into v's and dVn's arrays after E and in G.
  int nt0 = 0, nT = 0, nrows_n = 0;
  size_t nv_base = 0, nbhc = 0, ns_base = 0;
  const float *nS = nullptr, *ndS = nullptr;
  const bool pf = next >= 0;
  auto pf_state = [&](int kb) {
    if (pf && holds) {
      s32[kb] = frag_k_f32(nS, DV, 16 * w, 32 * kb, l);
      sD[kb] = frag_k_f32(ndS, DV, 16 * w, 32 * kb, l);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  {
    if (pf) {
      int nc, nh, nb;
      cb8_unit(next, NT, H, nc, nh, nb);
      chunk_span<true>(a.pack, NT, nc, a.T, nt0, nT);   // through the scalar cache: no wait on the copies above
      nrows_n = (nT - nt0 < C) ? nT - nt0 : C;
      nv_base = ((size_t)nb * a.T * H + nh) * DV;
      ns_base = (size_t)nb * a.T * H + nh;
      nbhc = ((size_t)nb * H + nh) * NT + nc;
      GV::template dma_rows_opaque<NW>(sdW, (const MT*)a.dO + nv_base + (size_t)nt0 * v_pitch, v_pitch, w, nrows_n, l);
      nS = a.Sc + nbhc * DK * DV;
      ndS = a.dSn + nbhc * DK * DV;
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // ---- T1 = dA A^T (column block cb, all four row tiles), then dL = strictLower(-A^T T1) on this wave's tiles
  {
    f4 T1[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) T1[mi] = f4{0.f, 0.f, 0.f, 0.f};
    // every operand read first; blocks of A above the diagonal are zero, so no wave-dependent skip is needed
    Frag<MT> bA[2], fz[6];
#pragma unroll
    for (int p = 0; p < 2; ++p) bA[p] = frag_tile<MT, GA>(tA, 16 * cb, 32 * p, l);   // B[s][t'] = A[t'][s]
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) fz[mi] = frag_tr(sAZ, CQ, 0, 16 * mi, l);
    fz[4] = frag_tr(sAZ, CQ, 32, 32, l);
    fz[5] = frag_tr(sAZ, CQ, 32, 48, l);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) mma(T1[mi], fz[mi], bA[0]);
    mma(T1[2], fz[4], bA[1]);              // dA is strictly lower: rows 0-31 have no terms at t' >= 32
    mma(T1[3], fz[5], bA[1]);
    pf_state(0);
    lds_barrier();                       // every wave has read dA^T: Z may overwrite it
    Frag<MT> T1f[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) T1f[p] = frag_acc<MT>(T1[2 * p], T1[2 * p + 1]);
    const int s = 16 * cb + n;
    const float rks = rk[s];
    float pR2[8], cR2 = 0.f;
    Frag<MT> fa[2][2];                     // A^T rows of the two tiles (A's zero upper blocks included)
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int p = 0; p < 2; ++p) fa[i][p] = frag_tr(tA, CP, 32 * p, 16 * (2 * hh + i));
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int mi = 2 * hh + i, r0 = 16 * mi + 4 * j;
      f4 dL = {0.f, 0.f, 0.f, 0.f};       // tiles above the diagonal (mi < cb) are masked by row > s below
#pragma unroll
      for (int p = 0; p < 2; ++p) mma(dL, fa[i][p], T1f[p]);
      const f4 rk4 = *reinterpret_cast<const f4*>(rk + r0), b4 = *reinterpret_cast<const f4*>(cs.beta + r0);
      float zt[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = r0 + r;
        const float dl = (row > s) ? -dL[r] : 0.f;
        const float r2 = dl * KG[i][r];
        pR2[4 * i + r] = r2;
        cR2 = fmaf(b4[r], r2, cR2);
        const float z = b4[r] * dl * gmv[i][r];     // Z[row][s] = Z[s][row] = beta_row P[row][s]
        zt[r] = z * rk4[r];
        if (mi == cb) {                              // diagonal tile: element by element
          if (row > s) {
            sAZ[s * CQ + row] = (bf16)zt[r];
            sAZ[row * CQ + s] = (bf16)(z * rks);
          } else if (row == s) {
            sAZ[s * CQ + row] = (bf16)0.f;
          }
        } else if (mi > cb) {
          sAZ[row * CQ + s] = (bf16)(z * rks);
        }
      }
      if (mi > cb)
        *reinterpret_cast<bf16x4*>(sAZ + s * CQ + r0) = bf16x4{(bf16)zt[0], (bf16)zt[1], (bf16)zt[2], (bf16)zt[3]};
    }
    pf_state(1);
    const float rs = group16_sum8(pR2, l);
    if ((n & 1) == 0) {
      const int idx = n >> 1;
      part[P_R2][cb][16 * (2 * hh + (idx >> 2)) + 4 * j + (idx & 3)] = rs;
    }
    cR2 = across_groups_sum(cR2);
    if (j == 0) colp[1][hh][s] = cR2;
  }
  lds_barrier();

  // ---- D: dQ^T += k^T (dM diag(rk))^T;  dK^T += q^T (diag(rq qs) dM) + k^T (diag(rk) Z)   (key block w)
  if (w < NBD) {
    Frag<MT> kT[2], qT[2];
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      kT[p] = frag_tr(tk, KP, 32 * p, 16 * w, l);
      qT[p] = frag_tr(tq, KP, 32 * p, 16 * w, l);
    }
    // token tile ti is one stage: its dM and Z fragments are read one stage ahead of its products
    Frag<MT> st[2][6];
    auto load = [&](int ti, Frag<MT>(&f)[6]) {
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (32 * p <= 16 * ti + 15) f[3 * p] = frag_tr(sMkT, CQ, 32 * p, 16 * ti, l);
        if (32 * p + 31 >= 16 * ti) f[3 * p + 1] = frag_k_raw(sMqT, CQ, 16 * ti, 32 * p, l);
        f[3 * p + 2] = frag_k_raw(sAZ, CQ, 16 * ti, 32 * p, l);
      }
    };
    load(0, st[0]);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      if (ti + 1 < 4) load(ti + 1, st[(ti + 1) & 1]);
      const Frag<MT>(&f)[6] = st[ti & 1];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (32 * p <= 16 * ti + 15) mma(dQt[ti], kT[p], f[3 * p]);
        if (32 * p + 31 >= 16 * ti) mma(dKt[ti], qT[p], f[3 * p + 1]);
        mma(dKt[ti], kT[p], f[3 * p + 2]);
      }
      if (ti == 1) pf_state(2);
    }
    pf_state(3);
    if (a.l2norm) {
      const int d0 = 16 * w + 4 * j;
#pragma unroll
      for (int ti = 0; ti < 4; ++ti) {
        const int t = 16 * ti + n;
        const f4 q4 = load4(tq + t * KP + d0), k4 = load4(tk + t * KP + d0);
        const float s1 = across_groups_sum(
            rq[t] * (((q4[0] * dQt[ti][0] + q4[1] * dQt[ti][1]) + q4[2] * dQt[ti][2]) + q4[3] * dQt[ti][3]));
        const float s2 = across_groups_sum(
            rk[t] * (((k4[0] * dKt[ti][0] + k4[1] * dKt[ti][1]) + k4[2] * dKt[ti][2]) + k4[3] * dKt[ti][3]));
        if (j == 0) {
          part[P_DQ][w][t] = s1;
          part[P_DK][w][t] = s2;
        }
      }
    }
  }
  if (pf) {                                // v (the next chunk-head's dO copies and states may be in flight)
    if (holds) wait_vmcnt<GV::rows_per_wave(NW) + NSTATE>();
    else wait_vmcnt<GV::rows_per_wave(NW)>();
  } else {
    wait_dma();                            // v
  }
  lds_barrier();
  if (a.l2norm && tid < 2 * C) {           // G's row dots, each summed once, in key-block order
    const int kind = tid >> 6, row = tid & (C - 1);
    float x = part[P_DQ + kind][0][row];
    for (int i = 1; i < NBD; ++i) x += part[P_DQ + kind][i][row];
    rowdot[kind][row] = x;
  }

  // ---- E: Y^T = dVn^T A (value block w), dv = beta Y staged in Vn's tile, v . Y row sums
  if (w < NBV) {
    const int c0 = 16 * w + 4 * j;        // this lane's 4 value features
    Frag<MT> fdv[2];
    Frag<MT> fy[4][2];
#pragma unroll
    for (int p = 0; p < 2; ++p) fdv[p] = frag_tr(tdV, VP, 32 * p, 16 * w, l);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (32 * p + 31 >= 16 * ti) fy[ti][p] = frag_tr(tA, CP, 32 * p, 16 * ti, l);
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      f4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int p = 0; p < 2; ++p)
        if (32 * p + 31 >= 16 * ti) mma(y, fdv[p], fy[ti][p]);
      const int t = 16 * ti + n;
      const float bt = cs.beta[t];
      *reinterpret_cast<bf16x4*>(tVn + t * VP + c0) = bf16x4{(bf16)(bt * y[0]), (bf16)(bt * y[1]), (bf16)(bt * y[2]),
                                                            (bf16)(bt * y[3])};
      const f4 v4 = load4(tO + t * VP + c0);
      const float s1 = across_groups_sum(((v4[0] * y[0] + v4[1] * y[1]) + v4[2] * y[2]) + v4[3] * y[3]);
      if (j == 0) part[P_VY][w][t] = s1;
    }
  }
  lds_barrier();

  // ---- G: the prologue's backward; dq and dk staged over q's and k's tiles
  f4 gq[4], gk[4];
  if (w < NBD) {
    const int d0 = 16 * w + 4 * j;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int t = 16 * ti + n;
      if (a.l2norm) {
        const float dq_dot = rowdot[0][t], dk_dot = rowdot[1][t];
        const float rqt = rq[t], rkt = rk[t];
        const f4 xq = load4(tq + t * KP + d0) * rqt, xk = load4(tk + t * KP + d0) * rkt;
        gq[ti] = (qs * rqt) * (dQt[ti] - xq * dq_dot);
        gk[ti] = rkt * (dKt[ti] - xk * dk_dot);
      } else {
        gq[ti] = qs * dQt[ti];
        gk[ti] = dKt[ti];
      }
    }
  }
  if (pf)                                  // v's array is free since E: the next chunk-head's Vn
    GV::template dma_rows_opaque<NW>(tO, (const MT*)a.Vn + nbhc * C * DV, DV, w, C, l);
  lds_barrier();                         // q and k tiles are read: they become the dq and dk staging
  if (pf) {                                // the next chunk-head's dVn into dVn's array (free since E), its g and beta
    GV::template dma_rows_opaque<NW>(L.R3, (const MT*)a.dVn + nbhc * C * DV, DV, w, C, l);
    const size_t o = ns_base + (size_t)(nt0 + l < nT ? nt0 + l : nT - 1) * H;
    gv = a.g[o];
    bv = a.beta[o];
  }
  if (w < NBD) {
    const int d0 = 16 * w + 4 * j;
#pragma unroll
    for (int ti = 0; ti < 4; ++ti) {
      const int t = 16 * ti + n;
      *reinterpret_cast<bf16x4*>(tq + t * KP + d0) =
          bf16x4{(bf16)gq[ti][0], (bf16)gq[ti][1], (bf16)gq[ti][2], (bf16)gq[ti][3]};
      *reinterpret_cast<bf16x4*>(tk + t * KP + d0) =
          bf16x4{(bf16)gk[ti][0], (bf16)gk[ti][1], (bf16)gk[ti][2], (bf16)gk[ti][3]};
    }
  }
  lds_barrier();
  // whole rows out, 16 bytes a lane, by waves 1..7 while wave 0 forms dbeta and dg (F): the partials F reads are not
  // written after E, so F runs off the path of the workgroup's last barrier
  if (w != 0) {
    constexpr int UK = DK / 8, UV = DV / 8, NTH = 64 * (NW - 1);
    const int wt = tid - 64;
    MT* dq = (MT*)a.dq + dqk_base + (size_t)t0 * dqk_pitch;
    MT* dk = (MT*)a.dk + dqk_base + (size_t)t0 * dqk_pitch;
    MT* dv = (MT*)a.dv + v_base + (size_t)t0 * v_pitch;
    for (int i = wt; i < nrows * UK; i += NTH) {
      const int row = i / UK, u = i - row * UK;
      const bf16x4 q0 = *reinterpret_cast<const bf16x4*>(tq + row * KP + 8 * u),   // rows are 8-byte aligned
                   q1 = *reinterpret_cast<const bf16x4*>(tq + row * KP + 8 * u + 4),
                   k0 = *reinterpret_cast<const bf16x4*>(tk + row * KP + 8 * u),
                   k1 = *reinterpret_cast<const bf16x4*>(tk + row * KP + 8 * u + 4);
      *reinterpret_cast<bf16x8*>(dq + row * dqk_pitch + 8 * u) = bf16x8{q0[0], q0[1], q0[2], q0[3], q1[0], q1[1], q1[2], q1[3]};
      *reinterpret_cast<bf16x8*>(dk + row * dqk_pitch + 8 * u) = bf16x8{k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
    }
    for (int i = wt; i < nrows * UV; i += NTH) {
      const int row = i / UV, u = i - row * UV;
      const bf16x4 lo = *reinterpret_cast<const bf16x4*>(tVn + row * VP + 8 * u),   // rows are 8-byte aligned
                   hi = *reinterpret_cast<const bf16x4*>(tVn + row * VP + 8 * u + 4);
      *reinterpret_cast<bf16x8*>(dv + row * v_pitch + 8 * u) = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  }

  // ---- F: dbeta and dg (wave 0, lane = chunk row), fixed-order sums of the partials
  if (w == 0) {
    const int r = l, t = t0 + r;
    auto sum = [&](int pi, int np) {
      float x = part[pi][0][r];
      for (int i = 1; i < np; ++i) x += part[pi][i][r];
      return x;
    };
    const float kx = sum(P_KX, NBD), qd = sum(P_QD, NBD), E = sum(P_E, NBD), r1 = sum(P_R1, 4), r2 = sum(P_R2, 4),
                vy = sum(P_VY, NBV);
    const float gmr = cs.gam[r], bt = cs.beta[r];
    const float db = fmaf(gmr, kx, vy) + r2;
    float dG = qd + bt * gmr * kx + (r1 - (colp[0][0][r] + colp[0][1][r])) + (bt * r2 - (colp[1][0][r] + colp[1][1][r]));
    if (r == C - 1) {
      float ss = partS[0];
      for (int i = 1; i < NBD; ++i) ss += partS[i];
      dG += cs.gam[C - 1] * ss;
    }
    // dg_t = sum_{s >= t} dG_s + sum_{r < t} E_r; the exclusive prefix by a shift, not incl - E: E on the last valid
    // row is O(1) while the earlier ones carry exp(G_last - G_r) and can be ~1e-9 of it
    const float rev = __shfl(dG, C - 1 - r, 64);
    const float suf = __shfl(wave_incl_scan(rev, l), C - 1 - r, 64);
    float Esh = wave_shift_up1(E);
    if (r == 0) Esh = 0.f;
    const float pre = wave_incl_scan(Esh, l);
    if (t < T) {
      a.dg[s_base + (size_t)t * H] = suf + pre;
      a.dbeta[s_base + (size_t)t * H] = db;
    }
  }
}

template <int DK, int DV>
__global__ void __launch_bounds__(512) chunk_bwd8_kernel(ChunkBwdArgs a) {
  CB8_LDS(DK, DV)
  cb8_stagger(a.stagger, blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
  Frag<float> s32[DV / 32], sD[DV / 32];
  float gv, bv;
  chunk_bwd8_body<DK, DV>(a, L, blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z), -1, true, L.R1,
                          L.R2, L.R7, s32, sD, gv, bv);
}

// Persistent form (DK = DV): workgroup i runs units i, i + stride, ... of the flat (chunk, head, batch row) order,
// each one's reads issued while the one before it computes, so only the first one's load phase is exposed.  The value
// tiles' arrays rotate: the next unit's dO goes into this one's dW array, its Vn into this one's dO/v array, and its
// dW array is this one's Vn/dv array.
template <int D>
__global__ void __launch_bounds__(512) chunk_bwd8xn_kernel(ChunkBwdArgs a, int units) {
  CB8_LDS(D, D)
  Frag<float> s32[D / 32], sD[D / 32];
  float gv, bv;
  bf16 *tO = L.R1, *tVn = L.R2, *sdW = L.R7;
  const int stride = gridDim.x;
  bool first = true;
  for (int u = blockIdx.x; u < units; u += stride) {
    const int next = u + stride < units ? u + stride : -1;
    chunk_bwd8_body<D, D>(a, L, u, next, first, tO, tVn, sdW, s32, sD, gv, bv);
    bf16* const t = sdW;
    sdW = tVn;
    tVn = tO;
    tO = t;
    first = false;
  }
}

// ---------------------------------------------------------------------------------------------------------------------
// decode: one token per head-row
// ---------------------------------------------------------------------------------------------------------------------
template <typename IT, int DK, int DV>
__global__ void __launch_bounds__(256) decode_kernel(DecodeArgs a) {
  constexpr int NCQ = DV / 4;       // column quads
  constexpr int RG = 256 / NCQ;     // row groups
  constexpr int RPG = DK / RG;      // rows per group
  static_assert(RG * NCQ == 256 && RPG * RG == DK, "decode tiling");
  __shared__ float sq[DK], sk[DK], sd[DV];
  __shared__ float red_k[RG][DV], red_q[RG][DV];
  __shared__ float sc[2];
  const int bh = blockIdx.x;
  const int l = lane_id(), w = wave_id();
  const size_t bhk = (size_t)(bh / a.H) * a.Hk + (bh % a.H) / (a.H / a.Hk);   // the key head of value head bh
  const IT* q = (const IT*)a.q + bhk * DK;
  const IT* k = (const IT*)a.k + bhk * DK;
  if (w == 0) {
    float qq = 0.f, kk = 0.f;
    for (int i = l; i < DK; i += 64) {
      const float x = to_f(q[i]), y = to_f(k[i]);
      qq = fmaf(x, x, qq);
      kk = fmaf(y, y, kk);
    }
    qq = across_groups_sum(group16_sum(qq));
    kk = across_groups_sum(group16_sum(kk));
    const float rq = a.l2norm ? 1.0f / sqrtf(qq + L2_EPS) : 1.f;
    const float rk = a.l2norm ? 1.0f / sqrtf(kk + L2_EPS) : 1.f;
    float qk = 0.f;
    for (int i = l; i < DK; i += 64) {
      const float x = to_f(q[i]) * rq * a.q_scale, y = to_f(k[i]) * rk;
      sq[i] = x;
      sk[i] = y;
      qk = fmaf(x, y, qk);
    }
    qk = across_groups_sum(group16_sum(qk));
    if (l == 0) sc[0] = qk;
  }
  __syncthreads();
  const int cq = threadIdx.x % NCQ, rg = threadIdx.x / NCQ;
  const float* sin = a.s_in + (size_t)bh * DK * DV;
  f4 st[RPG];
  f4 pk = {0.f, 0.f, 0.f, 0.f}, pq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < RPG; ++i) {
    const int row = rg * RPG + i;
    st[i] = *reinterpret_cast<const f4*>(sin + (size_t)row * DV + 4 * cq);
    pk += sk[row] * st[i];
    pq += sq[row] * st[i];
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    red_k[rg][4 * cq + e] = pk[e];
    red_q[rg][4 * cq + e] = pq[e];
  }
  __syncthreads();
  const float eg = expf(a.g[bh]);
  if (threadIdx.x < DV) {
    const int cc = threadIdx.x;
    float u = 0.f, oq = 0.f;
    for (int g2 = 0; g2 < RG; ++g2) {
      u += red_k[g2][cc];
      oq += red_q[g2][cc];
    }
    const float dd = a.beta[bh] * (to_f(((const IT*)a.v)[(size_t)bh * DV + cc]) - eg * u);
    sd[cc] = dd;
    ((IT*)a.o)[(size_t)bh * DV + cc] = from_f<IT>(fmaf(eg, oq, sc[0] * dd));
  }
  __syncthreads();
  const f4 d4 = *reinterpret_cast<const f4*>(sd + 4 * cq);
  float* so = a.s_out + (size_t)bh * DK * DV;
#pragma unroll
  for (int i = 0; i < RPG; ++i) {
    const int row = rg * RPG + i;
    *reinterpret_cast<f4*>(so + (size_t)row * DV + 4 * cq) = eg * st[i] + sk[row] * d4;
  }
}

// chunk_bwd8's launches (bf16 inputs): defined in gdr_chunk_bwd8.hip, a translation unit of their own that includes
// this file's device code and is compiled with LLVM's max-memory-clause scheduling strategy (chunk_bwd8 2.5% faster
// with it; applied to the whole library it slowed state_bwd by 4% and grew the spills of the float32 state kernels).
// xn: the persistent form (wgs workgroups over `units` chunk-heads); else one chunk-head a workgroup over `grid`.
void cb8_launch(const ChunkBwdArgs& a, int DK, int DV, bool xn, int wgs, int units, dim3 grid, hipStream_t st);

}  // namespace gdr

#ifndef GDR_CB8_ONLY   // gdr_chunk_bwd8.hip takes the device code above and nothing below
// The entry points fall into five parts by the kernels they instantiate; build.py compiles this file once per part
// (-DGDR_PART=1..5) in parallel, each object holding only its part's kernels.  Without GDR_PART every part is built.
#ifndef GDR_PART
#define GDR_PART 0
#endif
#define GDR_IN_PART(n) (GDR_PART == 0 || GDR_PART == (n))
// =====================================================================================================================
// C ABI
// =====================================================================================================================
using namespace gdr;

// y[b, t, hk, :] = sum of x[b, t, hk G + g, :] over the G = H / Hk value heads of a group, in head order with fp32
// accumulation: the key-head gradients of grouped heads.  One thread per 8 elements; rows_k = B T Hk.
template <typename T>
__global__ void __launch_bounds__(256) group_sum_kernel(const T* x, T* y, int64_t rows_k, int G, int D) {
  const int U = D / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows_k * U) return;
  const int64_t rk = i / U;
  const int u = (int)(i - rk * U);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < G; ++g) {
    const T* src = x + (rk * G + g) * D + 8 * u;
    const f4 lo = load4(src), hi = load4(src + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] += lo[e];
      acc[e + 4] += hi[e];
    }
  }
  T* dst = y + rk * D + 8 * u;
  store4<T>(dst, f4{acc[0], acc[1], acc[2], acc[3]});
  store4<T>(dst + 4, f4{acc[4], acc[5], acc[6], acc[7]});
}


// Key head widths: every multiple of 32 up to 256 (float32 operands; bf16 operands take 32, 64 and 128).
[[maybe_unused]] static bool key_width_ok(int64_t DK) { return DK >= 32 && DK <= 256 && DK % 32 == 0; }

[[maybe_unused]] static int check_common(const char* what, int64_t B, int64_t T, int64_t H, int64_t DK, int64_t DV,
                                         int dtype) {
  if (B < 1 || T < 1 || H < 1) return fail(MACAI_GDR_EINVAL, "%s: B, T, H must be >= 1 (got %lld, %lld, %lld)", what,
                                           (long long)B, (long long)T, (long long)H);
  if (!key_width_ok(DK))
    return fail(MACAI_GDR_EUNSUP, "%s: key head width must be a multiple of 32 in [32, 256] (got %lld)", what,
                (long long)DK);
  if (DK != 32 && DK != 64 && DK != 128 && dtype != MACAI_GDR_F32)
    return fail(MACAI_GDR_EUNSUP, "%s: key head width %lld takes float32 operands (bf16: 32, 64, 128; got dtype code %d)",
                what, (long long)DK, dtype);
  if (DV < 32 || DV % 32 != 0 || DV > 512)
    return fail(MACAI_GDR_EUNSUP, "%s: value head width must be a multiple of 32 in [32, 512] (got %lld)", what,
                (long long)DV);
  if (dtype != MACAI_GDR_F32 && dtype != MACAI_GDR_BF16)
    return fail(MACAI_GDR_EUNSUP, "%s: dtype code must be 0 (float32) or 1 (bfloat16), got %d", what, dtype);
  if (B * T * H * (DK > DV ? DK : DV) >= ((int64_t)1 << 31) * 4)
    return fail(MACAI_GDR_EINVAL, "%s: tensor too large", what);
  return MACAI_GDR_OK;
}

// Packed rows: `pack` (NULL = each batch row is one sequence) with its chunk count; sets NT.  The table's contents
// (built by the caller from cu_seqlens) are on the device and are not checked here.
[[maybe_unused]] static int pack_chunks(const char* what, const int32_t* pack, int64_t NT_packed, int64_t B, int64_t T,
                                        int64_t* NT) {
  if (!pack) {
    *NT = (T + C - 1) / C;
    return MACAI_GDR_OK;
  }
  if (NT_packed < 1 || NT_packed > T || NT_packed + B + 1 > ((int64_t)1 << 28))
    return fail(MACAI_GDR_EINVAL, "%s: packed rows need 1 <= chunks <= T (got %lld chunks, T = %lld)", what,
                (long long)NT_packed, (long long)T);
  if (((uintptr_t)pack & 3u) != 0) return fail(MACAI_GDR_EINVAL, "%s: the packed-row table must be 4-byte aligned", what);
  *NT = NT_packed;
  return MACAI_GDR_OK;
}

[[maybe_unused]] static int check_heads(const char* what, int64_t H, int64_t Hk) {
  if (Hk < 1 || H % Hk != 0)
    return fail(MACAI_GDR_EINVAL, "%s: key heads must divide value heads (got Hk = %lld, H = %lld)", what,
                (long long)Hk, (long long)H);
  return MACAI_GDR_OK;
}

#define DISPATCH_DK(DK, ...)                                   \
  switch (DK) {                                                \
    case 32: { constexpr int DKC = 32; __VA_ARGS__; } break;   \
    case 64: { constexpr int DKC = 64; __VA_ARGS__; } break;   \
    default: { constexpr int DKC = 128; __VA_ARGS__; } break;  \
  }
// float32 operands take every multiple of 32 up to 256 (the fp32 kernels stage key columns in passes or read chunk
// tiles from global memory where LDS is too small)
#define DISPATCH_DK_F32(DK, ...)                               \
  switch (DK) {                                                \
    case 32: { constexpr int DKC = 32; __VA_ARGS__; } break;   \
    case 64: { constexpr int DKC = 64; __VA_ARGS__; } break;   \
    case 96: { constexpr int DKC = 96; __VA_ARGS__; } break;   \
    case 160: { constexpr int DKC = 160; __VA_ARGS__; } break; \
    case 192: { constexpr int DKC = 192; __VA_ARGS__; } break; \
    case 224: { constexpr int DKC = 224; __VA_ARGS__; } break; \
    case 256: { constexpr int DKC = 256; __VA_ARGS__; } break; \
    default: { constexpr int DKC = 128; __VA_ARGS__; } break;  \
  }

// The current device's compute units (queried once per device), or 0 when the query fails.
[[maybe_unused]] static int device_cus() {
  static std::atomic<int> cus[64];
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 0) return 0;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

[[maybe_unused]] static int pick_waves(int64_t DV, int split, const char* what, int* nw_out, int* nslice_out) {
  // a workgroup holds NW in {1, 2, 4, 8} waves of 16 value columns; split = workgroups per head-row
  const int ncb = (int)(DV / 16);
  int nw;
  if (split <= 0) {
    nw = 8;
    while (ncb % nw) nw >>= 1;
  } else {
    if (ncb % split) return fail(MACAI_GDR_EINVAL, "%s: split %d does not divide the %d value-column slices", what, split, ncb);
    nw = ncb / split;
    if (nw != 1 && nw != 2 && nw != 4 && nw != 8)
      return fail(MACAI_GDR_EINVAL, "%s: split %d gives %d waves per workgroup (1, 2, 4 or 8 allowed)", what, split, nw);
  }
  *nw_out = nw;
  *nslice_out = ncb / nw;
  return MACAI_GDR_OK;
}

extern "C" {

#if GDR_IN_PART(1)
const char* macai_gdr_last_error(void) { return g_err; }

int macai_gdr_abi_version(void) { return MACAI_GDR_ABI_VERSION; }

int macai_gdr_prep(const void* q, const void* k, const void* v, const float* g, const float* beta, void* W, float* U,
                   void* Ke, float* GL, void* Qg, void* M, void* A, int64_t B, int64_t T, int64_t H, int64_t Hk,
                   int64_t DK, int64_t DV, int32_t dtype, int32_t use_l2norm, float q_scale, const int32_t* pack,
                   int64_t NT_packed, void* stream) {
  const char* what = "macai_gdr_prep";
  const bool mixed = dtype == MACAI_GDR_BF16_F32;   // bf16 q, k, v; float32 arithmetic and outputs
  if (mixed) dtype = MACAI_GDR_F32;
  int64_t NT = 0;
  int rc = check_common(what, pack ? 1 : B, T, H, DK, DV, dtype);
  if (!rc) rc = check_heads(what, H, Hk);
  if (!rc) rc = pack_chunks(what, pack, NT_packed, B, T, &NT);
  if (rc) return rc;
  if (!q || !k || !v || !g || !beta || !W || !U || !Ke || !GL || !Qg || !M)
    return fail(MACAI_GDR_EINVAL, "%s: null input or output pointer", what);
  const void* ps[] = {q, k, v, W, U, Ke, Qg, M, A};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  PrepArgs a{q, k, v, g, beta, W, U, Ke, GL, Qg, M, A, (int)B, (int)T, (int)H, (int)DV, (int)NT,
             use_l2norm, q_scale, (int)Hk, pack, 0};
  dim3 grid(a.NT, (unsigned)H, pack ? 1u : (unsigned)B);
  if (dtype != MACAI_GDR_F32) {            // prep8 (two workgroups a CU): stagger its first round when more follow
    const int cus = device_cus();
    if (cus > 0 && (int64_t)grid.x * grid.y * grid.z >= 4 * (int64_t)cus) a.stagger = 2 * cus;
  }
  hipStream_t st = (hipStream_t)stream;
  if (mixed) {
    DISPATCH_DK_F32(DK, hipLaunchKernelGGL((prep_kernel<bf16, float, DKC>), grid, dim3(512), 0, st, a));
  } else if (dtype == MACAI_GDR_F32) {
    DISPATCH_DK_F32(DK, hipLaunchKernelGGL((prep_kernel<float, float, DKC>), grid, dim3(512), 0, st, a));
  } else if (DV <= 128 || DV % 128 == 0) {
    DISPATCH_DK(DK, switch (DV) {
      case 32: hipLaunchKernelGGL((prep8_kernel<DKC, 32>), grid, dim3(512), 0, st, a); break;
      case 64: hipLaunchKernelGGL((prep8_kernel<DKC, 64>), grid, dim3(512), 0, st, a); break;
      case 96: hipLaunchKernelGGL((prep8_kernel<DKC, 96>), grid, dim3(512), 0, st, a); break;
      default: hipLaunchKernelGGL((prep8_kernel<DKC, 128>), grid, dim3(512), 0, st, a); break;
    })
  } else {
    DISPATCH_DK(DK, hipLaunchKernelGGL((prep_kernel<bf16, bf16, DKC>), grid, dim3(512), 0, st, a));
  }
  return launched(what);
}

#endif

#define DISPATCH_NW(NW, ...)                                  \
  switch (NW) {                                               \
    case 1: { constexpr int NWC = 1; __VA_ARGS__; } break;    \
    case 2: { constexpr int NWC = 2; __VA_ARGS__; } break;    \
    case 4: { constexpr int NWC = 4; __VA_ARGS__; } break;    \
    default: { constexpr int NWC = 8; __VA_ARGS__; } break;   \
  }

#if GDR_IN_PART(2)
int macai_gdr_state_fwd(const void* W, const float* U, const void* Ke, const float* GL, const void* Qg, const void* M,
                        const float* s0, void* o, float* sT, float* Sc, void* Vn, int64_t B, int64_t T, int64_t H,
                        int64_t DK, int64_t DV, int32_t dtype, int32_t flags, int32_t split, const int32_t* pack,
                        int64_t NT_packed, void* stream) {
  const char* what = "macai_gdr_state_fwd";
  const bool mixed = dtype == MACAI_GDR_BF16_F32;   // float32 operands, o in bf16
  if (mixed) dtype = MACAI_GDR_F32;
  int64_t NT = 0;
  int rc = check_common(what, pack ? 1 : B, T, H, DK, DV, dtype);
  if (!rc) rc = pack_chunks(what, pack, NT_packed, B, T, &NT);
  if (rc) return rc;
  const bool store = flags & MACAI_GDR_STORE_STATES, out = !(flags & MACAI_GDR_NO_OUTPUT);
  if ((flags & ~(MACAI_GDR_STORE_STATES | MACAI_GDR_NO_OUTPUT)) || (!out && !store))
    return fail(MACAI_GDR_EINVAL,
                "%s: flags must be 0 (output), STORE_STATES (output and states) or STORE_STATES | NO_OUTPUT (states)",
                what);
  if (!W || !U || !Ke || !GL) return fail(MACAI_GDR_EINVAL, "%s: null input pointer", what);
  if (out && (!Qg || !M || !o)) return fail(MACAI_GDR_EINVAL, "%s: the output needs Qg, M and o", what);
  if (store && (!Sc || !Vn)) return fail(MACAI_GDR_EINVAL, "%s: storing states needs Sc and Vn", what);
  const void* ps[] = {W, U, Ke, Qg, M, s0, sT, Sc, Vn};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  int nw, nslice;
  if ((rc = pick_waves(DV, split, what, &nw, &nslice))) return rc;
  StateFwdArgs a{W, U, Ke, GL, Qg, M, s0, o, out ? sT : nullptr, Sc, Vn, (int)B, (int)T, (int)H, (int)DV,
                 (int)NT, nslice, pack, mixed ? 1 : 0};
  const int HR = (int)(B * H);
  dim3 grid((unsigned)(8 * nslice * ((HR + 7) / 8)));
  dim3 block(64 * (nw + 1));   // nw compute waves and the loader wave
  hipStream_t st = (hipStream_t)stream;
#define LAUNCH_SF(MT, O, S) \
  DISPATCH_DK(DK, DISPATCH_NW(nw, hipLaunchKernelGGL((state_fwd_kernel<MT, DKC, NWC, O, S>), grid, block, 0, st, a)))
// float32: the key-split form (two waves a column slice) where it fits, else one wave a slice; the same bits
#define LAUNCH_SF32(O, S)                                                                                              \
  DISPATCH_DK_F32(DK, DISPATCH_NW(nw, {                                                                                \
    if constexpr (StateFwdLds<float, DKC, O, S, NWC, 2>::KS_OK)                                                        \
      hipLaunchKernelGGL((state_fwd_kernel<float, DKC, NWC, O, S, false, 2>), grid, dim3(64 * (2 * NWC + 1)), 0, st, a); \
    else                                                                                                               \
      hipLaunchKernelGGL((state_fwd_kernel<float, DKC, NWC, O, S>), grid, block, 0, st, a);                            \
  }))
#define LAUNCH_SO(S)                                                                                                  \
  {                                                                                                                   \
    const dim3 block2(64 * (2 * nw + 1));                                                                             \
    if (nw == 1) { DISPATCH_DK(DK, hipLaunchKernelGGL((state_out_kernel<DKC, 1, S>), grid, block2, 0, st, a)); }       \
    else { DISPATCH_DK(DK, hipLaunchKernelGGL((state_out_kernel<DKC, 2, S>), grid, block2, 0, st, a)); }              \
  }
  if (dtype == MACAI_GDR_F32) {
    if (out && store) { LAUNCH_SF32(true, true); }
    else if (out) { LAUNCH_SF32(true, false); }
    else { LAUNCH_SF32(false, true); }
  } else if (out && nw <= 2) {             // chain and output on separate waves
    if (store) { LAUNCH_SO(true); }
    else { LAUNCH_SO(false); }
  } else {
    if (out && store) { LAUNCH_SF(bf16, true, true); }
    else if (out) { LAUNCH_SF(bf16, true, false); }
    else { LAUNCH_SF(bf16, false, true); }
  }
#undef LAUNCH_SO
#undef LAUNCH_SF32
#undef LAUNCH_SF
  return launched(what);
}

#endif

#if GDR_IN_PART(3)
int macai_gdr_state_bwd(const void* Ke, const void* Qg, const void* W, const void* M, const float* GL,
                        const void* dO, const float* dsT, float* dSn, void* dVn, float* ds0, int64_t B, int64_t T,
                        int64_t H, int64_t DK, int64_t DV, int32_t dtype, int32_t split, const int32_t* pack,
                        int64_t NT_packed, void* stream) {
  const char* what = "macai_gdr_state_bwd";
  int64_t NT = 0;
  int rc = check_common(what, pack ? 1 : B, T, H, DK, DV, dtype);
  if (!rc) rc = pack_chunks(what, pack, NT_packed, B, T, &NT);
  if (rc) return rc;
  if (!Ke || !Qg || !W || !M || !GL || !dO || !dSn || !dVn || !ds0)
    return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  const void* ps[] = {Ke, Qg, W, M, dO, dsT, dSn, dVn, ds0};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  int nw, nslice;
  if ((rc = pick_waves(DV, split, what, &nw, &nslice))) return rc;
  StateBwdArgs a{Ke, Qg, W, M, GL, dO, dsT, dSn, dVn, ds0, (int)B, (int)T, (int)H, (int)DV, (int)NT, nslice, pack};
  const int HR = (int)(B * H);
  dim3 grid((unsigned)(8 * nslice * ((HR + 7) / 8)));
  dim3 block(64 * (nw + 1));   // nw compute waves and the loader wave
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MACAI_GDR_F32) {            // the key-split form where it fits (see macai_gdr_state_fwd)
    DISPATCH_DK_F32(DK, DISPATCH_NW(nw, {
      if constexpr (StateBwdLds<float, DKC, NWC, 2>::KS_OK)
        hipLaunchKernelGGL((state_bwd_kernel<float, DKC, NWC, 2>), grid, dim3(64 * (2 * NWC + 1)), 0, st, a);
      else
        hipLaunchKernelGGL((state_bwd_kernel<float, DKC, NWC>), grid, block, 0, st, a);
    }));
  } else {
    DISPATCH_DK(DK, DISPATCH_NW(nw, hipLaunchKernelGGL((state_bwd_kernel<bf16, DKC, NWC>), grid, block, 0, st, a)));
  }
  return launched(what);
}

int macai_gdr_state_pair(const void* W, const float* U, const void* Ke, const void* Qg, const void* M, const float* GL,
                         const float* s0, const void* dO, const float* dsT, float* Sc, void* Vn, float* dSn, void* dVn,
                         float* ds0, int64_t B, int64_t T, int64_t H, int64_t DK, int64_t DV, int32_t dtype,
                         int32_t split, const int32_t* pack, int64_t NT_packed, void* stream) {
  const char* what = "macai_gdr_state_pair";
  int64_t NT = 0;
  int rc = check_common(what, pack ? 1 : B, T, H, DK, DV, dtype);
  if (!rc) rc = pack_chunks(what, pack, NT_packed, B, T, &NT);
  if (rc) return rc;
  if (!W || !U || !Ke || !Qg || !M || !GL || !dO || !Sc || !Vn || !dSn || !dVn || !ds0)
    return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  const void* ps[] = {W, U, Ke, Qg, M, s0, dO, dsT, Sc, Vn, dSn, dVn, ds0};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  int nw, nslice;
  if ((rc = pick_waves(DV, split, what, &nw, &nslice))) return rc;
  const int NTi = (int)NT;
  StateFwdArgs af{W, U, Ke, GL, nullptr, nullptr, s0, nullptr, nullptr, Sc, Vn, (int)B, (int)T, (int)H, (int)DV, NTi,
                  nslice, pack};
  StateBwdArgs ab{Ke, Qg, W, M, GL, dO, dsT, dSn, dVn, ds0, (int)B, (int)T, (int)H, (int)DV, NTi, nslice, pack};
  const int HR = (int)(B * H);
  const int nfwd = 8 * nslice * ((HR + 7) / 8);   // a multiple of 8: the second pass keeps state_map's XCD layout
  dim3 grid((unsigned)(2 * nfwd));
  dim3 block(64 * (nw + 1));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MACAI_GDR_F32) {            // the key-split form where both passes take it
    DISPATCH_DK_F32(DK, DISPATCH_NW(nw, {
      if constexpr (StateFwdLds<float, DKC, false, true, NWC, 2>::KS_OK && StateBwdLds<float, DKC, NWC, 2>::KS_OK)
        hipLaunchKernelGGL((state_pair_kernel<float, DKC, NWC, 2>), grid, dim3(64 * (2 * NWC + 1)), 0, st, af, ab,
                           nfwd);
      else
        hipLaunchKernelGGL((state_pair_kernel<float, DKC, NWC>), grid, block, 0, st, af, ab, nfwd);
    }));
  } else {
    DISPATCH_DK(DK, DISPATCH_NW(nw, hipLaunchKernelGGL((state_pair_kernel<bf16, DKC, NWC>), grid, block, 0, st, af, ab,
                                                       nfwd)));
  }
  return launched(what);
}

#endif

#if GDR_IN_PART(4)
int macai_gdr_state_map(const void* W, const float* U, const void* Ke, const float* GL, float* maps, int64_t B,
                        int64_t T, int64_t H, int64_t DK, int64_t DV, int32_t dtype, int32_t split, const int32_t* pack,
                        int64_t NT_packed, void* stream) {
  const char* what = "macai_gdr_state_map";
  int64_t NT = 0;
  int rc = check_common(what, pack ? 1 : B, T, H, DK, DV, dtype);
  if (!rc) rc = pack_chunks(what, pack, NT_packed, B, T, &NT);
  if (rc) return rc;
  if (!W || !U || !Ke || !GL || !maps) return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  const void* ps[] = {W, U, Ke, maps};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  int nw, nslice;
  if ((rc = pick_waves(DK + DV, split, what, &nw, &nslice))) return rc;
  StateFwdArgs a{W, U, Ke, GL, nullptr, nullptr, nullptr, nullptr, maps, nullptr, nullptr, (int)B, (int)T, (int)H,
                 (int)DV, (int)NT, nslice, pack};
  const int HR = (int)(B * H);
  dim3 grid((unsigned)(8 * nslice * ((HR + 7) / 8)));
  dim3 block(64 * (nw + 1));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MACAI_GDR_F32) {
    DISPATCH_DK_F32(DK, DISPATCH_NW(nw, hipLaunchKernelGGL((state_fwd_kernel<float, DKC, NWC, false, false, true>), grid,
                                                           block, 0, st, a)));
  } else {
    DISPATCH_DK(DK, DISPATCH_NW(nw, hipLaunchKernelGGL((state_fwd_kernel<bf16, DKC, NWC, false, false, true>), grid,
                                                       block, 0, st, a)));
  }
  return launched(what);
}

int macai_gdr_state_scan(const float* maps, const float* s0, float* starts, int64_t rows, int64_t nseg, int64_t H,
                         int64_t DK, int64_t DV, void* stream) {
  const char* what = "macai_gdr_state_scan";
  if (rows < 1 || nseg < 1 || H < 1 || rows > 65535 || H > 65535)
    return fail(MACAI_GDR_EINVAL, "%s: rows, segments and heads must be >= 1 (and rows, heads <= 65535)", what);
  if (!key_width_ok(DK))
    return fail(MACAI_GDR_EUNSUP, "%s: key head width must be a multiple of 32 in [32, 256] (got %lld)", what,
                (long long)DK);
  if (DV < 16 || DV % 16 != 0 || DV > 512)
    return fail(MACAI_GDR_EUNSUP, "%s: value head width must be a multiple of 16 in [16, 512] (got %lld)", what,
                (long long)DV);
  if (!maps || !starts) return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  if (!aligned16(maps) || !aligned16(s0) || !aligned16(starts))
    return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  const dim3 grid((unsigned)(DV / 16), (unsigned)H, (unsigned)rows);
  hipStream_t st = (hipStream_t)stream;
  DISPATCH_DK_F32(DK, hipLaunchKernelGGL((state_scan_kernel<DKC>), grid, dim3(256), 0, st, maps, s0, starts, (int)nseg,
                                         (int)H, (int)DV));
  return launched(what);
}

#endif

#if GDR_IN_PART(5)
int macai_gdr_chunk_bwd(const void* q, const void* k, const void* v, const float* g, const float* beta, const void* dO,
                        const void* A, const float* Sc, const float* dSn, const void* Vn,
                        const void* dVn, void* dq, void* dk, void* dv, float* dg, float* dbeta, int64_t B, int64_t T,
                        int64_t H, int64_t Hk, int64_t DK, int64_t DV, int32_t dtype, int32_t use_l2norm, float q_scale,
                        const int32_t* pack, int64_t NT_packed, void* stream) {
  const char* what = "macai_gdr_chunk_bwd";
  const bool mixed = dtype == MACAI_GDR_BF16_F32;   // bf16 q, k, v and dq, dk, dv; float32 dO and operands
  if (mixed) dtype = MACAI_GDR_F32;
  int64_t NT = 0;
  int rc = check_common(what, pack ? 1 : B, T, H, DK, DV, dtype);
  if (!rc) rc = check_heads(what, H, Hk);
  if (!rc && mixed && Hk != H)
    return fail(MACAI_GDR_EUNSUP, "%s: bf16 tensors with float32 operands take Hk == H (got Hk = %lld, H = %lld)", what,
                (long long)Hk, (long long)H);
  if (!rc) rc = pack_chunks(what, pack, NT_packed, B, T, &NT);
  if (rc) return rc;
  if (dtype != MACAI_GDR_F32 && DV != 32 && DV != 64 && DV != 96 && DV != 128)
    return fail(MACAI_GDR_EUNSUP, "%s: the bf16 backward takes value head widths 32, 64, 96 or 128 (got %lld)", what,
                (long long)DV);
  if (DV > 256)
    return fail(MACAI_GDR_EUNSUP, "%s: the backward takes value head widths up to 256 (got %lld)", what, (long long)DV);
  if (!q || !k || !v || !g || !beta || !dO || !A || !Sc || !dSn || !Vn || !dVn || !dq || !dk || !dv || !dg ||
      !dbeta)
    return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  const void* ps[] = {q, k, v, dO, A, Sc, dSn, Vn, dVn};
  for (const void* p : ps)
    if (!aligned16(p)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  ChunkBwdArgs a{q, k, v, g, beta, dO, A, Sc, dSn, Vn, dVn, dq, dk, dv, dg, dbeta, (int)B, (int)T, (int)H,
                 (int)DV, (int)NT, use_l2norm, q_scale, (int)Hk, pack, 0};
  dim3 grid(a.NT, (unsigned)H, pack ? 1u : (unsigned)B);
  const int64_t units = (int64_t)grid.x * grid.y * grid.z;
  bool xn = false;                         // persistent workgroups, one a CU (DK = DV, more chunk-heads than CUs)
  if (dtype != MACAI_GDR_F32) {            // chunk_bwd8 (one workgroup a CU): stagger its first round when more follow
    const int cus = device_cus();
    xn = DK == DV && cus > 0 && units > cus && units < (int64_t)1 << 30;
    if (!xn && cus > 0 && units >= 2 * (int64_t)cus) a.stagger = cus;   // (the persistent form measured slower with it)
  }
  hipStream_t st = (hipStream_t)stream;
// (the key widths 32, 64, 128 and 256 with value widths up to 128 have their value width as a template constant; every
// other width pair takes it at run time, DV = 0 below)
#define LAUNCH_CB(MT)                                                                                               \
  DISPATCH_DK_F32(DK, if constexpr (DKC != 32 && DKC != 64 && DKC != 128 && DKC != 256) {                             \
    hipLaunchKernelGGL((chunk_bwd_kernel<MT, DKC, 0>), grid, dim3(64 * cb32_waves(DKC)), 0, st, a);                 \
  } else switch (DV) {                                                                                                 \
    case 32: hipLaunchKernelGGL((chunk_bwd_kernel<MT, DKC, 32>), grid, dim3(64 * cb32_waves(DKC)), 0, st, a); break; \
    case 64: hipLaunchKernelGGL((chunk_bwd_kernel<MT, DKC, 64>), grid, dim3(64 * cb32_waves(DKC)), 0, st, a); break; \
    case 96: hipLaunchKernelGGL((chunk_bwd_kernel<MT, DKC, 96>), grid, dim3(64 * cb32_waves(DKC)), 0, st, a); break; \
    case 128: hipLaunchKernelGGL((chunk_bwd_kernel<MT, DKC, 128>), grid, dim3(64 * cb32_waves(DKC)), 0, st, a); break; \
    default: hipLaunchKernelGGL((chunk_bwd_kernel<MT, DKC, 0>), grid, dim3(64 * cb32_waves(DKC)), 0, st, a); break; \
  })
  if (mixed) {                             // the value width a template constant at 128 only (fewer instances)
    DISPATCH_DK_F32(DK, if (DV == 128 && (DKC == 32 || DKC == 64 || DKC == 128 || DKC == 256)) {
      hipLaunchKernelGGL((chunk_bwd_kernel<float, DKC, 128, bf16>), grid, dim3(64 * cb32_waves(DKC)), 0, st, a);
    } else {
      hipLaunchKernelGGL((chunk_bwd_kernel<float, DKC, 0, bf16>), grid, dim3(64 * cb32_waves(DKC)), 0, st, a);
    })
  } else if (dtype == MACAI_GDR_F32) {
    LAUNCH_CB(float);
  } else {
    const int cus = xn ? device_cus() : 0;
    cb8_launch(a, (int)DK, (int)DV, xn, (int)(xn && units > cus ? cus : units), (int)units, grid, st);
  }
#undef LAUNCH_CB
  return launched(what);
}

#endif

#if GDR_IN_PART(1)
int macai_gdr_decode(const void* q, const void* k, const void* v, const float* g, const float* beta,
                     const float* s_in, void* o, float* s_out, int64_t B, int64_t H, int64_t Hk, int64_t DK,
                     int64_t DV, int32_t dtype, int32_t use_l2norm, float q_scale, void* stream) {
  const char* what = "macai_gdr_decode";
  if (B < 1 || H < 1) return fail(MACAI_GDR_EINVAL, "%s: B and H must be >= 1", what);
  if (int rc = check_heads(what, H, Hk)) return rc;
  if (!((DK == 128 && DV == 128) || (DK == 64 && DV == 64) || (DK == 128 && DV == 64) || (DK == 64 && DV == 128)))
    return fail(MACAI_GDR_EUNSUP, "%s: head widths (DK, DV) must be 64 or 128 each (got %lld, %lld)", what,
                (long long)DK, (long long)DV);
  if (dtype != MACAI_GDR_F32 && dtype != MACAI_GDR_BF16)
    return fail(MACAI_GDR_EUNSUP, "%s: dtype code must be 0 or 1, got %d", what, dtype);
  if (!q || !k || !v || !g || !beta || !s_in || !o || !s_out) return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  if (!aligned16(s_in) || !aligned16(s_out)) return fail(MACAI_GDR_EINVAL, "%s: states must be 16-byte aligned", what);
  DecodeArgs a{q, k, v, g, beta, s_in, o, s_out, (int)B, (int)H, use_l2norm, q_scale, (int)Hk};
  dim3 grid((unsigned)(B * H));
  hipStream_t st = (hipStream_t)stream;
#define LAUNCH_DEC(IT)                                                                                           \
  if (DK == 128 && DV == 128) hipLaunchKernelGGL((decode_kernel<IT, 128, 128>), grid, dim3(256), 0, st, a);    \
  else if (DK == 64 && DV == 64) hipLaunchKernelGGL((decode_kernel<IT, 64, 64>), grid, dim3(256), 0, st, a);   \
  else if (DK == 128) hipLaunchKernelGGL((decode_kernel<IT, 128, 64>), grid, dim3(256), 0, st, a);             \
  else hipLaunchKernelGGL((decode_kernel<IT, 64, 128>), grid, dim3(256), 0, st, a);
  if (dtype == MACAI_GDR_F32) {
    LAUNCH_DEC(float)
  } else {
    LAUNCH_DEC(bf16)
  }
#undef LAUNCH_DEC
  return launched(what);
}

int macai_gdr_group_sum(const void* x, void* y, int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D, int32_t dtype,
                        void* stream) {
  const char* what = "macai_gdr_group_sum";
  if (B < 1 || T < 1 || H < 1) return fail(MACAI_GDR_EINVAL, "%s: B, T, H must be >= 1", what);
  if (int rc = check_heads(what, H, Hk)) return rc;
  if (D < 8 || D % 8 != 0) return fail(MACAI_GDR_EUNSUP, "%s: row width must be a multiple of 8 (got %lld)", what,
                                       (long long)D);
  if (dtype != MACAI_GDR_F32 && dtype != MACAI_GDR_BF16)
    return fail(MACAI_GDR_EUNSUP, "%s: dtype code must be 0 or 1, got %d", what, dtype);
  if (!x || !y) return fail(MACAI_GDR_EINVAL, "%s: null pointer", what);
  if (!aligned16(x) || !aligned16(y)) return fail(MACAI_GDR_EINVAL, "%s: pointers must be 16-byte aligned", what);
  if (B * T * H * D >= ((int64_t)1 << 31) * 4) return fail(MACAI_GDR_EINVAL, "%s: tensor too large", what);
  const int64_t rows_k = B * T * Hk, units = rows_k * (D / 8);
  const dim3 grid((unsigned)((units + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  if (dtype == MACAI_GDR_F32)
    hipLaunchKernelGGL((group_sum_kernel<float>), grid, dim3(256), 0, st, (const float*)x, (float*)y, rows_k,
                       (int)(H / Hk), (int)D);
  else
    hipLaunchKernelGGL((group_sum_kernel<bf16>), grid, dim3(256), 0, st, (const bf16*)x, (bf16*)y, rows_k,
                       (int)(H / Hk), (int)D);
  return launched(what);
}

#endif

}  // extern "C"
#endif  // GDR_CB8_ONLY

/* macai_gdr.h -- C ABI of the MI355X (gfx950) chunked gated delta rule.
 *
 * The drop-in boundary of the reference's hot path (macai.gated_delta).  The reference launches four Metal kernels per
 * training step through torch.mps compiled shaders, `lib.<kernel>(*tensors, *uint_scalars, threads=..., group_size=...)`
 * (reference src/macai/gated_delta/op.py:71, 159, 217, 234, 241-242), plus the query/key prologue (_norm.py:97, 113).
 * Each entry point below replaces one of those passes; the caller (PyTorch, through ctypes) owns every buffer,
 * including the per-chunk scratch, and passes raw device pointers, sizes and the HIP stream (hipStream_t as void*).
 * The library allocates nothing and keeps no state between calls; every call only enqueues work on `stream`.
 *
 * Layouts (all contiguous, row-major); H counts value heads, Hk key heads (H a multiple of Hk; value head h uses key
 * head h / (H / Hk), the grouped-value layout of Qwen3.5 / Qwen3-Next without repeating q and k first):
 *   q, k        [B, T, Hk, DK]  dtype (float32 or bfloat16; raw, or already normalised when use_l2norm = 0)
 *   dq, dk      [B, T, H, DK]   dtype, per value head (macai_gdr_group_sum folds a group into [B, T, Hk, DK])
 *   v, o, dO    [B, T, H, DV]   dtype
 *   g, beta     [B, T, H]       float32   (g = log decay <= 0)
 *   states      [B, H, DK, DV]  float32   (initial_state, final state, their gradients)
 *   per chunk   NT = ceil(T / 64) chunks of 64 tokens, padding rows zero (written by macai_gdr_prep), all row-major
 *               with the chunk's tokens as rows (the kernels read the transposes they need from LDS):
 *     W, Qg, Ke   [B, H, NT, 64, DK] dtype   W = A diag(beta gamma) K^;  diag(gamma) Q^;  diag(e) K^
 *     U           [B, H, NT, 64, DV] float32  U = A diag(beta) V
 *     M           [B, H, NT, 64, 64] dtype   M = (Q^ K^T) * exp(G_i - G_j) (lower with the diagonal)
 *     A           [B, H, NT, 64, 64] dtype   A = (I + L)^-1 (solved in fp32)
 *     GL          [B, H, NT]         float32 exp(G_last) of each chunk
 *     Sc          [B, H, NT, DK, DV] float32 state entering each chunk
 *     dSn         [B, H, NT, DK, DV] float32 dLoss/dS_{c+1}
 *     Vn, dVn     [B, H, NT, 64, DV] dtype   per-token corrections U - W S_c and their gradient
 *   G_r = sum_{s<=r} g_s inside the chunk, gamma = exp(G), e = exp(G_last - G), q^ / k^ the prologue's outputs.
 * With use_l2norm = 1 the kernels apply the reference prologue (_norm.py:1-10) themselves: q^ = q * rsqrt(|q|^2 + 1e-6)
 * * q_scale, k^ = k * rsqrt(|k|^2 + 1e-6), and the backward returns gradients w.r.t. the raw q and k.
 * Supported widths: DK in {32, 64, 128}, and with float32 operands every multiple of 32 up to 256; DV a multiple of
 * 32 up to 512 (the backward: up to 128 with bf16 operands, up to 256 with float32).
 * Pointers must be 16-byte aligned.
 *
 * Packed rows (several sequences in one row, transformers' cu_seqlens): pass `pack`, a device int32 table, and its
 * chunk count NT (`pack` = NULL: every batch row is one sequence and NT = ceil(T / 64)).  Sequence n spans tokens
 * cu[n] .. cu[n+1] of a single row and is chunked on its own (ceil(len / 64) chunks, the last one partial); the
 * state restarts at each sequence.  Then B counts sequences: token tensors are [1, T, H, D], per-chunk tensors
 * [1, H, NT, ...], states [B, H, DK, DV].  Table layout ([2 NT + B + 1] int32): each chunk's first token, then the
 * end of each chunk's sequence, then each sequence's first chunk (B + 1 entries, the last = NT).  The library does
 * not read the table on the host; a wrong table is undefined behaviour.
 *
 * Return value: 0 on success, else an error code below; macai_gdr_last_error() describes the last failure of the
 * calling thread.  Argument checks run before any launch, so they are testable without a GPU.
 */
#ifndef MACAI_GDR_H
#define MACAI_GDR_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MACAI_GDR_ABI_VERSION 13

/* dtype codes (the rule takes F32 and BF16; the producers also F16) */
#define MACAI_GDR_F32 0
#define MACAI_GDR_BF16 1
#define MACAI_GDR_F16 2
/* bf16 tensors in memory with float32 arithmetic and float32 per-chunk operands: taken by macai_gdr_prep (q, k, v
 * bf16), macai_gdr_state_fwd (o bf16) and macai_gdr_chunk_bwd (q, k, v, dq, dk, dv bf16, dO float32, Hk == H).  The
 * same bits as the float32 call on the exactly upcast inputs with its bf16 results rounded to nearest even, without
 * the casts' passes (the reference upcasts bf16 inputs and computes in float32, op.py:276-297). */
#define MACAI_GDR_BF16_F32 3

/* error codes */
#define MACAI_GDR_OK 0
#define MACAI_GDR_EINVAL 1  /* bad shape, null or misaligned pointer, inconsistent flags */
#define MACAI_GDR_EUNSUP 2  /* unsupported head width or dtype */
#define MACAI_GDR_ELAUNCH 3 /* HIP launch error (hipGetLastError) */

/* state-pass flags (the reference's gdc_fwd flags, _chunked.py:335-338) */
#define MACAI_GDR_STORE_STATES 1 /* store Sc and Vn for the backward (with or without the output) */
#define MACAI_GDR_NO_OUTPUT 8    /* write neither o nor the final state */

const char* macai_gdr_last_error(void);
int macai_gdr_abi_version(void);

/* Per-chunk preparation (north star (1), the intra-chunk kernel), every chunk independent: G, L, A = (I + L)^-1 and
 * W, U, Ke, GL, Qg, M; A itself when A is non-NULL (the backward's per-chunk pass needs it).  Replaces
 * `lib.gdc_prep(q, k, g, beta, gc, a, m, kg, T, H, ...)` (reference op.py:63-72; kernel _chunked.py:220-313) and the
 * fused prologue l2n_fwd (_norm.py:97). */
int macai_gdr_prep(const void* q, const void* k, const void* v, const float* g, const float* beta, void* W, float* U,
                   void* Ke, float* GL, void* Qg, void* M, void* A, int64_t B, int64_t T, int64_t H, int64_t Hk,
                   int64_t DK, int64_t DV, int32_t dtype, int32_t use_l2norm, float q_scale, const int32_t* pack,
                   int64_t NT, void* stream);

/* The sequential state pass (north star (2) + (3)): S <- exp(G_last) S + K^T diag(e) (U - W S) over the chunks from
 * s0 (NULL = zeros).  flags = 0: the output O = diag(gamma) Q S + M Vn to o (dtype) and the final state to sT when
 * sT != NULL (needs Qg, M); flags = STORE_STATES | NO_OUTPUT: Sc and Vn for the backward (the backward's recompute);
 * flags = STORE_STATES: both (a training forward that keeps the states for its backward).  split = workgroups per
 * head-row's value columns (DV / 16 / split must be 1, 2, 4 or 8; 0 = automatic).  Replaces `lib.gdc_fwd(q, k, v,
 * beta, s0, gc, a, m, o, sT, sc, vn, xu, ckpt, T, H, DV, flags, ...)` (reference op.py:159, 217; kernel
 * _chunked.py:315-659). */
int macai_gdr_state_fwd(const void* W, const float* U, const void* Ke, const float* GL, const void* Qg, const void* M,
                        const float* s0, void* o, float* sT, float* Sc, void* Vn, int64_t B, int64_t T, int64_t H,
                        int64_t DK, int64_t DV, int32_t dtype, int32_t flags, int32_t split, const int32_t* pack,
                        int64_t NT, void* stream);

/* The reverse state pass (north star (4)): from dS_NT = dsT (NULL = zeros) back over the chunks, dVn = M^T dO +
 * diag(e) K dS, dS <- exp(G_last) dS + (diag(gamma) Q)^T dO - W^T dVn; stores dSn (= dS_{c+1}) and dVn per chunk and
 * writes ds0 = dLoss/d initial_state.  Replaces `lib.gdc_bwd_state(q, k, beta, do, dsT, gc, a, m, dsn, dvn, ds0, T,
 * H, DV, ...)` (reference op.py:234; kernel _chunked.py:661-903). */
int macai_gdr_state_bwd(const void* Ke, const void* Qg, const void* W, const void* M, const float* GL,
                        const void* dO, const float* dsT, float* dSn, void* dVn, float* ds0, int64_t B, int64_t T,
                        int64_t H, int64_t DK, int64_t DV, int32_t dtype, int32_t split, const int32_t* pack,
                        int64_t NT, void* stream);

/* The backward's recompute pass (macai_gdr_state_fwd with STORE_STATES | NO_OUTPUT: Sc, Vn) and its reverse pass
 * (macai_gdr_state_bwd: dSn, dVn, ds0) in one launch, side by side on the CUs: they read prep's outputs, not each
 * other's.  Each is a sequential chain of chunks whose speed hardly depends on its share of the CUs, so running them
 * at once (with `split` chosen for half the chip) nearly hides one.  Replaces the reference's two launches
 * `lib.gdc_fwd(..., flags 1 | 8)` and `lib.gdc_bwd_state(...)` (op.py:217, 234). */
int macai_gdr_state_pair(const void* W, const float* U, const void* Ke, const void* Qg, const void* M, const float* GL,
                         const float* s0, const void* dO, const float* dsT, float* Sc, void* Vn, float* dSn, void* dVn,
                         float* ds0, int64_t B, int64_t T, int64_t H, int64_t DK, int64_t DV, int32_t dtype,
                         int32_t split, const int32_t* pack, int64_t NT, void* stream);

/* Sequence parallelism for long rows (no counterpart in the reference, whose state pass walks a row's chunks in one
 * chain): the state pass is affine in its starting state, S_end = A S_0 + B, so a row split into segments (packed-row
 * sequences of one row) can run its segments side by side.  macai_gdr_state_map writes each sequence's map
 * [A | B] (float32 [B, H, DK, DK + DV]: A = the pass from the identity with U taken as zero, B = the pass from zero),
 * reading what macai_gdr_state_fwd reads for its states (W, U, Ke, GL).  macai_gdr_state_scan composes them in order
 * along each row: starts[r, s] = the state entering segment s of row r, starts[r, 0] = s0[r] (NULL = zeros),
 * starts[r, s + 1] = A_{r,s} starts[r, s] + B_{r,s} (maps and starts [rows * nseg, H, ...], s0 [rows, H, DK, DV]).
 * macai_gdr_state_fwd over the segments from `starts` then gives the row's output and, for its last segment, the final
 * state.  split as in macai_gdr_state_fwd over the DK + DV columns. */
int macai_gdr_state_map(const void* W, const float* U, const void* Ke, const float* GL, float* maps, int64_t B,
                        int64_t T, int64_t H, int64_t DK, int64_t DV, int32_t dtype, int32_t split, const int32_t* pack,
                        int64_t NT, void* stream);
int macai_gdr_state_scan(const float* maps, const float* s0, float* starts, int64_t rows, int64_t nseg, int64_t H,
                         int64_t DK, int64_t DV, void* stream);

/* The per-chunk backward (north star (4)): dq, dk (w.r.t. the raw inputs when use_l2norm; per value head, [B, T, H,
 * DK]), dv in dtype; dg, dbeta in float32; one writer per element (bitwise deterministic).  Replaces
 * `lib.gdc_bwd_chunk(q, k, beta, do, gc, a, kg, m, sc, dsn, vn, xu, dvn, dq, dk, dv, dg, dbeta, T, H, DV, ...)`
 * (reference op.py:241-242; kernel _chunked.py:905-1177) and the prologue's backward l2n_bwd (_norm.py:113). */
int macai_gdr_chunk_bwd(const void* q, const void* k, const void* v, const float* g, const float* beta, const void* dO,
                        const void* A, const float* Sc, const float* dSn, const void* Vn,
                        const void* dVn, void* dq, void* dk, void* dv, float* dg, float* dbeta, int64_t B, int64_t T,
                        int64_t H, int64_t Hk, int64_t DK, int64_t DV, int32_t dtype, int32_t use_l2norm,
                        float q_scale, const int32_t* pack, int64_t NT, void* stream);

/* The inference forward in one call: macai_gdr_prep (without A) then macai_gdr_state_fwd with the output (flags 0),
 * the per-chunk operands W, U, Ke, GL, Qg, M carved from `workspace` (256-byte aligned, at least
 * macai_gdr_forward_workspace(...) bytes; its contents on entry do not matter).  o [B, T, H, DV] in dtype and sT (or
 * NULL) as macai_gdr_state_fwd writes them; split 0 = automatic (the smallest split giving every CU a workgroup with
 * at most four column waves a workgroup).  The same kernels and bits as the two calls.  Replaces the drop-in's
 * no-grad forward, the reference's `_prep` + `lib.gdc_fwd(..., flags 0)` (op.py:63-72, 159). */
int macai_gdr_forward(const void* q, const void* k, const void* v, const float* g, const float* beta,
                      const float* s0, void* o, float* sT, void* workspace, int64_t workspace_bytes, int64_t B,
                      int64_t T, int64_t H, int64_t Hk, int64_t DK, int64_t DV, int32_t dtype, int32_t use_l2norm,
                      float q_scale, int32_t split, const int32_t* pack, int64_t NT, void* stream);

/* Bytes of macai_gdr_forward's workspace for a shape (NT = the packed-row chunk count, or 0 for B rows of T). */
int64_t macai_gdr_forward_workspace(int64_t B, int64_t T, int64_t H, int64_t DK, int64_t DV, int32_t dtype,
                                    int64_t NT);

/* macai_gdr_forward without a workspace argument and without allocating: no counterpart in the reference; for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The per-chunk operands live in a fixed device array of MACAI_GDR_NOALLOC_SCRATCH_BYTES, one per device,
 * reserved by the first call on that device (the array sits alone in its code object, which the runtime loads on that
 * call's address lookup, not when the library loads) and held for the process's lifetime; a shape whose operands
 * (macai_gdr_forward_workspace) exceed it is refused with EINVAL before any launch.  Calls on one device share that array: calls that overlap on one device (different
 * streams, or threads) race and must be serialised by the caller.  Same arguments and bits as macai_gdr_forward.
 * Under graph capture: make one call on the device before capturing -- the first call there looks up the array's
 * address (hipGetSymbolAddress, not a stream operation); the captured launches then replay with the same bits. */
#define MACAI_GDR_NOALLOC_SCRATCH_BYTES ((int64_t)128 << 20)
int macai_gdr_forward_noalloc(const void* q, const void* k, const void* v, const float* g, const float* beta,
                              const float* s0, void* o, float* sT, int64_t B, int64_t T, int64_t H, int64_t Hk,
                              int64_t DK, int64_t DV, int32_t dtype, int32_t use_l2norm, float q_scale, int32_t split,
                              const int32_t* pack, int64_t NT, void* stream);

/* One recurrent step per sequence (T = 1): q, k [B, 1, Hk, DK], v [B, 1, H, DV] dtype; g, beta [B, 1, H] float32;
 * s_in, s_out [B, H, DK, DV] float32 (s_out may equal s_in).  S' = e^g S + k beta (v - e^g S^T k)^T, o = S'^T q.  The
 * math of the reference's recurrence (op.py:308-313) and of transformers' torch_recurrent_gated_delta_rule
 * (modeling_qwen3_5.py:330-380), which the reference leaves unpatched (patch.py:27-29).  (DK, DV) in {64, 128}^2. */
int macai_gdr_decode(const void* q, const void* k, const void* v, const float* g, const float* beta,
                     const float* s_in, void* o, float* s_out, int64_t B, int64_t H, int64_t Hk, int64_t DK,
                     int64_t DV, int32_t dtype, int32_t use_l2norm, float q_scale, void* stream);

/* Key-head gradients of grouped heads: y [B, T, Hk, D] = the sum over each group's H / Hk value heads of x [B, T, H,
 * D] (fp32 accumulation in head order, dtype in and out; D a multiple of 8).  Replaces the backward of the
 * q.repeat_interleave(H / Hk, dim=2) / k.repeat_interleave(...) that precede the rule in the model
 * (transformers modeling_qwen3_5.py:500-502; reference layer/_qwen3_5.py:155-157), which the grouped layout removes. */
int macai_gdr_group_sum(const void* x, void* y, int64_t B, int64_t T, int64_t H, int64_t Hk, int64_t D, int32_t dtype,
                        void* stream);

/* ---- the producers of the rule's inputs (the linear-attention layer's convolution path and gates) ----
 *
 * The convolution path: x [B, T, C] (the input projection's output, C = 2 KD + VD), w [C, 4] float32 taps;
 * u[t, c] = sum_j w[c, j] x[t - 3 + j, c] (zero before the start, float32), y = u sigmoid(u) rounded once; q, k =
 * the first two KD-channel blocks as [B, T, KD / DK * REP, DK] in x's dtype, each key head written REP times
 * (REP = 1: key heads only, the layout the rule reads natively; REP = value heads / key heads: transformers' repeat),
 * v = the last VD channels as [B, T, VD / DV, DV] in vdtype.  dtype, vdtype: F32, BF16 or F16.  Replaces the
 * reference's conv_fwd kernel launch (layer/_conv.py:191-193; kernel 1-24, 47-82). */
int macai_gdr_conv_fwd(const void* x, const float* w, void* q, void* k, void* v, int64_t B, int64_t T, int64_t C,
                       int64_t KD, int64_t DK, int64_t REP, int64_t DV, int32_t dtype, int32_t vdtype, void* stream);

/* Its backward: dx [B, T, C] in x's dtype from dq, dk (summed over the REP copies) and dv, u recomputed from x; with
 * dwp (float32 [macai_gdr_conv_partials(B, T, C)] scratch) and dw (float32 [C, 4]) non-NULL, also the taps'
 * gradient (partials a tile of time steps, then a fixed-order sum: deterministic).  Replaces conv_bwd and dw_sum
 * (layer/_conv.py:221-231; kernel 84-130, 150-159). */
int macai_gdr_conv_bwd(const void* x, const float* w, const void* dq, const void* dk, const void* dv, void* dx,
                       float* dwp, float* dw, int64_t B, int64_t T, int64_t C, int64_t KD, int64_t DK, int64_t REP,
                       int64_t DV, int32_t dtype, int32_t vdtype, void* stream);

/* float32 elements of the conv backward's dw partials for a shape. */
int64_t macai_gdr_conv_partials(int64_t B, int64_t T, int64_t C);

/* The gates: beta = sigmoid(b), g = -exp(A_log) softplus(a + dt_bias) (PyTorch's softplus threshold 20), both
 * float32 [n] from b, a [n] in dtype (n = rows x H, head h = i % H) and A_log, dt_bias [H] float32.  Replaces the
 * reference's gates_fwd (layer/_gates.py:91-93; kernel 22-39). */
int macai_gdr_gates_fwd(const void* b, const void* a, const float* A_log, const float* dt_bias, float* beta, float* g,
                        int64_t n, int64_t H, int32_t dtype, void* stream);

/* Their backward: db = dbeta beta (1 - beta), da = dg (-exp(A_log)) sigmoid(a + dt_bias) (1 above the threshold), in
 * dtype; with dA_log and ddt_bias (float32 [H]) non-NULL also the sums over the rows of dg g and dg (-exp(A_log))
 * sigmoid(a + dt_bias) (one workgroup a head, fixed order).  Replaces gates_bwd and the reference's PyTorch
 * reductions for trained gates (layer/_gates.py:100-118; kernel 41-55). */
int macai_gdr_gates_bwd(const void* b, const void* a, const float* A_log, const float* dt_bias, const float* dbeta,
                        const float* dg, void* db, void* da, float* dA_log, float* ddt_bias, int64_t n, int64_t H,
                        int32_t dtype, void* stream);

/* ---- measurement ---- */

/* A streaming probe of the device's memory ceilings (no counterpart in the reference; bench.py --ceilings): mode 0
 * reads `bytes` from src (dst: a 16-byte sink, written by practically no lane), 1 writes them to dst, 2 copies src to
 * dst; 16-byte units, grid-stride over `blocks` workgroups of 256 lanes. */
int macai_gdr_probe_stream(int32_t mode, const void* src, void* dst, int64_t bytes, int32_t blocks, void* stream);

/* A probe of the matrix cores' throughput (no counterpart in the reference; the MFMA half of its bench/hw_ceilings.py,
 * bench.py --ceilings): `blocks` workgroups of 4 waves, each wave `iters` rounds of 8 independent chains of one MFMA,
 * mode 0 v_mfma_f32_16x16x32_bf16 (the bf16 kernels' shape), 1 v_mfma_f32_16x16x4_f32 (the float32 kernels'), 2
 * v_mfma_f32_32x32x16_bf16; out: blocks x 256 floats (the accumulators' sums).  macai_gdr_probe_mfma_flops gives the
 * FLOP count of such a launch (2 per multiply-add), or -1 for bad arguments. */
int macai_gdr_probe_mfma(int32_t mode, int32_t iters, void* out, int32_t blocks, void* stream);
int64_t macai_gdr_probe_mfma_flops(int32_t mode, int32_t iters, int32_t blocks);

#ifdef __cplusplus
}
#endif

#endif /* MACAI_GDR_H */

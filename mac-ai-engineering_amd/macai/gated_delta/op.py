"""The gated delta rule on MI355X: autograd functions over the HIP kernels, and a drop-in for transformers'
torch_chunk_gated_delta_rule (same arguments, same returns).

Mirrors the reference's src/macai/gated_delta/op.py: `GatedDeltaRule` keeps its autograd contract (op.py:116-257),
`chunk_gated_delta_rule` its drop-in signature and behaviour (op.py:264-298), `l2norm` and `recurrent_reference` its
helpers (op.py:260-261, 301-314).  The per-call passes (op.py:63-113, 159, 217, 234, 241-242) become the C-ABI calls of
include/macai_gdr.h on the current HIP stream.  What the training forward keeps for the backward follows
RECOMPUTE_STATES (the reference's switch, op.py:27-33).
"""
import collections
import contextlib
import math
import weakref

import torch

from . import _native as N

CHUNK = 64   # chunk length of the kernels; the drop-in's chunk_size is accepted and not used (as op.py:266-269)
# Head widths.  The float32 kernels take key heads of every multiple of 32 up to 256 and, in the backward, value heads
# of every multiple of 32 up to 256 (the reference takes any multiple of 32: op.py:124-125, _chunked.py:1228-1229; its
# tests reach 256, tests/test_harness.py:214-230).  The bf16 kernels take key heads of 32, 64 and 128 and, in the
# backward, value heads up to 128: other widths run the float32 kernels, with 2-byte inputs upcast exactly and the
# results cast back.
BF16_MAX_DK = 128
BF16_DK = (32, 64, 128)
BF16_MAX_DV_BWD = 128
MAX_DK = MAX_DV_BWD = 256
# FUSED_NORM (the reference's switch and default, op.py:19-21): with use_qk_l2norm_in_kernel=True the drop-in's
# query / key prologue (l2 normalisation, the query's DK^-1/2 scale) runs inside the kernels, its backward inside the
# per-chunk backward (True); False runs the normalisation as PyTorch operations in float32 (autograd takes its
# backward) and leaves the kernels only the scale.  The kernels then do not normalise the keys, so a bf16 call runs
# on the float32 kernels with the normalised query and key kept in float32 (unless BF16_UNNORMALIZED, which rounds
# them to bf16): rounding the normalised keys to bf16 adds their quantization to every product (dg 7.9e-3, o 7.5e-3
# worst over 30 random draws of the oracle's rounding model, against 5-7e-3 with the kernels' own normalisation).
FUSED_NORM = True
# BF16_OPERANDS: bfloat16 inputs run on bf16 MFMA operands with fp32 accumulation and an fp32 state (True, the
# default: the fast path, outputs and gradients within ~5e-3 of float64).  False upcasts them exactly and runs the
# float32 kernels, as the reference computes every input (op.py:276-285, 297): dg and dbeta then come within ~1e-5 of
# float64 (the bf16 operands' rounding, not the fp32 state, sets the default's error), at the float32 kernels' speed.
BF16_OPERANDS = True
# BF16_UNNORMALIZED: bf16 operands also for calls whose keys the kernels do not normalise (use_qk_l2norm_in_kernel=
# False).  Off by default: those calls run on the float32 kernels, because the bf16 operands' rounding is amplified
# as beta |k|^2 grows and only unit-norm keys keep it under the 1e-2 bar (the oracle's rounding model over N(0, 1)
# keys, |k|^2 ~ DK: 6e-3 to 1.2e-1; the same keys normalised: 5-6e-3).  A caller whose keys already have unit norm can
# turn it on, or pass use_qk_l2norm_in_kernel=True (normalising a unit vector again changes it by rounding only).
BF16_UNNORMALIZED = False
# BF16_MIN_TOKENS: bf16 calls that save for a backward, on rows shorter than this many tokens, run on the float32
# kernels.  With few tokens the bf16 operands' rounding is not averaged out -- dg and dq of a row of a few tokens are
# sums of few, cancelling terms, and dg of a row of about one chunk is small against its terms: the oracle's rounding
# model of the bf16 path puts 12 of 160 random rows of 2, 3, 5 and 8 tokens over the 1e-2 bar (dg up to 5.7e-2), 2
# of 150 rows of 64 tokens and 1 of 150 of 65 (dg up to 1.7e-2, through Vn in the per-chunk backward's dO Vn^T), and
# none of 150 each at 72, 80, 88, 96, 100, 112 and 128 tokens -- and the float32 kernels cost next to nothing at that
# size.  The forward's outputs are not affected (the model's worst o and sT over 60 draws of 1-16 tokens: 8e-3, as on
# long rows), so a forward without gradients keeps the bf16 kernels.  0 keeps every length on the bf16 kernels.
BF16_MIN_TOKENS = 80
# BF16_STATE_GRAD: the backward of a bf16 call whose final state receives a gradient (sT in the loss, or passed on
# to a later segment's backward) keeps the bf16 operands (True) or runs on the float32 kernels (False, the default:
# the inputs upcast exactly, the states recomputed, dq, dk, dv cast back).  A final-state gradient of the size of the
# output's feeds the last chunk's state gradient and, through it, dg's Vn dS^T terms and dbeta's dVn, whose bf16
# rounding then no longer averages out: over random draws of 64-200 tokens with an N(0, 1) final-state gradient the
# bf16 backward put dg or dbeta over the 1e-2 bar in about one draw in six (dg up to 3.0e-2, dbeta up to 1.7e-2; the
# oracle's rounding model and the kernels agree to three digits), against at most 6.8e-3 over the same draws without
# it.  A backward without a final-state gradient (output_final_state=False, or sT unused) keeps the bf16 kernels.
BF16_STATE_GRAD = False
# VALUE_SPLIT: workgroups a head-row's value columns are split over in the state passes (each owns DV / VALUE_SPLIT
# columns as DV / 16 / VALUE_SPLIT waves of 16 columns): "auto" (split_for) or 1, 2, 4, 8, ...
VALUE_SPLIT = "auto"
# the passes' calls by what they ran, "fwd s<split>" / "bwd <state passes> s<split>" with <state passes> "pair"
# (recompute and reverse pass in one launch), "recompute+reverse" (two launches) or "reverse" (the forward kept the
# states); counted at every call, no GPU work
CALLS = collections.Counter()
# Measurement hook: set to a list to record (pass, start event, end event) around every launch, on the launch stream;
# None (the default) records nothing.
EVENTS = None
# The backward's recompute pass (storing S_c, Vn) and its reverse pass need only prep's outputs, not each other: with
# OVERLAP they run in one launch (macai_gdr_state_pair), each on about half the CUs.  Both are sequential chunk chains
# whose speed hardly depends on how many CUs they get, so this nearly hides one of them -- with 2-byte operands.  On
# float32 operands the pair is the slower choice (config 1: 311 us for the pair against 97 + 182 us as two launches,
# the step 1.162 against 1.125 ms), so "auto" (the default) pairs the passes for bf16 and fp16 operands only; True
# pairs them always, False never.  Same bits every way.
OVERLAP = "auto"
# MIXED_IO (no counterpart in the reference, which upcasts): a bf16 call computed on the float32 kernels (the routing
# rules of compute_dtype) hands its bf16 q, k, v to the kernels as they are -- prep and the per-chunk backward read
# them exactly into float32, the state pass writes o and the per-chunk backward dq, dk, dv in bf16, one rounding each
# -- instead of upcasting them and casting the results back (8 passes over token tensors a training step, ~70 us at
# config 1).  The same bits either way; dO is still upcast (the reverse pass reads it as a float32 tile).  Grouped
# heads (Hk < H) upcast, as their dq, dk are summed over each group in float32 first.
MIXED_IO = True


def pairs_states(dtype) -> bool:
    """Whether the recompute backward runs its two state passes as one launch for operands of this dtype."""
    return OVERLAP is True or (OVERLAP == "auto" and dtype != torch.float32)
# RECOMPUTE_STATES (the reference's switch and default, op.py:27-33; outputs and gradients have the same bits either
# way):
# True (the default) -- the training forward keeps only its inputs; the backward reruns prep (with A) and recomputes
# the chunk states S_c and Vn beside its reverse pass (macai_gdr_state_pair).
# False -- the training forward runs prep in its backward mode (A as well) and its state pass stores S_c and Vn beside
# the output; it keeps those and prep's per-chunk operands W, U, Ke, Qg, M, GL, A for the backward, which then runs
# only the reverse state pass and the per-chunk backward.  At D = 128 in bf16 that is 2,816 bytes per token-head, 11x
# q's (176 MiB a layer at B = 4, T = 1024, H = 16), in one allocation saved with save_for_backward (so saved-tensor
# hooks, activation checkpointing and offload see it and it goes with the graph).
RECOMPUTE_STATES = True
# KEEP_PREP (no counterpart in the reference, whose switch has two settings): with RECOMPUTE_STATES, the training
# forward also keeps prep's per-chunk operands with A (W, U, Ke, Qg, M, A, GL: 1,536 bytes per token-head at D = 128
# in bf16, 96 MiB a layer at B = 4, T = 1024, H = 16, a little over half of what RECOMPUTE_STATES = False keeps), and
# the backward skips its prep but still recomputes the chunk states beside its reverse pass (macai_gdr_state_pair).
# Outputs and gradients have the same bits in every mode.  False (the default) is the reference's form.
KEEP_PREP = False
# SEQUENCE_SPLIT: segments a long row's forward without gradients runs side by side.  A state pass is a chain over
# the row's chunks; with few head-rows (one long prefill) it fills few CUs and its length is the row's.  The pass is
# affine in its starting state, so the row splits into segments: each segment's map [A | B] (macai_gdr_state_map,
# from the identity and from zero), their composition in order (macai_gdr_state_scan) for each segment's starting
# state, and the output pass over all segments at once.  The maps cost a second chain over DK + DV columns, so the
# split pays only where the plain pass leaves most CUs idle.  "auto": for a single row (B = 1, no cu_seqlens) whose
# plain pass has at most 128 workgroups of 16 columns (H x DV / 16 <= 128), the largest power of two P with P x H <= 128
# head-rows and at least 32 chunks a segment (P = 1 otherwise); an int forces P.  The map pass then runs 8 waves of
# columns a workgroup where that keeps its workgroups to one a CU (split_for's waves=8).  Measured at T = 32,768,
# D = 128, H = 16: P = 8 (maps 143 us, scan 26, output 195) against P = 4 (maps 178, scan 15, output 205) and the
# plain pass's 566 us; at H = 32 the plain pass already fills the chip (256 workgroups) and a split in 2 took 810
# against 637 us.
SEQUENCE_SPLIT = "auto"


def _launch(name: str, entry: str, *args):
    """One C-ABI launch; timed on the launch stream when EVENTS is a list."""
    if EVENTS is None:
        N.call(entry, *args)
        return
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    N.call(entry, *args)
    e1.record()
    EVENTS.append((name, e0, e1))


def valid_splits(dv: int) -> list:
    """Splits the state kernels take: s divides the dv / 16 column slices and leaves 1, 2, 4 or 8 waves per
    workgroup."""
    slices = dv // 16
    return [s for s in range(1, slices + 1) if slices % s == 0 and slices // s in (1, 2, 4, 8)]


_SPLITS = {}     # (rows, T, dv, share, VALUE_SPLIT) -> split: the launch path asks on every call


def split_for(rows: int, T: int, dv: int, share: int = 1, waves: int = 4) -> int:
    """The value split for a pass (_split_for's rule), remembered per shape and VALUE_SPLIT setting."""
    key = (rows, T, dv, share, waves, VALUE_SPLIT)
    s = _SPLITS.get(key)
    if s is None:
        s = _SPLITS[key] = _split_for(rows, T, dv, share, waves)
    return s


def _split_for(rows: int, T: int, dv: int, share: int = 1, waves: int = 4) -> int:
    """VALUE_SPLIT's choice for `rows` head-rows (B x H) of value width dv, for a pass that gets 1 / share of the
    chip: "auto" takes the largest valid split whose workgroups fit the pass's share of the CUs at once (rows x split
    <= 256 / share: a state pass's workgroup holds its CU's LDS, and a second round of a sequential pass would double
    its time), else the smallest; an int setting is rounded down to a valid split.  "auto" leaves out the splits with
    8 waves of columns per workgroup where another exists: with the loader wave that is 9 waves, 3 on one SIMD, which
    caps a wave at 168 VGPRs: the 128-wide state kernels spill there (the backward's pair pass ran 2.1-2.8x slower
    than at 4 waves); waves=8 admits them (the segment map pass at key heads up to 128, whose kernel holds 118-151
    VGPRs at 8 waves; at 256 it spills)."""
    valid = valid_splits(dv)
    if VALUE_SPLIT == "auto":
        valid = [s for s in valid if (dv // 16) // s <= waves] or valid
        fits = [s for s in valid if rows * s * share <= 256]
        return fits[-1] if fits else valid[0]
    want = int(VALUE_SPLIT)
    below = [s for s in valid if s <= want]
    return below[-1] if below else valid[0]


def _check(q, k, v, g, beta, s0, nseq=None):
    """q, k [B, T, Hk, DK], v [B, T, H, DV] with H a multiple of Hk (grouped value heads: value head h reads key head
    h // (H // Hk), the layout of q.repeat_interleave(H // Hk, dim=2)); g, beta [B, T, H]; s0 [B, H, DK, DV] -- or,
    for packed rows (nseq sequences in one row), B = 1 and s0 [nseq, H, DK, DV]."""
    if not q.is_cuda:
        raise RuntimeError("macai's gated delta rule runs on a HIP device (MI355X); got tensors on " + str(q.device))
    if q.dim() != 4 or k.shape != q.shape or v.dim() != 4 or v.shape[:2] != q.shape[:2]:
        raise ValueError(f"q, k [B, T, Hk, DK] and v [B, T, H, DV] expected, got {tuple(q.shape)}, {tuple(k.shape)}, "
                         f"{tuple(v.shape)}")
    B, T, Hk, DK = q.shape
    H = v.shape[2]
    if Hk == 0 or H % Hk != 0:
        raise ValueError(f"the key heads of q and k ({Hk}) must divide the value heads of v ({H})")
    if g.shape != (B, T, H) or beta.shape != (B, T, H):
        raise ValueError(f"g and beta must be [B, T, H] = {(B, T, H)}, got {tuple(g.shape)}, {tuple(beta.shape)}")
    if nseq is not None and B != 1:
        raise ValueError(f"packed rows (cu_seqlens) take a batch of one row, got B = {B}")
    S = B if nseq is None else nseq
    if s0 is not None and s0.shape != (S, H, DK, v.shape[-1]):
        raise ValueError(f"initial_state must be [{'B' if nseq is None else 'sequences'}, H, DK, DV] = "
                         f"{(S, H, DK, v.shape[-1])}, got {tuple(s0.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError(f"q, k, v must share a dtype, got {q.dtype}, {k.dtype}, {v.dtype}")
    if g.dtype != torch.float32 or beta.dtype != torch.float32 or (s0 is not None and s0.dtype != torch.float32):
        raise ValueError("g, beta and the state must be float32")


def _dims(q, v, pack=None):
    """(B, T, H value heads, Hk key heads, DK, DV, NT); with packed rows B is the number of sequences and NT the
    chunks of all of them."""
    B, T, Hk, DK = q.shape
    if pack is not None:
        return pack[2], T, v.shape[2], Hk, DK, v.shape[-1], pack[1]
    return B, T, v.shape[2], Hk, DK, v.shape[-1], math.ceil(T / CHUNK)


# packed-row tables by cu_seqlens tensor: a model passes the same one to every layer, and building the table reads it
# back to the host (a synchronisation), so it is built once per tensor (and per in-place change of it)
_PACKS = {}   # id(tensor) -> (weak reference, (version, T, device), table); an entry goes when its tensor does


def _pack(cu_seqlens, T: int, device):
    """The packed-row table of include/macai_gdr.h for sequences cu[n] .. cu[n+1] of one row of T tokens: each
    sequence chunked on its own.  Returns (table [2 NT + N + 1] int32 on `device`, NT, N)."""
    key = cu_seqlens if isinstance(cu_seqlens, torch.Tensor) else None
    if key is not None:
        hit = _PACKS.get(id(key))
        if hit is not None and hit[0]() is key and hit[1] == (key._version, T, str(device)):
            return hit[2]
    cu = torch.as_tensor(cu_seqlens).reshape(-1).to("cpu", torch.int64).tolist()
    if len(cu) < 2 or cu[0] != 0 or cu[-1] != T or any(b < a for a, b in zip(cu, cu[1:])):
        raise ValueError(f"cu_seqlens must rise from 0 to T = {T} (got {cu[:8]}{'...' if len(cu) > 8 else ''})")
    t0s, ends, c0 = [], [], [0]
    for a, b in zip(cu, cu[1:]):
        for t in range(a, b, CHUNK):
            t0s.append(t)
            ends.append(b)
        c0.append(len(t0s))
    table = torch.tensor(t0s + ends + c0, dtype=torch.int32, device=device)
    out = (table, len(t0s), len(cu) - 1)
    if key is not None:
        if id(key) not in _PACKS:
            weakref.finalize(key, _PACKS.pop, id(key), None)
        _PACKS[id(key)] = (weakref.ref(key), (key._version, T, str(device)), out)
    return out


def _pack_args(pack):
    return (None, 0) if pack is None else (N.ptr(pack[0]), pack[1])


def _on(dev):
    """The device guard a launch needs: none when dev is already the current device (the common case, and the guard
    costs host time on every call)."""
    return contextlib.nullcontext() if dev.index == torch.cuda.current_device() else torch.cuda.device(dev)


_LAYOUTS = {}    # scratch layouts by shape: (part offsets, total bytes)


def _layout(shape):
    """(part offsets, total bytes) of the scratch for `shape`; every part starts on a 256-byte boundary."""
    lay = _LAYOUTS.get(shape)
    if lay is None:
        offs, total = {}, 0
        for name, n in _scratch_sizes(*shape).items():
            offs[name] = total if n else None
            total += (n + 255) & ~255
        lay = _LAYOUTS[shape] = (offs, max(total, 1))
    return lay


def _parts(buf, shape):
    """{name: device address or None, "buf": buf, "shape": shape} for a scratch allocation of `shape`.  Addresses are
    taken from buf each time, so a buffer that a saved-tensor hook moved and brought back is addressed where it is
    now."""
    base = buf.data_ptr()
    out = {name: (None if o is None else base + o) for name, o in _layout(shape)[0].items()}
    out["buf"], out["shape"] = buf, shape
    return out


def _carve(dev, shape):
    """One allocation for the per-chunk scratch of a call, `shape` = (Bc, H, NT, DK, DV, element size, prep, with_A,
    states, grads) as _scratch_sizes takes it.  Returns _parts of it.  The kernels take raw addresses, so the parts
    need no tensor views."""
    return _parts(torch.empty(_layout(shape)[1], device=dev, dtype=torch.uint8), shape)


def _scratch_sizes(Bc, H, NT, DK, DV, es, prep: bool, with_A: bool, states: bool, grads: bool):
    """Byte counts of the per-chunk tensors, all [Bc, H, NT, ...] row-major: prep's W, U, Ke, GL, Qg, M (and A); the
    chunk states Sc (fp32) and Vn; the reverse pass's dSn (fp32) and dVn."""
    n = Bc * H * NT
    z = lambda on, b: b if on else 0
    return dict(W=z(prep, n * CHUNK * DK * es), U=z(prep, n * CHUNK * DV * 4), Ke=z(prep, n * CHUNK * DK * es),
                GL=z(prep, n * 4), Qg=z(prep, n * CHUNK * DK * es), M=z(prep, n * CHUNK * CHUNK * es),
                A=z(prep and with_A, n * CHUNK * CHUNK * es), Sc=z(states, n * DK * DV * 4),
                Vn=z(states, n * CHUNK * DV * es), dSn=z(grads, n * DK * DV * 4), dVn=z(grads, n * CHUNK * DV * es))


def _as(x, dt):
    """x in dtype dt, contiguous and 16-byte aligned (the kernels' vector accesses): x itself when it already is
    (skips two calls on the launch path), a copy when it is not -- also when only its start is misaligned, as a view
    at an odd offset of a larger tensor is (the reference's _even, op.py:58-60, copies such a tensor too)."""
    if x.dtype == dt and x.is_contiguous() and x.data_ptr() % 16 == 0:
        return x
    y = x.to(dt).contiguous()
    return y if y.data_ptr() % 16 == 0 else y.clone()


def _prep(q, k, v, g, beta, l2norm: bool, q_scale: float, r, stream, pack=None, name="prep_fwd", mixed=False):
    """The per-chunk operands (row-major, tokens as rows) into the scratch r (addresses from _carve): W, U, diag(e) K^,
    exp(G_last), diag(gamma) Q^, M, and A when r has it (the backward's per-chunk pass needs it).  Per-chunk tensors
    are [B, H, NT, ...] ([1, H, NT, ...] for packed rows).  mixed: bf16 q, k, v read into float32 arithmetic and
    float32 operands (macai_gdr_prep's MACAI_GDR_BF16_F32)."""
    B, T, H, Hk, DK, DV, NT = _dims(q, v, pack)
    P = N.ptr
    code = N.BF16_F32 if mixed else N.dtype_code(q.dtype)
    _launch(name, "macai_gdr_prep", P(q), P(k), P(v), P(g), P(beta), r["W"], r["U"], r["Ke"], r["GL"], r["Qg"], r["M"],
            r["A"], B, T, H, Hk, DK, DV, code, int(l2norm), q_scale, *_pack_args(pack), stream)


def segments_for(B: int, T: int, H: int, DV: int, pack=None, save: bool = False) -> int:
    """SEQUENCE_SPLIT's number of segments for a forward of B rows of T tokens over H value heads of DV columns (1: no
    split).  A forward that saves for a backward never splits: the training step keeps the bits of the unsplit pass."""
    if save or pack is not None or B != 1:
        return 1
    NT = math.ceil(T / CHUNK)
    if SEQUENCE_SPLIT != "auto":
        return max(1, min(int(SEQUENCE_SPLIT), NT))
    if H * (DV // 16) > 128:
        return 1
    P = 1
    while 2 * P * H <= 128 and NT // (2 * P) >= 32:
        P *= 2
    return P


_SEGS = {}       # (T, P, device) -> the packed-row table of a row split into P segments of whole chunks


def _segment_table(T: int, P: int, device):
    """The packed-row table (include/macai_gdr.h) of one row of T tokens as P sequences of consecutive whole chunks:
    chunk c spans tokens 64 c .. 64 c + 63 (the row's end bounds its last chunk), segment s owns chunks
    ceil(NT / P) s .. (the last one the rest).  Returns (table, NT)."""
    key = (T, P, str(device))
    hit = _SEGS.get(key)
    if hit is None:
        NT = math.ceil(T / CHUNK)
        L = math.ceil(NT / P)
        c0 = [min(s * L, NT) for s in range(P)] + [NT]
        table = torch.tensor([c * CHUNK for c in range(NT)] + [T] * NT + c0, dtype=torch.int32, device=device)
        hit = _SEGS[key] = (table, NT)
    return hit


def _forward_segments(q, k, v, g, beta, s0, l2norm: bool, q_scale: float, want_sT: bool, nseg: int):
    """The forward of one row split into nseg segments (SEQUENCE_SPLIT): prep, the segments' maps, their composition
    into each segment's starting state, then the output pass over the segments side by side."""
    _, T, H, Hk, DK, DV, NT = _dims(q, v)
    dev, dt = q.device, q.dtype
    code, stream = N.dtype_code(dt), N.stream_of(q)
    f32 = torch.float32
    P = N.ptr
    r = _carve(dev, (1, H, NT, DK, DV, q.element_size(), True, False, False, False))
    _prep(q, k, v, g, beta, l2norm, q_scale, r, stream, None, "prep_fwd")
    table, NT = _segment_table(T, nseg, dev)
    # the maps of all segments but the last (its map composes into no later start): the first nseg - 1 sequences of
    # the table
    maps = torch.empty(nseg - 1, H, DK, DK + DV, device=dev, dtype=f32)
    _launch("state_map", "macai_gdr_state_map", r["W"], r["U"], r["Ke"], r["GL"], P(maps), nseg - 1, T, H, DK, DV,
            code, split_for((nseg - 1) * H, T, DK + DV, waves=8 if DK <= 128 else 4), P(table), NT, stream)
    starts = torch.empty(nseg, H, DK, DV, device=dev, dtype=f32)
    _launch("state_scan", "macai_gdr_state_scan", P(maps), P(s0), P(starts), 1, nseg, H, DK, DV, stream)
    o = torch.empty(1, T, H, DV, device=dev, dtype=dt)
    sTs = torch.empty(nseg, H, DK, DV, device=dev, dtype=f32) if want_sT else None
    split = split_for(nseg * H, T, DV)
    _launch("state_fwd_out", "macai_gdr_state_fwd", r["W"], r["U"], r["Ke"], r["GL"], r["Qg"], r["M"], P(starts), P(o),
            P(sTs), None, None, nseg, T, H, DK, DV, code, 0, split, P(table), NT, stream)
    CALLS[f"fwd seg{nseg} s{split}"] += 1
    return o, (None if sTs is None else sTs[nseg - 1:]), None


def _forward(q, k, v, g, beta, s0, l2norm: bool, q_scale: float, want_sT: bool, pack=None, keep=False, save=True,
             mixed=False):
    """prep, then the state pass with the output: returns (o in q's dtype, sT or None, and for the backward, when
    keep, prep's operands with A and the chunk states Sc, Vn, or, when the forward saves and KEEP_PREP, prep's
    operands with A alone; else None).  A single long row whose forward saves
    nothing for a backward may run as segments side by side (SEQUENCE_SPLIT).  mixed: bf16 q, k, v computed in
    float32 (float32 per-chunk operands; o written in bf16)."""
    B, T, H, Hk, DK, DV, NT = _dims(q, v, pack)
    nseg = segments_for(B, T, H, DV, pack, save or keep)
    if nseg > 1:
        if mixed:                          # the segmented passes take one operand type: upcast exactly
            q, k, v = q.float(), k.float(), v.float()
            o, sT, r = _forward_segments(q, k, v, g, beta, s0, l2norm, q_scale, want_sT, nseg)
            return o.to(torch.bfloat16), sT, r
        return _forward_segments(q, k, v, g, beta, s0, l2norm, q_scale, want_sT, nseg)
    Bc = q.shape[0]
    dev, dt = q.device, q.dtype
    code, stream = (N.BF16_F32 if mixed else N.dtype_code(dt)), N.stream_of(q)
    keep_prep = save and KEEP_PREP and not keep       # prep's operands with A, without the chunk states
    es = 4 if mixed else q.element_size()
    r = _carve(dev, (Bc, H, NT, DK, DV, es, True, keep or keep_prep, keep, False))
    _prep(q, k, v, g, beta, l2norm, q_scale, r, stream, pack, "prep_fwd", mixed)
    o = torch.empty(Bc, T, H, DV, device=dev, dtype=dt)
    sT = torch.empty(B, H, DK, DV, device=dev, dtype=torch.float32) if want_sT else None
    split = split_for(B * H, T, DV)
    P = N.ptr
    _launch("state_fwd_out", "macai_gdr_state_fwd", r["W"], r["U"], r["Ke"], r["GL"], r["Qg"], r["M"], P(s0), P(o), P(sT),
            r["Sc"], r["Vn"], B, T, H, DK, DV, code, N.STORE_STATES if keep else 0, split, *_pack_args(pack), stream)
    CALLS[f"fwd s{split}"] += 1
    return o, sT, (r if keep or keep_prep else None)


def _backward(q, k, v, g, beta, s0, do, dsT, l2norm: bool, q_scale: float, pack=None, r=None, mixed=False):
    """Recompute (prep, unless the forward kept its operands in `r`, and the state pass storing S_c and Vn, unless the
    forward kept them too), the reverse state pass, the per-chunk backward.  Returns (dq, dk, dv in q's dtype; dg,
    dbeta, ds0 float32).  With grouped heads (Hk < H) the per-chunk backward writes dq, dk per value head and
    macai_gdr_group_sum folds each group (the backward of the repeat the grouped layout replaces).  mixed: bf16 q, k,
    v (and dq, dk, dv) with float32 arithmetic, operands and dO (Hk == H)."""
    B, T, H, Hk, DK, DV, NT = _dims(q, v, pack)
    Bc = q.shape[0]
    dev, dt = q.device, q.dtype
    f32 = torch.float32
    assert not mixed or (Hk == H and do.dtype == f32), "mixed types: Hk == H and a float32 dO"
    mt = f32 if mixed else dt              # the operands' type (the state passes run on it)
    code, stream = N.dtype_code(mt), N.stream_of(q)
    code_io = N.BF16_F32 if mixed else code   # prep and the per-chunk backward read (and write) q's dtype
    es = 4 if mixed else q.element_size()
    kept = r is not None and r["Sc"] is not None   # the forward kept prep's operands and the chunk states: only the
    if kept:                                       # reverse pass is left
        g2 = _carve(dev, (Bc, H, NT, DK, DV, es, False, False, False, True))
    elif r is not None:                            # it kept prep's operands (KEEP_PREP): no prep here
        g2 = _carve(dev, (Bc, H, NT, DK, DV, es, False, False, True, True))
    else:
        r = g2 = _carve(dev, (Bc, H, NT, DK, DV, es, True, True, True, True))
        _prep(q, k, v, g, beta, l2norm, q_scale, r, stream, pack, "prep_bwd", mixed)
    P = N.ptr
    pk = _pack_args(pack)
    pair = pairs_states(mt) and not kept
    split = split_for(B * H, T, DV, 2 if pair else 1)
    st = r if kept else g2
    Sc, Vn, dSn, dVn = st["Sc"], st["Vn"], g2["dSn"], g2["dVn"]
    ds0 = torch.empty(B, H, DK, DV, device=dev, dtype=f32)
    if kept:
        _launch("state_bwd", "macai_gdr_state_bwd", r["Ke"], r["Qg"], r["W"], r["M"], r["GL"], P(do), P(dsT), dSn, dVn,
                P(ds0), B, T, H, DK, DV, code, split, *pk, stream)
    elif pair:
        _launch("state_pair", "macai_gdr_state_pair", r["W"], r["U"], r["Ke"], r["Qg"], r["M"], r["GL"], P(s0), P(do),
                P(dsT), Sc, Vn, dSn, dVn, P(ds0), B, T, H, DK, DV, code, split, *pk, stream)
    else:
        _launch("state_fwd_store", "macai_gdr_state_fwd", r["W"], r["U"], r["Ke"], r["GL"], None, None, P(s0), None,
                None, Sc, Vn, B, T, H, DK, DV, code, N.STORE_STATES | N.NO_OUTPUT, split, *pk, stream)
        _launch("state_bwd", "macai_gdr_state_bwd", r["Ke"], r["Qg"], r["W"], r["M"], r["GL"], P(do), P(dsT), dSn, dVn,
                P(ds0), B, T, H, DK, DV, code, split, *pk, stream)
    CALLS[f"bwd {'reverse' if kept else 'pair' if pair else 'recompute+reverse'} s{split}"] += 1
    if Hk == H:
        dqh, dkh = torch.empty_like(q), torch.empty_like(k)
    else:
        dqh = torch.empty(Bc, T, H, DK, device=dev, dtype=dt)
        dkh = torch.empty_like(dqh)
    dv = torch.empty_like(v)
    dg, dbeta = torch.empty_like(g), torch.empty_like(beta)
    _launch("chunk_bwd", "macai_gdr_chunk_bwd", P(q), P(k), P(v), P(g), P(beta), P(do), r["A"], Sc, dSn, Vn, dVn,
            P(dqh), P(dkh), P(dv), P(dg), P(dbeta), B, T, H, Hk, DK, DV, code_io, int(l2norm), q_scale, *pk, stream)
    if Hk == H:
        return dqh, dkh, dv, dg, dbeta, ds0
    dq, dk = torch.empty_like(q), torch.empty_like(k)
    _launch("group_sum", "macai_gdr_group_sum", P(dqh), P(dq), Bc, T, H, Hk, DK, code, stream)
    _launch("group_sum", "macai_gdr_group_sum", P(dkh), P(dk), Bc, T, H, Hk, DK, code, stream)
    return dq, dk, dv, dg, dbeta, ds0


def _backward_routed(q, k, v, g, beta, s0, do, dsT, l2norm: bool, q_scale: float, pack=None, r=None, mixed=False):
    """_backward, or -- for bf16 operands with a final-state gradient while BF16_STATE_GRAD is off -- _backward on the
    float32 kernels: q, k, v read exactly (mixed types where MIXED_IO and Hk == H, else upcast), dO upcast, the states
    recomputed (the forward's kept bf16 operands, if any, are not used), dq, dk, dv rounded to bf16."""
    if mixed or dsT is None or q.dtype != torch.bfloat16 or BF16_STATE_GRAD:
        return _backward(q, k, v, g, beta, s0, do, dsT, l2norm, q_scale, pack, r, mixed)
    CALLS["bwd f32 for a final-state gradient"] += 1
    f32 = torch.float32
    if MIXED_IO and k.shape[2] == v.shape[2]:
        return _backward(q, k, v, g, beta, s0, do.to(f32), dsT, l2norm, q_scale, pack, None, True)
    dq, dk, dv, dg, dbeta, ds0 = _backward(q.to(f32), k.to(f32), v.to(f32), g, beta, s0, do.to(f32), dsT, l2norm,
                                           q_scale, pack)
    return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg, dbeta, ds0


def _save(ctx, inputs, r):
    """Save the inputs and, when the forward kept its per-chunk scratch (RECOMPUTE_STATES False, or KEEP_PREP), that
    allocation with them: save_for_backward hands both to saved-tensor hooks and frees them with the graph."""
    ctx.save_for_backward(*inputs, None if r is None else r["buf"])
    ctx.kept_shape = None if r is None else r["shape"]


def _saved(ctx):
    """(inputs, the kept scratch's parts or None) from _save."""
    *inputs, buf = ctx.saved_tensors
    return inputs, (None if buf is None else _parts(buf, ctx.kept_shape))


class GatedDeltaRule(torch.autograd.Function):
    """o, S_T = recurrence(q, k, v, g, beta, S_0) on [B, T, H, D] tensors (q already normalised and scaled): the
    reference's contract (op.py:116-257).  q and k may also have fewer heads Hk dividing H (grouped value heads,
    value head h using key head h // (H // Hk)); their gradients then come back in that shape.  q, k, v float32 or
    bfloat16 (o in that dtype), g, beta, s0 float32. backward -> (dq, dk, dv, dg, dbeta, ds0, None); None upstream
    gradients count as zeros (op.py:194-200)."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, s0, save: bool):
        _check(q, k, v, g, beta, s0)
        ctx.io_dtype = q.dtype             # o and the q, k, v gradients come back in it
        _widths(q.shape[-1], v.shape[-1], save)
        if q.dtype != compute_dtype(q.dtype, q.shape[-1], v.shape[-1], save, tokens=q.shape[1]):
            q, k, v = q.float(), k.float(), v.float()
        q, k, v = (_as(t, t.dtype) for t in (q, k, v))
        g, beta, s0 = (_as(t, torch.float32) for t in (g, beta, s0))
        keep = save and not RECOMPUTE_STATES
        with _on(q.device):
            o, sT, r = _forward(q, k, v, g, beta, s0, False, 1.0, True, keep=keep, save=save)
        if save:
            _save(ctx, (q, k, v, g, beta, s0), r)
        ctx.set_materialize_grads(False)   # an unused sT's gradient arrives as None, not as zeros (BF16_STATE_GRAD)
        return o.to(ctx.io_dtype), sT

    @staticmethod
    def backward(ctx, do, dsT):
        (q, k, v, g, beta, s0), r = _saved(ctx)
        do = torch.zeros_like(v) if do is None else _as(do, v.dtype)
        dsT = None if dsT is None else _as(dsT, torch.float32)
        with _on(q.device):
            dq, dk, dv, dg, dbeta, ds0 = _backward_routed(q, k, v, g, beta, s0, do, dsT, False, 1.0, None, r)
        dt = ctx.io_dtype
        return dq.to(dt), dk.to(dt), dv.to(dt), dg, dbeta, ds0, None


class _DropIn(torch.autograd.Function):
    """The drop-in's rule on the raw query / key: the l2norm prologue (and q's DK^-1/2 scale) is applied inside the
    kernels and its backward fused into the per-chunk backward (the reference runs it as separate L2NormScale passes,
    _norm.py:81-114).  s0 may be None (zeros); sT is returned only when want_sT.  pack: the packed-row table of
    _pack (cu_seqlens) or None."""

    @staticmethod
    def forward(ctx, query, key, value, g, beta, s0, l2norm: bool, q_scale: float, want_sT: bool, save: bool,
                pack=None, mixed=False):
        keep = save and not RECOMPUTE_STATES
        with _on(query.device):
            o, sT, r = _forward(query, key, value, g, beta, s0, l2norm, q_scale, want_sT, pack, keep, save, mixed)
        if save:
            _save(ctx, (query, key, value, g, beta, s0), r)
            ctx.cfg = (l2norm, q_scale, s0 is not None)
            ctx.pack = pack
            ctx.mixed = mixed
        ctx.set_materialize_grads(False)   # an unused sT's gradient arrives as None, not as zeros (BF16_STATE_GRAD)
        if sT is None:
            return o
        return o, sT

    @staticmethod
    def backward(ctx, do, dsT=None):
        (query, key, value, g, beta, s0), r = _saved(ctx)
        l2norm, q_scale, has_s0 = ctx.cfg
        ddt = torch.float32 if ctx.mixed else value.dtype
        do = torch.zeros_like(value, dtype=ddt) if do is None else _as(do, ddt)
        dsT = None if dsT is None else _as(dsT, torch.float32)
        with _on(query.device):
            dq, dk, dv, dg, dbeta, ds0 = _backward_routed(query, key, value, g, beta, s0, do, dsT, l2norm, q_scale,
                                                          ctx.pack, r, ctx.mixed)
        return dq, dk, dv, dg, dbeta, (ds0 if has_s0 else None), None, None, None, None, None, None


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return x * torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)


def compute_dtype(dtype, DK: int, DV: int = 0, save: bool = False, normalized: bool = True, tokens: int = None):
    """The operand type the kernels compute a call in: bfloat16 inputs on bf16 MFMA at key widths 32, 64, 128 and --
    when the call saves for a backward -- value widths up to 128 (unless BF16_OPERANDS is off), when the kernels
    normalise the keys (normalized: use_qk_l2norm_in_kernel with FUSED_NORM; unless BF16_UNNORMALIZED) and, when the
    call saves for a backward, the rows hold at least BF16_MIN_TOKENS tokens (tokens:
    the row length; None: not checked); float16, float32 and everything else on the float32 kernels."""
    bf16 = (dtype == torch.bfloat16 and DK in BF16_DK and BF16_OPERANDS and (normalized or BF16_UNNORMALIZED)
            and (not save or (DV <= BF16_MAX_DV_BWD and (tokens is None or tokens >= BF16_MIN_TOKENS))))
    return torch.bfloat16 if bf16 else torch.float32


def _widths(DK: int, DV: int, save: bool):
    """Refuse head widths no kernel takes, before any work (the C ABI refuses them too)."""
    if DK % 32 or not 32 <= DK <= MAX_DK:
        raise NotImplementedError(f"key head width must be a multiple of 32 in [32, {MAX_DK}], got {DK}")
    if DV % 32 or not 32 <= DV <= 512:
        raise NotImplementedError(f"value head width must be a multiple of 32 in [32, 512], got {DV}")
    if save and DV > MAX_DV_BWD:
        raise NotImplementedError(f"the backward takes value head widths up to {MAX_DV_BWD}, got {DV}")


def eager_prologue(query, key, cdt):
    """FUSED_NORM = False: the l2 normalisation of query and key as PyTorch operations in float32 (the reference's
    unfused prologue, op.py:279-283), rounded to the compute dtype cdt; the kernels then apply only the query's
    DK^-1/2 scale (use_qk_l2norm_in_kernel=False).  Autograd takes the normalisation's backward."""
    return l2norm(query.float()).to(cdt), l2norm(key.float()).to(cdt)


def plan(B: int, T: int, H: int, DK: int, DV: int, save: bool, Hk: int = None, dtype=torch.bfloat16,
         cus: int = 256, l2norm: bool = True) -> dict:
    """What a drop-in call of these dimensions runs under the current settings (the reference's plan, op.py:105-113,
    for this build's kernels): the chunk length (64 for every pass), the operand type, the forward's segments, value
    split and state-pass kernel, and -- when the forward saves for a backward -- whether the backward recomputes
    (RECOMPUTE_STATES) and reruns prep (KEEP_PREP), its state passes, their split, the per-chunk backward's kernel and
    the operands of a backward that receives a gradient of the final state (BF16_STATE_GRAD).  cus: the device's
    compute units (the persistent per-chunk backward runs where there are more chunk-heads than CUs); l2norm: the call's
    use_qk_l2norm_in_kernel."""
    Hk = Hk or H
    cdt = compute_dtype(dtype, DK, DV, save, l2norm and FUSED_NORM, T)
    bf = cdt == torch.bfloat16
    NT = math.ceil(T / CHUNK)
    recompute = save and RECOMPUTE_STATES
    nseg = segments_for(B, T, H, DV, None, save)
    out = {"fwd_chunk": CHUNK, "bwd_chunk": CHUNK, "operands": "bf16" if bf else "f32",
           # bf16 tensors handed to the float32 kernels as they are (MIXED_IO), not upcast
           "mixed_io": bool(dtype == torch.bfloat16 and not bf and MIXED_IO and Hk == H),
           "prep": ("prep8" if bf and (DV <= 128 or DV % 128 == 0) else "prep"), "segments": nseg,
           "fused_norm": FUSED_NORM, "recompute": recompute}
    if nseg > 1:
        out["map_split"] = split_for((nseg - 1) * H, T, DK + DV, waves=8 if DK <= 128 else 4)
        out["fwd_split"] = split_for(nseg * H, T, DV)
    else:
        out["fwd_split"] = split_for(B * H, T, DV)
    waves = DV // 16 // out["fwd_split"]
    out["fwd_state_pass"] = "state_out" if bf and waves <= 2 else "state_fwd"
    if save:
        pair = recompute and pairs_states(cdt)
        out["bwd_state_passes"] = "pair" if pair else "recompute+reverse" if recompute else "reverse"
        out["bwd_prep"] = "rerun" if recompute and not KEEP_PREP else "kept"
        out["bwd_split"] = split_for(B * H, T, DV, 2 if pair else 1)
        units = B * H * NT
        out["chunk_bwd"] = (("chunk_bwd8xn" if DK == DV and units > cus else "chunk_bwd8") if bf else "chunk_bwd")
        # a backward that receives a gradient of the final state (BF16_STATE_GRAD)
        out["state_grad_operands"] = "f32" if bf and not BF16_STATE_GRAD else out["operands"]
    return out


def chunk_gated_delta_rule(query, key, value, g, beta, chunk_size: int = 64, initial_state=None,
                           output_final_state: bool = False, use_qk_l2norm_in_kernel: bool = False, **kwargs):
    """Drop-in for transformers' torch_chunk_gated_delta_rule: query, key [B, T, H, DK]; value [B, T, H, DV]; g (log
    decay, <= 0) and beta [B, T, H]; initial_state [B, H, DK, DV] or None.  query and key may also come with fewer
    heads Hk dividing H, unrepeated (value head h reads key head h // (H // Hk), as after repeat_interleave).
    cu_seqlens (packed rows, transformers' varlen form): B = 1 and the row holds the sequences cu[n] .. cu[n+1],
    each run on its own from initial_state[n] (initial_state [N, H, DK, DV] or None); the final state is [N, H, DK,
    DV]. The reference refuses cu_seqlens (op.py:270-273); here each sequence is chunked separately inside the
    kernels. Returns the output [B, T, H, DV] in the query's dtype and the final state (float32) when
    output_final_state, else None.  chunk_size is accepted and unused (the kernels use 64-token chunks).  bfloat16
    inputs run on bf16 MFMA with fp32 accumulation and an fp32 state; float32 inputs on fp32 MFMA; float16 inputs,
    and bfloat16 ones with key heads wider than 128 (up to 256), with BF16_OPERANDS off, with keys the kernels do not
    normalise (use_qk_l2norm_in_kernel=False, unless BF16_UNNORMALIZED) or, with gradients, rows shorter than
    BF16_MIN_TOKENS, are upcast exactly and computed as float32, the output cast back (the reference runs every input this way: its
    prologue and `value.float()` run the rule in float32, op.py:276-285, 297).  With use_qk_l2norm_in_kernel=False
    the query is only scaled by DK^-1/2 (op.py:279-283), inside the kernels."""
    cu = kwargs.get("cu_seqlens")
    if query.shape[0] == 0 or query.shape[1] == 0:
        return _no_tokens((query, key, value, g, beta), initial_state, output_final_state, cu)
    pack = None if cu is None else _pack(cu, query.shape[1], query.device)
    dtype = query.dtype
    grads = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (query, key, value, g, beta, initial_state))
    _widths(query.shape[-1], value.shape[-1], grads)
    cdt = compute_dtype(dtype, query.shape[-1], value.shape[-1], grads, bool(use_qk_l2norm_in_kernel) and FUSED_NORM,
                        query.shape[1])
    if use_qk_l2norm_in_kernel and not FUSED_NORM:
        query, key = eager_prologue(query, key, cdt)
        use_qk_l2norm_in_kernel = False
    # bf16 tensors computed in float32: read as they are, not upcast (MIXED_IO)
    mixed = (MIXED_IO and cdt == torch.float32 and query.dtype == key.dtype == value.dtype == torch.bfloat16
             and key.shape[2] == value.shape[2])
    tdt = torch.bfloat16 if mixed else cdt
    q, k, v = _as(query, tdt), _as(key, tdt), _as(value, tdt)
    gf, bf = _as(g, torch.float32), _as(beta, torch.float32)
    s0 = None if initial_state is None else _as(initial_state, torch.float32)
    _check(q, k, v, gf, bf, s0, None if pack is None else pack[2])
    tensors = (q, k, v, gf, bf) + (() if s0 is None else (s0,))
    save = torch.is_grad_enabled() and any(t.requires_grad for t in tensors)
    res = _DropIn.apply(q, k, v, gf, bf, s0, bool(use_qk_l2norm_in_kernel), q.shape[-1] ** -0.5,
                        bool(output_final_state), save, pack, mixed)
    out, sT = (res, None) if not output_final_state else res
    return (out if out.dtype == dtype else out.to(dtype)), sT


def _no_tokens(inputs, initial_state, output_final_state, cu=None):
    """A call without tokens (B = 0 or T = 0; inputs: query, key, value, g, beta): an empty output, and each starting
    state passed through as the final one (zeros without one), as the reference's torch path returns when it loops
    over no chunks (transformers modeling_qwen3_5.py:248-327); the inputs' gradients are empty and the state's is the
    final state's."""
    query, value = inputs[0], inputs[2]
    if not query.is_cuda:
        raise RuntimeError("macai's gated delta rule runs on a HIP device (MI355X); got tensors on " + str(query.device))
    B, T, H, DV = value.shape
    out = value.new_zeros(B, T, H, DV, dtype=query.dtype)
    if torch.is_grad_enabled() and any(t.requires_grad for t in inputs):
        out = out + sum(t.sum() for t in inputs) * 0      # empty: the output still hangs off the inputs
    if not output_final_state:
        return out, None
    S = B if cu is None else cu.numel() - 1
    if initial_state is None:
        return out, torch.zeros(S, H, query.shape[-1], DV, device=value.device, dtype=torch.float32)
    return out, initial_state.float().clone()


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state=None, output_final_state: bool = False,
                               use_qk_l2norm_in_kernel: bool = False, **kwargs):
    """Drop-in for transformers' torch_recurrent_gated_delta_rule (modeling_qwen3_5.py:330-380), the decode path the
    reference leaves to PyTorch (patch.py:27-29).  One token (T = 1) without autograd runs the decode kernel (one
    streaming pass over the fp32 state); longer inputs, or inputs that need gradients, run the chunked kernels, which
    compute the same recurrence."""
    T = query.shape[1]
    if query.shape[0] == 0 or T == 0:
        return _no_tokens((query, key, value, g, beta), initial_state, output_final_state, kwargs.get("cu_seqlens"))
    needs_grad = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (query, key, value, g, beta, initial_state))
    widths = (query.shape[-1], value.shape[-1])
    if (T != 1 or needs_grad or kwargs.get("cu_seqlens") is not None
            or not all(w in (64, 128) for w in widths)):   # the decode kernel's head widths
        return chunk_gated_delta_rule(query, key, value, g, beta, initial_state=initial_state,
                                      output_final_state=output_final_state,
                                      use_qk_l2norm_in_kernel=use_qk_l2norm_in_kernel,
                                      cu_seqlens=kwargs.get("cu_seqlens"))
    dtype = query.dtype
    cdt = torch.bfloat16 if dtype == torch.bfloat16 else torch.float32
    q, k, v = (_as(x, cdt) for x in (query, key, value))
    gf, bf = _as(g, torch.float32), _as(beta, torch.float32)
    B, _, Hk, DK = q.shape
    H, DV = v.shape[2], v.shape[-1]
    s_in = (torch.zeros(B, H, DK, DV, device=q.device, dtype=torch.float32) if initial_state is None
            else _as(initial_state, torch.float32))
    _check(q, k, v, gf, bf, s_in)
    o = torch.empty(B, 1, H, DV, device=q.device, dtype=cdt)
    s_out = torch.empty_like(s_in)
    with _on(q.device):
        N.call("macai_gdr_decode", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(gf), N.ptr(bf), N.ptr(s_in), N.ptr(o),
               N.ptr(s_out), B, H, Hk, DK, DV, N.dtype_code(cdt), int(bool(use_qk_l2norm_in_kernel)), DK ** -0.5,
               N.stream_of(q))
    return o.to(dtype), (s_out if output_final_state else None)


def recurrent_reference(q, k, v, g, beta, s0):
    """The rule one token at a time in plain PyTorch, for [B, T, H, D] inputs with q already normalised and scaled:
    per token the state decays by e^g, the prediction k^T S is corrected towards v by beta, and the output reads the
    updated state with q.  Kept for callers of the reference's helper of this name (op.py:301-314); no kernel path
    calls it.  Returns (o [B, T, H, DV], S_T)."""
    state = s0.clone()
    steps = []
    for qt, kt, vt, gt, bt in zip(q.unbind(1), k.unbind(1), v.unbind(1), g.unbind(1), beta.unbind(1)):
        state = state * torch.exp(gt)[:, :, None, None]
        miss = (vt - torch.matmul(kt.unsqueeze(-2), state).squeeze(-2)) * bt.unsqueeze(-1)
        state = state + kt.unsqueeze(-1) * miss.unsqueeze(-2)
        steps.append(torch.matmul(qt.unsqueeze(-2), state).squeeze(-2))
    return torch.stack(steps, 1), state

"""Each HIP pass against the float64 oracle's intermediates (W, U, M, A, S_c, Vn, dS_{c+1}, dVn) and outputs, float32
inputs already normalised (the GatedDeltaRule contract), ragged lengths."""
import pytest
import torch

import _parity

from oracle import gdr

from _gpu import passes

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk", "dv", "dg", "dbeta", "ds0")


@pytest.mark.parametrize("shape", [(1, 64, 1, 128, 128), (2, 100, 3, 64, 64), (1, 37, 2, 128, 64), (1, 130, 2, 32, 96)])
def test_passes_fp32(shape):
    B, T, H, DK, DV = shape
    print(f"case passes_fp32 {shape}", flush=True)
    q, k, v, g, b, s0 = gdr.harness_inputs(B, T, H, DK, DV, seed=3)
    gen = torch.Generator().manual_seed(9)
    do = torch.randn(B, T, H, DV, generator=gen, dtype=torch.float64)
    dsT = torch.randn(B, H, DK, DV, generator=gen, dtype=torch.float64)
    o, sT, P = gdr.chunked_forward(q, k, v, g, b, s0)
    grads, P = gdr.chunked_backward(q, k, v, g, b, s0, do, dsT, P=P)
    dev = "cuda"
    args = [x.float().to(dev).contiguous() for x in (q, k, v, g, b, s0, do, dsT)]
    r = passes(*args)
    ref = dict(W=P["W"], U=P["U"], M=P["M"], A=P["A"], Sc=P["Sc"], Vn=P["Vn"], dSn=P["dSn"], dVn=P["dVn"], o=o, sT=sT,
               Ke=P["e"][..., None] * P["K"], Qg=P["gam"][..., None] * P["Q"], GL=P["gam"][..., -1])
    ref.update(dict(zip(NAMES, grads)))
    assert r["W2_equal"], "the forward- and backward-mode preps must give the same bits"
    assert r["store_equal"], "the output pass storing the states must give the output and recompute passes' bits"
    _parity.check({n: gdr.rel(r[n], ref[n]) for n in ref}, 2e-4)


@pytest.mark.parametrize("shape", [(1, 64, 1, 128, 128), (2, 100, 3, 64, 64), (1, 37, 2, 128, 64), (1, 130, 2, 32, 96),
                                   (1, 200, 2, 128, 32), (2, 256, 2, 128, 128), (1, 77, 1, 64, 128)])
def test_passes_bf16(shape):
    """bf16 operands (the bf16 per-chunk backward is its own 8-wave kernel): outputs and every gradient against float64
    of the same bf16 values, at the bf16 bar 1e-2; inputs already normalised, ragged lengths, every key/value width
    class of the backward."""
    B, T, H, DK, DV = shape
    print(f"case passes_bf16 {shape}", flush=True)
    q, k, v, g, b, s0 = gdr.harness_inputs(B, T, H, DK, DV, seed=4)
    gen = torch.Generator().manual_seed(10)
    do = torch.randn(B, T, H, DV, generator=gen, dtype=torch.float64)
    dsT = torch.randn(B, H, DK, DV, generator=gen, dtype=torch.float64)
    rb = lambda x: x.to(torch.bfloat16).double()
    rf = lambda x: x.float().double()
    q, k, v, do = rb(q), rb(k), rb(v), rb(do)
    g, b, s0, dsT = rf(g), rf(b), rf(s0), rf(dsT)
    o, sT, P = gdr.chunked_forward(q, k, v, g, b, s0)
    grads, _ = gdr.chunked_backward(q, k, v, g, b, s0, do, dsT, P=P)
    dev = "cuda"
    bf = lambda x: x.to(dev, torch.bfloat16).contiguous()
    f32 = lambda x: x.to(dev, torch.float32).contiguous()
    r = passes(bf(q), bf(k), bf(v), f32(g), f32(b), f32(s0), bf(do), f32(dsT))
    assert r["W2_equal"] and r["store_equal"]
    ref = dict(o=o, sT=sT, **dict(zip(NAMES, grads)))
    _parity.check({n: gdr.rel(r[n].double(), ref[n]) for n in ref}, 1e-2)


@pytest.mark.parametrize("shape,dtype,split", [((2, 150, 3, 3, 128, 128), torch.bfloat16, 0),
                                               ((1, 100, 4, 2, 64, 64), torch.float32, 0),
                                               ((4, 1024, 16, 16, 128, 128), torch.bfloat16, 0),
                                               ((2, 77, 2, 2, 128, 96), torch.bfloat16, 3)])
def test_one_call_forward_equals_the_two_passes(shape, dtype, split):
    """macai_gdr_forward (prep and the output pass in one call, operands in a caller's workspace) gives the bits of
    macai_gdr_prep + macai_gdr_state_fwd with the drop-in's own split, and of the drop-in's no-grad forward."""
    from macai.gated_delta import _native as N
    from macai.gated_delta import chunk_gated_delta_rule, op
    B, T, H, Hk, DK, DV = shape
    print("case one-call forward", shape, dtype, split, flush=True)
    inp = gdr.make_inputs(B, T, Hk, H, DK, DV, dtype, s0=True, seed=31)
    q, k = (inp[n][:, :, ::H // Hk].contiguous().cuda() for n in ("query", "key"))
    v, g, beta, s0 = (inp[n].cuda() for n in ("value", "g", "beta", "initial_state"))
    code, st, P = N.dtype_code(dtype), N.stream_of(q), N.ptr
    nbytes = N.lib().macai_gdr_forward_workspace(B, T, H, DK, DV, code, 0)
    ws = torch.full((nbytes,), 255, dtype=torch.uint8, device="cuda")
    o = torch.full((B, T, H, DV), float("nan"), dtype=dtype, device="cuda")
    sT = torch.full((B, H, DK, DV), float("nan"), device="cuda")
    use = split or op.split_for(B * H, T, DV)
    N.call("macai_gdr_forward", P(q), P(k), P(v), P(g), P(beta), P(s0), P(o), P(sT), P(ws), nbytes, B, T, H, Hk, DK,
           DV, code, 1, DK ** -0.5, split, None, 0, st)
    old = op.VALUE_SPLIT
    try:
        op.VALUE_SPLIT = use
        with torch.no_grad():
            ro, rsT = chunk_gated_delta_rule(q, k, v, g, beta, initial_state=s0, output_final_state=True,
                                             use_qk_l2norm_in_kernel=True)
    finally:
        op.VALUE_SPLIT = old
    torch.cuda.synchronize()
    assert torch.equal(o, ro) and torch.equal(sT, rsT)


# ---- sequence parallelism: segment maps, their composition, the segmented forward -------------------------------------
@pytest.mark.parametrize("dtype,T,P,DK,DV", [(torch.float32, 64 * 13 + 5, 3, 128, 128),
                                             (torch.bfloat16, 64 * 9, 2, 128, 128), (torch.float32, 64 * 8, 8, 128, 128),
                                             (torch.float32, 64 * 6 + 9, 3, 256, 128), (torch.bfloat16, 64 * 7, 2, 64, 64),
                                             (torch.float32, 64 * 12 + 3, 5, 32, 64), (torch.bfloat16, 64 * 8, 4, 64, 128)])
def test_segment_maps_and_scan(dtype, T, P, DK, DV):
    """macai_gdr_state_map on a row split into P segments of whole chunks (the last one ragged) against the oracle's
    segment_map of each segment, and macai_gdr_state_scan's starting states against the oracle's chunk states at the
    segment boundaries.  float32 at the harness bar 2e-4 (relative to the largest entry of each map), bf16 at 1e-2.
    Key heads of 256 (float32) take the map pass's direct form (the chunk's tiles read from memory, not LDS) and the
    scan's form that reads each map from memory; below 256 the scan's MFMA steps run on 2, 4 or 8 row tiles."""
    from macai.gated_delta import _native as N
    from macai.gated_delta import op
    print(f"case segment maps {dtype} T={T} P={P} DK={DK} DV={DV}", flush=True)
    H = 2
    q, k, v, g, b, s0 = gdr.harness_inputs(1, T, H, DK, DV, seed=5)
    g = g * 0.02          # weak decay: A stays O(1) over a segment (under the harness's g it underflows float32)
    rd = (lambda x: x.to(torch.bfloat16).double()) if dtype == torch.bfloat16 else (lambda x: x.float().double())
    q, k, v = rd(q), rd(k), rd(v)
    g, b, s0 = g.float().double(), b.float().double(), s0.float().double()
    _, _, Pr = gdr.chunked_forward(q, k, v, g, b, s0)
    dev, f32 = "cuda", torch.float32
    x = [t.to(dev, dtype).contiguous() for t in (q, k, v)] + [t.to(dev, f32).contiguous() for t in (g, b, s0)]
    NT = -(-T // 64)
    es = 2 if dtype == torch.bfloat16 else 4
    e = lambda *s, d=dtype: torch.empty(*s, device=dev, dtype=d)
    W, U, Ke, GL, Qg, M = e(1, H, NT, 64, DK), e(1, H, NT, 64, DV, d=f32), e(1, H, NT, 64, DK), e(1, H, NT, d=f32), \
        e(1, H, NT, 64, DK), e(1, H, NT, 64, 64)
    code, st, Pt = N.dtype_code(dtype), N.stream_of(x[0]), N.ptr
    N.call("macai_gdr_prep", *map(Pt, x[:5]), Pt(W), Pt(U), Pt(Ke), Pt(GL), Pt(Qg), Pt(M), None, 1, T, H, H, DK, DV,
           code, 0, 1.0, None, 0, st)
    table, NT2 = op._segment_table(T, P, dev)
    assert NT2 == NT
    maps = e(P, H, DK, DK + DV, d=f32)
    N.call("macai_gdr_state_map", Pt(W), Pt(U), Pt(Ke), Pt(GL), Pt(maps), P, T, H, DK, DV, code, 0, Pt(table), NT, st)
    starts = e(P, H, DK, DV, d=f32)
    N.call("macai_gdr_state_scan", Pt(maps), Pt(x[5]), Pt(starts), 1, P, H, DK, DV, st)
    torch.cuda.synchronize()
    maps, starts = maps.cpu(), starts.cpu()
    c0 = table.cpu().tolist()[2 * NT:]
    bar = 1e-2 if dtype == torch.bfloat16 else 2e-4
    errs = {}
    for s in range(P):
        t0, t1 = 64 * c0[s], min(64 * c0[s + 1], T)
        A, Bm = gdr.segment_map(q[:, t0:t1], k[:, t0:t1], v[:, t0:t1], g[:, t0:t1], b[:, t0:t1])
        errs[f"A{s}"] = gdr.rel(maps[s:s + 1, :, :, :DK], A)
        errs[f"B{s}"] = gdr.rel(maps[s:s + 1, :, :, DK:], Bm)
        errs[f"start{s}"] = gdr.rel(starts[s:s + 1], Pr["Sc"][:, :, c0[s]])
    _parity.check(errs, bar)


@pytest.mark.parametrize("dtype,P,DK", [(torch.float32, 2, 128), (torch.float32, 4, 128), (torch.bfloat16, 2, 128),
                                        (torch.bfloat16, 4, 128), (torch.bfloat16, 2, 256)])
def test_segmented_forward(dtype, P, DK):
    """A single row's forward without gradients split into P segments (op.SEQUENCE_SPLIT, taken when nothing is saved
    for a backward): output and final state against the float64 oracle, float32 at 2e-4 and bf16 at 1e-2; the passes
    run are the segmented ones; with a starting state and a ragged length; key heads of 256 (bf16 inputs upcast to the
    float32 kernels).  The decay is weak (g scaled by 0.02), so each segment's output depends on the state carried
    into it: under the generator's own decay a state is forgotten within a chunk or two and a wrong starting state
    would go unseen."""
    from macai.gated_delta import chunk_gated_delta_rule, op
    print(f"case segmented forward {dtype} P={P} DK={DK}", flush=True)
    inp = gdr.make_inputs(1, 64 * 40 + 17, 4, 4, DK, 128, dtype, s0=True, seed=12)
    inp["g"] = inp["g"] * 0.02
    names = ("query", "key", "value", "g", "beta")
    old = op.SEQUENCE_SPLIT
    before = dict(op.CALLS)
    try:
        op.SEQUENCE_SPLIT = P
        with torch.no_grad():
            o, sT = chunk_gated_delta_rule(*(inp[n].to("cuda") for n in names),
                                           initial_state=inp["initial_state"].to("cuda"), output_final_state=True,
                                           use_qk_l2norm_in_kernel=True)
            torch.cuda.synchronize()
    finally:
        op.SEQUENCE_SPLIT = old
    ran = [k_ for k_, v_ in op.CALLS.items() if v_ != before.get(k_, 0)]
    assert len(ran) == 1 and ran[0].startswith(f"fwd seg{P} "), ran
    ro, rsT, _ = gdr.dropin_f64(*(inp[n] for n in names + ("initial_state",)))
    bar = 1e-2 if dtype == torch.bfloat16 else 2e-4
    _parity.check({"o": gdr.rel(o.cpu(), ro), "sT": gdr.rel(sT.cpu(), rsT)}, bar)

"""Each HIP pass against the float64 oracle's intermediates (W, U, M, A, S_c, Vn, dS_{c+1}, dVn) and outputs, float32
inputs already normalised (the GatedDeltaRule contract), ragged lengths."""
import pytest
import torch

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
    errs = {n: gdr.rel(r[n], ref[n]) for n in ref}
    print(errs)
    bad = {n: e for n, e in errs.items() if not e < 2e-4}
    assert not bad, bad


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
    errs = {n: gdr.rel(r[n].double(), ref[n]) for n in ref}
    print(errs)
    bad = {n: e for n, e in errs.items() if not e < 1e-2}
    assert not bad, bad

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
    tr = lambda x: x.transpose(-1, -2)
    ref = dict(W=P["W"], U=P["U"], M=P["M"], Mt=tr(P["M"]), A=P["A"], At=tr(P["A"]), Sc=P["Sc"], Vn=P["Vn"],
               dSn=P["dSn"], dVn=P["dVn"], o=o, sT=sT, KeT=tr(P["e"][..., None] * P["K"]),
               Ke=P["e"][..., None] * P["K"], Qg=P["gam"][..., None] * P["Q"], QgT=tr(P["gam"][..., None] * P["Q"]),
               WT=tr(P["W"]), GL=P["gam"][..., -1])
    ref.update(dict(zip(NAMES, grads)))
    assert r["W2_equal"], "the forward- and backward-mode preps must give the same W and KeT bits"
    errs = {n: gdr.rel(r[n], ref[n]) for n in ref}
    print(errs)
    bad = {n: e for n, e in errs.items() if not e < 2e-4}
    assert not bad, bad

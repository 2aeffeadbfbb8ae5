"""GPU parity of grouped value heads (Hk key heads < H value heads, q and k not repeated): the layout of Qwen3.5 /
Qwen3-Next, whose layer repeats q and k over each group before the rule (transformers modeling_qwen3_5.py:500-502;
reference layer/_qwen3_5.py:155-157).  Value head h reads key head h // (H // Hk); dq and dk are the sums over each
group of the per-value-head gradients.

Reference values: the float64 oracle on the repeated q, k (gdr.make_inputs draws q, k per key head and repeats them),
its dquery / dkey summed over each group (the backward of repeat_interleave).  Bars: bf16 1e-2; fp32 2e-4 (the
GatedDeltaRule harness bar).  The grouped forward must equal the repeated one bit for bit: every value head reads the
same q, k values either way.
"""
import pytest
import torch

import _parity

from macai.gated_delta import chunk_gated_delta_rule, op, recurrent_gated_delta_rule
from oracle import gdr

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("dquery", "dkey", "dvalue", "dg", "dbeta", "dstate")


@pytest.fixture(autouse=True)
def _bf16_backward(monkeypatch):
    """The backward with the final state's gradient stays on the bf16 kernels (op.BF16_STATE_GRAD), and so do rows
    shorter than op.BF16_MIN_TOKENS: these tests pin the bf16 kernels' grouped-head forms (by default such calls run
    the float32 kernels)."""
    monkeypatch.setattr(op, "BF16_STATE_GRAD", True)
    monkeypatch.setattr(op, "BF16_MIN_TOKENS", 0)


def _say(*a):
    print(*a, flush=True)


def _grouped(inp, G):
    """The inputs with q, k reduced to their key heads (every G-th head of the repeated tensors)."""
    out = dict(inp)
    out["query"], out["key"] = inp["query"][:, :, ::G].contiguous(), inp["key"][:, :, ::G].contiguous()
    return out


def _run(inp, dsT):
    names = ("query", "key", "value", "g", "beta")
    leaves = [inp[n].to(DEV).requires_grad_(True) for n in names]
    s0 = inp["initial_state"].to(DEV).requires_grad_(True)
    o, sT = chunk_gated_delta_rule(*leaves, initial_state=s0, output_final_state=True, use_qk_l2norm_in_kernel=True)
    torch.autograd.backward([o, sT], [inp["do"].to(DEV), dsT.to(DEV)])
    torch.cuda.synchronize()
    return o.detach().cpu(), sT.detach().cpu(), {n: x.grad.cpu() for n, x in zip(NAMES, leaves + [s0])}


@pytest.mark.parametrize("shape,dtype", [((1, 100, 2, 4, 128, 128), torch.bfloat16),
                                         ((2, 77, 1, 3, 64, 64), torch.bfloat16),
                                         ((1, 130, 2, 8, 128, 64), torch.bfloat16),
                                         ((1, 90, 2, 4, 64, 128), torch.float32)])
def test_grouped_heads_fwd_bwd(shape, dtype):
    B, T, Hk, Hv, DK, DV = shape
    G = Hv // Hk
    _say("case", shape, dtype)
    inp = gdr.make_inputs(B, T, Hk, Hv, DK, DV, dtype, s0=True, seed=21)
    dsT = torch.randn(B, Hv, DK, DV, generator=torch.Generator().manual_seed(22))
    ro, rsT, rg = gdr.dropin_f64(*(inp[n] for n in ("query", "key", "value", "g", "beta", "initial_state")),
                                 do=inp["do"], dsT=dsT)
    rg = dict(rg)
    for n in ("dquery", "dkey"):                      # the backward of the repeat: sum over each group
        rg[n] = rg[n].view(B, T, Hk, G, DK).sum(3)
    o, sT, g = _run(_grouped(inp, G), dsT)
    assert g["dquery"].shape == (B, T, Hk, DK) and g["dkey"].shape == (B, T, Hk, DK)
    errs = {"o": gdr.rel(o, ro), "sT": gdr.rel(sT, rsT)}
    errs.update({n: gdr.rel(g[n], rg[n]) for n in NAMES})
    _say("errors:", {k: f"{v:.2e}" for k, v in errs.items()})
    _parity.check(errs, 1e-2 if dtype == torch.bfloat16 else 2e-4)
    # the forward reads the same q, k values as the repeated layout: the same bits
    o_rep, sT_rep, _ = _run(inp, dsT)
    assert torch.equal(o, o_rep) and torch.equal(sT, sT_rep)


def test_grouped_decode_step():
    """One decode step with Hk = 16 key heads for 32 value heads (config 4's layout, unrepeated) equals the step on the
    repeated q, k bit for bit."""
    _say("case grouped decode")
    inp = gdr.config_inputs(4)
    Hv, Hk = inp["value"].shape[2], 16
    names = ("query", "key", "value", "g", "beta")
    args = [inp[n].to(DEV) for n in names]
    grouped = [args[0][:, :, ::Hv // Hk].contiguous(), args[1][:, :, ::Hv // Hk].contiguous()] + args[2:]
    s0 = inp["initial_state"].to(DEV)
    with torch.no_grad():
        o1, s1 = recurrent_gated_delta_rule(*args, initial_state=s0, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
        o2, s2 = recurrent_gated_delta_rule(*grouped, initial_state=s0, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
        torch.cuda.synchronize()
    assert torch.equal(o1.cpu(), o2.cpu()) and torch.equal(s1.cpu(), s2.cpu())


def test_group_sum_is_the_repeat_backward():
    """macai_gdr_group_sum against the autograd backward of repeat_interleave (float32: exact sums in head order)."""
    from macai.gated_delta import _native as N
    B, T, H, Hk, D = 2, 33, 12, 3, 128
    x = torch.randn(B, T, H, D, device=DEV)
    y = torch.empty(B, T, Hk, D, device=DEV)
    N.call("macai_gdr_group_sum", N.ptr(x), N.ptr(y), B, T, H, Hk, D, N.F32, N.stream_of(x))
    ref = x.view(B, T, Hk, H // Hk, D).sum(3)
    torch.cuda.synchronize()
    assert torch.allclose(y, ref, rtol=1e-6, atol=1e-6)

"""GPU parity of the state chain across many chunks, forward and backward (tests/_chain.py: the cases, their weak
decay and their float64 oracle).

Each case runs at least 16 chunks a sequence with a starting state and an upstream gradient of the final state, at a
decay under which the carried state S_c and the carried gradient dS_{c+1} reach every chunk's output and gradients.
So these tests see the chain itself: the forward's S <- exp(G_last) S + K^T diag(e) Vn (reference
_chunked.py:643-653) in state_out / state_fwd, the STORE path that feeds the backward, state_pair's two halves and the
stored mode's state_bwd (dS <- exp(G_last) dS + ..., _chunked.py:886-898), chunk_bwd's use of S_c and dS_{c+1} from
deep in the chain, the grouped-head and packed-row forms, and config 3's segment maps and scan over 8 segments.
tests/test_oracle.py::test_chain_cases_catch_planted_mistakes shows on the CPU that a carried decay of gamma_last^2,
or G_last taken one row early, in either chain moves these very cases past these bars.

Bars: bf16 inputs 1e-2 (the north star's); float32 inputs 2x the reference torch path's own float32 error against
float64 on the same inputs (transformers' algorithm in float32, autograd backward), each the largest over the case's
four draws: one draw's float32 error (a few units in the last place) varies up to a few times between seeds.
"""
import functools

import pytest
import torch

import _chain
import _parity
from macai.gated_delta import chunk_gated_delta_rule, op
from oracle import gdr

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _say(*a):
    print(*a, flush=True)


@pytest.fixture(autouse=True)
def _bf16_backward(monkeypatch):
    """The bf16 cases keep the backward with the final state's gradient on the bf16 kernels (op.BF16_STATE_GRAD; by
    default it runs the float32 kernels): their chains are what these tests pin."""
    monkeypatch.setattr(op, "BF16_STATE_GRAD", True)


@functools.lru_cache(maxsize=None)
def _case(name, seed=None):
    inp = _chain.inputs(name, seed)
    return inp, _chain.oracle(name, inp)


def _run(inp):
    """The drop-in forward + backward on the GPU; returns {o, sT, the six gradients} on the CPU."""
    leaves = [inp[n].to(DEV).requires_grad_(True) for n in _chain.NAMES]
    s0 = inp["initial_state"].to(DEV).requires_grad_(True)
    kw = {} if inp["cu"] is None else {"cu_seqlens": inp["cu"].to(DEV)}
    o, sT = chunk_gated_delta_rule(*leaves, initial_state=s0, output_final_state=True, use_qk_l2norm_in_kernel=True,
                                   **kw)
    torch.autograd.backward([o, sT], [inp["do"].to(DEV), inp["dsT"].to(DEV)])
    torch.cuda.synchronize()
    out = {"o": o.detach().cpu(), "sT": sT.detach().cpu()}
    out.update({n: x.grad.cpu() for n, x in zip(_chain.GRADS, leaves + [s0])})
    return out


def _torch_path_errors(inp, ref):
    """The reference torch path's float32 errors against float64 (the anchor of the float32 bar): transformers'
    algorithm in float32 with an autograd backward, on the same inputs (dense cases)."""
    rep = inp["value"].shape[2] // inp["query"].shape[2]
    leaves = [inp[n].float().clone().requires_grad_(True) for n in _chain.NAMES]
    s0 = inp["initial_state"].clone().requires_grad_(True)
    q, k = (x.repeat_interleave(rep, 2) if rep > 1 else x for x in leaves[:2])
    o, sT = gdr.torch_chunk_gated_delta_rule(q, k, *leaves[2:], initial_state=s0, output_final_state=True,
                                             use_qk_l2norm_in_kernel=True, inverse="solve")
    torch.autograd.backward([o, sT], [inp["do"].float(), inp["dsT"]])
    got = {"o": o, "sT": sT}
    got.update({n: x.grad for n, x in zip(_chain.GRADS, leaves + [s0])})
    return _chain.errors(got, ref)


# the passes the config-1 shape runs in each mode (the pair pass at split 2 = four column waves a workgroup)
CONFIG1_CALLS = {True: {"fwd s4": 1, "bwd pair s2": 1}, False: {"fwd s4": 1, "bwd reverse s4": 1}}


@pytest.mark.parametrize("recompute", [True, False], ids=["recompute", "stored"])
@pytest.mark.parametrize("name", ["config1_bf16", "fp32", "grouped_bf16", "packed_bf16"])
def test_chain_fwd_bwd(name, recompute):
    fp32 = _chain.CASES[name]["dtype"] == torch.float32
    errs, anchor = {}, {}
    for seed in _chain.seeds(name):
        _say(f"case chain {name} seed={seed} recompute={recompute}")
        inp, ref = _case(name, seed)
        old, before = op.RECOMPUTE_STATES, dict(op.CALLS)
        try:
            op.RECOMPUTE_STATES = recompute
            got = _run(inp)
        finally:
            op.RECOMPUTE_STATES = old
        ran = {k: v - before.get(k, 0) for k, v in op.CALLS.items() if v != before.get(k, 0)}
        _say("passes run:", ran)
        if name == "config1_bf16":
            assert ran == CONFIG1_CALLS[recompute], ran
        e = _chain.errors(got, ref)
        _say("errors:", {k: f"{v:.2e}" for k, v in e.items()})
        errs = {n: max(errs.get(n, 0.0), x) for n, x in e.items()}
        if fp32:
            a = _torch_path_errors(inp, ref)
            _say("torch-path fp32 errors:", {k: f"{v:.2e}" for k, v in a.items()})
            anchor = {n: max(anchor.get(n, 0.0), x) for n, x in a.items()}
    bars = {n: 2 * anchor[n] for n in errs} if fp32 else _chain.BF16_BAR
    _parity.check(errs, bars, recompute=recompute, decay=_chain.DECAY)


@pytest.mark.parametrize("split", ["auto", 1])
def test_chain_config3_prefill(split):
    """Config 3 (one row of 32,768 tokens, 512 chunks, Hv = 16): the default 8 segments (segment maps, their
    composition, the output pass from each segment's start) and the plain chain (SEQUENCE_SPLIT = 1)."""
    _say(f"case chain config3 split={split}")
    name = "config3_bf16"
    inp, ref = _case(name)
    old, before = op.SEQUENCE_SPLIT, dict(op.CALLS)
    try:
        op.SEQUENCE_SPLIT = split
        with torch.no_grad():
            o, sT = chunk_gated_delta_rule(*(inp[n].to(DEV) for n in _chain.NAMES), output_final_state=True,
                                           use_qk_l2norm_in_kernel=True)
            torch.cuda.synchronize()
    finally:
        op.SEQUENCE_SPLIT = old
    ran = [k_ for k_, v_ in op.CALLS.items() if v_ != before.get(k_, 0)]
    _say("passes run:", ran)
    assert len(ran) == 1 and ran[0].startswith("fwd seg8 " if split == "auto" else "fwd s"), ran
    _parity.check(_chain.errors({"o": o.cpu(), "sT": sT.cpu()}, ref), _chain.BF16_BAR, decay=_chain.DECAY)

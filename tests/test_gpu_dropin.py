"""GPU parity of the drop-in and the autograd contract against the float64 oracle (reference tests/test_harness.py,
test_gated_delta.py, test_chunking.py, test_layer.py:48-85 patterns).

Bars (error = max|a - r| / max|r| per tensor, r = float64 on the same dtype-representable values):
  * float32 inputs through the drop-in: every output and gradient <= 2 x the reference torch path's own float32 error
    (transformers' algorithm in float32 on the CPU, oracle.torch_chunk_gated_delta_rule) -- the north-star bar;
  * bfloat16 inputs: every output and gradient <= 1e-2 (the north star; the reference's own bf16 bar was 2e-2);
  * the GatedDeltaRule contract on the harness cases: 2e-4, stress and nearly parallel keys 5e-4, long 1e-3
    (reference tests/test_harness.py:34-97).
"""
import pytest
import torch

import _parity
from macai.gated_delta import GatedDeltaRule, chunk_gated_delta_rule, op, recurrent_gated_delta_rule
from oracle import gdr

pytestmark = pytest.mark.gpu
DEV = "cuda"
NAMES = ("dquery", "dkey", "dvalue", "dg", "dbeta", "dstate")
BF16_BAR = 1e-2


def _say(*a):
    print(*a, flush=True)


def run_dropin(inp, grads=True, dsT=None, final=True, l2norm=True):
    """The drop-in on the GPU from the CPU inputs dict; returns (o, sT, grads dict) on the CPU."""
    names = ("query", "key", "value", "g", "beta")
    leaves = [inp[n].to(DEV).requires_grad_(grads) for n in names]
    s0 = inp["initial_state"]
    if s0 is not None:
        s0 = s0.to(DEV).requires_grad_(grads)
    o, sT = chunk_gated_delta_rule(*leaves, initial_state=s0, output_final_state=final,
                                   use_qk_l2norm_in_kernel=l2norm)
    assert o.dtype == inp["query"].dtype and (sT is None or sT.dtype == torch.float32)
    g = {}
    if grads:
        outs, gos = [o], [inp["do"].to(DEV)]
        if dsT is not None:
            outs.append(sT)
            gos.append(dsT.to(DEV))
        torch.autograd.backward(outs, gos)
        for n, x in zip(NAMES, leaves + ([s0] if s0 is not None else [])):
            g[n] = x.grad.cpu()
    torch.cuda.synchronize()
    return o.detach().cpu(), (None if sT is None else sT.detach().cpu()), g


def torch_path_errors(inp, ro, rsT, rg, dsT=None, l2norm=True):
    """The reference torch path's own float32 errors against float64 (the anchor of the 2x bar)."""
    names = ("query", "key", "value", "g", "beta")
    leaves = [inp[n].float().clone().requires_grad_(True) for n in names]
    s0 = inp["initial_state"]
    if s0 is not None:
        s0 = s0.clone().requires_grad_(True)
    o, sT = gdr.torch_chunk_gated_delta_rule(*leaves, initial_state=s0, output_final_state=True,
                                             use_qk_l2norm_in_kernel=l2norm, inverse="solve")
    outs, gos = [o], [inp["do"].float()]
    if dsT is not None:
        outs.append(sT)
        gos.append(dsT)
    torch.autograd.backward(outs, gos)
    e = {"o": gdr.rel(o, ro), "sT": gdr.rel(sT, rsT)}
    for n, x in zip(NAMES, leaves + ([s0] if s0 is not None else [])):
        e[n] = gdr.rel(x.grad, rg[n])
    return e


def check_dropin(inp, bar=None, anchor=False, dsT=None, grads=True, l2norm=True):
    ro, rsT, rg = gdr.dropin_f64(*(inp[n] for n in ("query", "key", "value", "g", "beta", "initial_state")),
                                 do=inp["do"] if grads else None, dsT=dsT, use_qk_l2norm_in_kernel=l2norm)
    o, sT, g = run_dropin(inp, grads=grads, dsT=dsT, l2norm=l2norm)
    errs = {"o": gdr.rel(o, ro), "sT": gdr.rel(sT, rsT)}
    for n, x in g.items():
        errs[n] = gdr.rel(x, rg[n])
    bars = {n: bar for n in errs}
    if anchor:
        ref = torch_path_errors(inp, ro, rsT, rg, dsT, l2norm)
        bars = {n: 2 * ref[n] for n in errs}
        _say("torch-path fp32 errors:", {k: f"{v:.2e}" for k, v in ref.items()})
    _parity.check(errs, bars, recompute=op.RECOMPUTE_STATES)
    return errs


# ---- BASELINE configs ------------------------------------------------------------------------------------------------
def test_config0_fp32_forward():
    """Config 0: fp32, forward only, o and sT within 2x the torch path's fp32 error."""
    _say("case config0")
    inp = gdr.config_inputs(0)
    ro, rsT, _ = gdr.dropin_f64(*(inp[n] for n in ("query", "key", "value", "g", "beta", "initial_state")))
    with torch.no_grad():
        o, sT, _ = run_dropin(inp, grads=False)
        to, tsT = gdr.torch_chunk_gated_delta_rule(*(inp[n] for n in ("query", "key", "value", "g", "beta")),
                                                   output_final_state=True, use_qk_l2norm_in_kernel=True)
    _parity.check({"o": gdr.rel(o, ro), "sT": gdr.rel(sT, rsT)},
                  {"o": 2 * gdr.rel(to, ro), "sT": 2 * gdr.rel(tsT, rsT)})


@pytest.mark.parametrize("recompute", [True, False], ids=["recompute", "stored"])
@pytest.mark.parametrize("cfg", [1, 2])
def test_config_bf16_fwd_bwd(cfg, recompute, monkeypatch):
    """Configs 1 and 2 at full size: bf16 q/k/v/dO, fp32 g/beta (config 2: Hk=16 repeated to Hv=32, an initial state
    and its gradient, the final state used, its backward kept on the bf16 kernels by op.BF16_STATE_GRAD): every output
    and gradient within 1e-2.  recompute: the backward reruns
    prep and recomputes the chunk states beside its reverse pass in one launch (the reference's default and BASELINE
    config 1's form; at config 1's 64 head-rows that is macai_gdr_state_pair at split 2, four column waves a
    workgroup); stored: the forward keeps them."""
    _say(f"case config{cfg} recompute={recompute}")
    monkeypatch.setattr(op, "BF16_STATE_GRAD", True)
    inp = gdr.config_inputs(cfg)
    dsT = torch.randn(inp["value"].shape[0], inp["value"].shape[2], 128, 128,
                      generator=torch.Generator().manual_seed(77)) if cfg == 2 else None
    old, before = op.RECOMPUTE_STATES, dict(op.CALLS)
    try:
        op.RECOMPUTE_STATES = recompute
        check_dropin(inp, bar=BF16_BAR, dsT=dsT)
    finally:
        op.RECOMPUTE_STATES = old
    ran = {k: v - before.get(k, 0) for k, v in op.CALLS.items() if v != before.get(k, 0)}
    _say("passes run:", ran)
    if cfg == 1:
        assert ran == ({"fwd s4": 1, "bwd pair s2": 1} if recompute else {"fwd s4": 1, "bwd reverse s4": 1}), ran


@pytest.mark.parametrize("split", ["auto", 1])
@pytest.mark.parametrize("Hv", [16, 32])
def test_config3_long_prefill_forward(Hv, split):
    """Config 3: one row of 32,768 tokens (512 sequential chunks), bf16, forward only, the final state returned; as
    segments side by side (the default at Hv = 16: 8 of them) and as one chain (SEQUENCE_SPLIT = 1, and the default
    at Hv = 32, whose plain pass already fills the chip)."""
    _say(f"case config3 Hv={Hv} split={split}")
    inp = gdr.config_inputs(3, Hv=Hv)
    names = ("query", "key", "value", "g", "beta")
    old = op.SEQUENCE_SPLIT
    before = dict(op.CALLS)
    try:
        op.SEQUENCE_SPLIT = split
        with torch.no_grad():
            o, sT = chunk_gated_delta_rule(*(inp[n].to(DEV) for n in names), output_final_state=True,
                                           use_qk_l2norm_in_kernel=True)
            torch.cuda.synchronize()
    finally:
        op.SEQUENCE_SPLIT = old
    ran = [k_ for k_, v_ in op.CALLS.items() if v_ != before.get(k_, 0)]
    seg = split == "auto" and Hv == 16
    assert len(ran) == 1 and ran[0].startswith("fwd seg8 " if seg else "fwd s"), ran
    assert seg or not ran[0].startswith("fwd seg"), ran
    q, k = gdr.prologue(inp["query"].double(), inp["key"].double())
    ro, rsT = gdr.chunked_forward_segments(q, k, inp["value"].double(), inp["g"].double(), inp["beta"].double(),
                                           torch.zeros(1, Hv, 128, 128, dtype=torch.float64))
    _parity.check({"o": gdr.rel(o.cpu(), ro), "sT": gdr.rel(sT.cpu(), rsT)}, BF16_BAR,
                  value_split=op.split_for(Hv, 32768, 128))


def test_config4_decode_step():
    """Config 4: one decode step per sequence (64 x 32 heads, fp32 state) through the recurrent drop-in, against the
    oracle's one-step recurrence; the state's error is small enough to also hold at the fp32 2e-4 bar."""
    _say("case config4")
    inp = gdr.config_inputs(4)
    names = ("query", "key", "value", "g", "beta")
    with torch.no_grad():
        o, sT = recurrent_gated_delta_rule(*(inp[n].to(DEV) for n in names), initial_state=inp["initial_state"].to(DEV),
                                           output_final_state=True, use_qk_l2norm_in_kernel=True)
        torch.cuda.synchronize()
    q, k = gdr.prologue(inp["query"].double(), inp["key"].double())
    ro, rs = gdr.decode_step(q[:, 0], k[:, 0], inp["value"].double()[:, 0], inp["g"].double()[:, 0],
                             inp["beta"].double()[:, 0], inp["initial_state"].double())
    assert o.dtype == torch.bfloat16
    _parity.check({"o": gdr.rel(o.cpu()[:, 0], ro), "sT": gdr.rel(sT.cpu(), rs)}, {"o": BF16_BAR, "sT": 2e-4})


# ---- float32 drop-in at the north-star bar ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape,s0", [((2, 100, 4, 128), True), ((1, 256, 4, 64), False), ((2, 512, 16, 128), False),
                                      ((1, 45, 3, 128), True)])
def test_dropin_fp32_within_twice_the_torch_path(shape, s0):
    """Every output and gradient (final-state gradient included) <= 2 x the torch path's own fp32 error vs float64
    (reference tests/test_gated_delta.py:37-56 shape first; test_layer.py:48-85 bar)."""
    B, T, H, D = shape
    _say(f"case dropin_fp32 {shape} s0={s0}")
    inp = gdr.make_inputs(B, T, H, H, D, D, torch.float32, s0=s0, seed=1)
    dsT = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9))
    check_dropin(inp, anchor=True, dsT=dsT)


@pytest.mark.parametrize("kernels", ["default", "bf16"])
@pytest.mark.parametrize("shape", [(2, 50, 3, 128), (2, 45, 3, 128), (1, 1, 2, 64), (3, 130, 2, 32), (1, 1, 2, 128),
                                   (1, 2, 2, 128), (2, 1, 3, 128), (2, 2, 3, 128), (1, 3, 1, 128)])
def test_dropin_bf16_small(shape, kernels):
    """bf16 drop-in end to end with a starting state and the final state used (reference test_harness.py:139-166),
    including one- to three-token rows at D = 128, where a chunk has a single valid row or two.  "default": rows
    shorter than op.BF16_MIN_TOKENS run on the float32 kernels, and the backward of the others, which gets
    the final state's gradient, too (op.BF16_STATE_GRAD); "bf16": both switches keep every part on the bf16 kernels,
    whose one- to three-row chunks these draws hold to the bar too."""
    B, T, H, D = shape
    _say(f"case dropin_bf16 {shape} {kernels}")
    inp = gdr.make_inputs(B, T, H, H, D, D, torch.bfloat16, s0=True, seed=8)
    dsT = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9))
    old = op.BF16_MIN_TOKENS, op.BF16_STATE_GRAD
    try:
        if kernels == "bf16":
            op.BF16_MIN_TOKENS, op.BF16_STATE_GRAD = 0, True
        p = op.plan(B, T, H, D, D, True)
        assert p["operands"] == ("f32" if kernels == "default" and T < op.BF16_MIN_TOKENS else "bf16")
        assert p["state_grad_operands"] == ("f32" if kernels == "default" else "bf16")
        check_dropin(inp, bar=BF16_BAR, dsT=dsT)
    finally:
        op.BF16_MIN_TOKENS, op.BF16_STATE_GRAD = old


@pytest.mark.parametrize("shape", [(2, 50, 3, 128), (1, 130, 2, 64)])
def test_dropin_fp16(shape):
    """float16 q, k, v, dO (reference test_harness.py:100-117, bar 5e-3): computed as float32 like the reference (its
    prologue and value.float() upcast them), the output and the gradients of q, k, v returned in float16."""
    B, T, H, D = shape
    _say(f"case dropin_fp16 {shape}")
    inp = gdr.make_inputs(B, T, H, H, D, D, torch.float16, s0=True, seed=4)
    dsT = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9))
    errs = check_dropin(inp, bar=5e-3, dsT=dsT)
    assert errs["o"] < 1e-3        # float32 arithmetic: only the float16 output's rounding remains


@pytest.mark.parametrize("why", ["unnormalized", "short", "one_chunk"])
def test_bf16_calls_on_the_float32_kernels(why):
    """bf16 calls the bf16 operands do not serve run on the float32 kernels: keys the kernels do not normalise
    (use_qk_l2norm_in_kernel=False; raw N(0, 1) keys at DK = 32, 200 tokens, seed 501, a draw on which the bf16
    operands' rounding model misses the bar twelvefold) and rows shorter than op.BF16_MIN_TOKENS (two tokens, seed
    50217: the model's dg 5.7e-2; one chunk, seed 134086: 1.7e-2; tests/test_host.py).  The output and every gradient
    are those of the same values given as float32, cast back, bit for bit, and within 1e-2 of float64."""
    _say(f"case bf16 on the float32 kernels: {why}")
    if why == "unnormalized":
        inp, l2 = gdr.make_inputs(2, 200, 1, 2, 32, 32, torch.bfloat16, s0=True, seed=501), False
        assert op.plan(2, 200, 2, 32, 32, True, l2norm=False)["operands"] == "f32"
    elif why == "short":
        inp, l2 = gdr.make_inputs(1, 2, 1, 1, 32, 32, torch.bfloat16, s0=False, seed=50217), True
        assert op.plan(1, 2, 1, 32, 32, True)["operands"] == "f32"
    else:
        inp, l2 = gdr.make_inputs(1, 64, 2, 2, 64, 128, torch.bfloat16, s0=False, seed=134086), True
        assert op.plan(1, 64, 2, 64, 128, True)["operands"] == "f32"
    check_dropin(inp, bar=BF16_BAR, l2norm=l2)
    f32 = {n: (x.float() if x is not None and x.dtype == torch.bfloat16 else x) for n, x in inp.items()}
    o, sT, g = run_dropin(inp, l2norm=l2)
    o2, sT2, g2 = run_dropin(f32, l2norm=l2)
    assert torch.equal(o, o2.to(o.dtype)) and torch.equal(sT, sT2)
    for n in g:
        assert torch.equal(g[n], g2[n].to(g[n].dtype)), n


@pytest.mark.parametrize("case", ["f32_switch", "raw_keys", "wide_keys", "short_row", "state_grad", "stored",
                                  "kept_prep", "segments"])
def test_mixed_io_changes_no_bits(case, monkeypatch):
    """A bf16 call computed on the float32 kernels hands its bf16 q, k, v to them as they are (op.MIXED_IO: prep and
    the per-chunk backward read them exactly, the state pass writes o and the per-chunk backward dq, dk, dv in bf16,
    one rounding each) instead of upcasting them and casting the results back: the same bits in each route that sends
    a bf16 call to the float32 kernels (BF16_OPERANDS off, raw keys, key width 256, a short row, a final-state
    gradient's backward), in both kept modes and through the segmented forward (which upcasts); packed rows in
    tests/test_gpu_packed.py."""
    _say(f"case mixed io bits {case}")
    bf = torch.bfloat16
    dsT, l2, grads = None, True, True
    inp = gdr.make_inputs(2, 150, 2, 2, 128, 128, bf, s0=True, seed=41)
    if case in ("f32_switch", "stored", "kept_prep"):
        monkeypatch.setattr(op, "BF16_OPERANDS", False)
        if case == "stored":
            monkeypatch.setattr(op, "RECOMPUTE_STATES", False)
        if case == "kept_prep":
            monkeypatch.setattr(op, "KEEP_PREP", True)
    elif case == "raw_keys":
        l2 = False
    elif case == "wide_keys":
        inp = gdr.make_inputs(1, 100, 2, 2, 256, 64, bf, s0=True, seed=42)
    elif case == "short_row":
        inp = gdr.make_inputs(2, 40, 2, 2, 64, 64, bf, s0=True, seed=43)
    elif case == "state_grad":
        dsT = torch.randn(2, 2, 128, 128, generator=torch.Generator().manual_seed(44))
    elif case == "segments":
        monkeypatch.setattr(op, "BF16_OPERANDS", False)
        monkeypatch.setattr(op, "SEQUENCE_SPLIT", 4)
        inp = gdr.make_inputs(1, 64 * 12 + 5, 2, 2, 128, 128, bf, s0=True, seed=45)
        grads = False
    runs = []
    for mixed in (True, False):
        monkeypatch.setattr(op, "MIXED_IO", mixed)
        runs.append(run_dropin(inp, grads=grads, dsT=dsT, l2norm=l2))
    o, sT, g = runs[0]
    o2, sT2, g2 = runs[1]
    assert o.dtype == bf and torch.equal(o, o2) and torch.equal(sT, sT2)
    for n in g:
        assert g[n].dtype == g2[n].dtype and torch.equal(g[n], g2[n]), n


def test_final_state_gradient_backward_on_the_float32_kernels():
    """A bf16 call whose final state receives a gradient runs its backward on the float32 kernels (op.BF16_STATE_GRAD
    off, the default): on a 150-token draw with an N(0, 1) final-state gradient (seed 209), where the bf16 backward's
    dg is 2.4e-2 from float64 (the oracle's rounding model gives the same; tests/test_host.py), every output and
    gradient is within 1e-2, and the gradients are those of the call run wholly on the float32 kernels
    (op.BF16_OPERANDS off) bit for bit, cast to bf16 -- the backward recomputes from the inputs, so only the output o
    keeps the bf16 forward's rounding.  With op.BF16_STATE_GRAD the bf16 backward runs and misses the bar on dg."""
    _say("case final-state gradient backward")
    inp = gdr.make_inputs(1, 150, 2, 2, 128, 128, torch.bfloat16, s0=True, seed=209)
    dsT = torch.randn(1, 2, 128, 128, generator=torch.Generator().manual_seed(216))
    key = "bwd f32 for a final-state gradient"
    before = op.CALLS[key]
    errs = check_dropin(inp, bar=BF16_BAR, dsT=dsT)
    assert op.CALLS[key] == before + 1
    o, sT, g = run_dropin(inp, dsT=dsT)
    old = op.BF16_OPERANDS, op.BF16_STATE_GRAD
    try:
        op.BF16_OPERANDS = False
        o32, sT32, g32 = run_dropin(inp, dsT=dsT)
        op.BF16_OPERANDS, op.BF16_STATE_GRAD = True, True
        before = op.CALLS[key]
        ob, sTb, gb = run_dropin(inp, dsT=dsT)
        assert op.CALLS[key] == before
    finally:
        op.BF16_OPERANDS, op.BF16_STATE_GRAD = old
    for n in g:
        assert torch.equal(g[n], g32[n].to(g[n].dtype)), n
    rg = gdr.dropin_f64(*(inp[n] for n in ("query", "key", "value", "g", "beta", "initial_state")), do=inp["do"],
                        dsT=dsT)[2]
    _say(f"dg with the bf16 backward {gdr.rel(gb['dg'], rg['dg']):.2e}, rerouted {errs['dg']:.2e}")
    assert gdr.rel(gb["dg"], rg["dg"]) > BF16_BAR and errs["dg"] < 1e-3


def test_large_starting_state():
    """A starting state of N(0, 1) entries (what a weakly decaying head carries over a long prefix is of that order):
    every output and gradient within 1e-2.  On this draw (seed 8073) the per-chunk backward's S_c dO^T with S_c rounded
    once to bf16 put dg at 1.5e-2; as a hi + lo pair 3.1e-3 (tests/test_oracle.py::
    test_chunk_state_enters_dq_and_dg_as_a_pair)."""
    _say("case large starting state")
    inp = gdr.make_inputs(1, 150, 2, 2, 32, 128, torch.bfloat16, s0=True, seed=8073)
    inp["initial_state"] = inp["initial_state"] * 50.0
    errs = check_dropin(inp, bar=BF16_BAR)
    assert errs["dg"] < 5e-3, errs["dg"]


def test_calls_without_tokens():
    """B = 0 or T = 0: an empty output, the starting state passed through as the final one (zeros without one) and its
    gradient the final state's, as the reference's torch path returns when it loops over no chunks (transformers
    modeling_qwen3_5.py:248-327); the decode entry the same; no key heads is refused with a ValueError."""
    for B, T in ((2, 0), (0, 5)):
        q, k, v = (torch.randn(B, T, 2, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True) for _ in range(3))
        g = torch.zeros(B, T, 2, device=DEV, requires_grad=True)
        s0 = torch.randn(B, 2, 64, 64, device=DEV, requires_grad=True)
        o, sT = chunk_gated_delta_rule(q, k, v, g, g, initial_state=s0, output_final_state=True,
                                       use_qk_l2norm_in_kernel=True)
        assert o.shape == (B, T, 2, 64) and o.dtype == torch.bfloat16 and torch.equal(sT, s0)
        dsT = torch.randn_like(sT)
        torch.autograd.backward([o, sT], [torch.zeros_like(o), dsT])
        assert torch.equal(s0.grad, dsT)
        o, sT = chunk_gated_delta_rule(q, k, v, g, g, output_final_state=True)
        assert sT.shape == (B, 2, 64, 64) and not sT.any()
        o, sT = recurrent_gated_delta_rule(q, k, v, g, g, initial_state=s0, output_final_state=True)
        assert o.shape == (B, T, 2, 64) and torch.equal(sT, s0)
    q = torch.zeros(1, 3, 0, 64, device=DEV)
    with pytest.raises(ValueError, match="key heads"):
        chunk_gated_delta_rule(q, q, torch.zeros(1, 3, 2, 64, device=DEV), torch.zeros(1, 3, 2, device=DEV),
                               torch.zeros(1, 3, 2, device=DEV))


def _prenormalised(inp):
    """The inputs with query and key already l2-normalised (in float64, then rounded to their dtype): what a caller
    that runs its own prologue passes with use_qk_l2norm_in_kernel=False."""
    out = dict(inp)
    for n in ("query", "key"):
        out[n] = gdr.l2norm(inp[n].double()).to(inp[n].dtype)
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_dropin_unfused_prologue(dtype):
    """use_qk_l2norm_in_kernel=False: no normalisation, only the query's DK^-1/2 scale (reference op.py:279-283), on
    pre-normalised inputs.  bf16: on the bf16 kernels (op.BF16_UNNORMALIZED, which such a caller may set; by default
    these calls take the float32 kernels), the final-state gradient's backward too (op.BF16_STATE_GRAD), every output
    and gradient within 1e-2 on each of four seeds.  float32:
    within 2x the torch path's own float32 error, both taken as the largest over the four seeds: one draw of that
    error varies up to 6x between seeds of this shape (dbeta 1.3e-7 to 7.7e-7), too noisy a yardstick for a single
    case."""
    _say(f"case dropin_unfused {dtype}")
    worst, anchor = {}, {}
    for seed in range(4):
        inp = _prenormalised(gdr.make_inputs(2, 100, 3, 3, 128, 128, dtype, s0=True, seed=12 + seed))
        dsT = torch.randn(2, 3, 128, 128, generator=torch.Generator().manual_seed(9 + seed))
        if dtype == torch.bfloat16:
            old = op.BF16_UNNORMALIZED, op.BF16_STATE_GRAD
            try:
                op.BF16_UNNORMALIZED, op.BF16_STATE_GRAD = True, True
                assert op.plan(2, 100, 3, 128, 128, True, l2norm=False)["operands"] == "bf16"
                check_dropin(inp, bar=BF16_BAR, dsT=dsT, l2norm=False)
            finally:
                op.BF16_UNNORMALIZED, op.BF16_STATE_GRAD = old
            continue
        ro, rsT, rg = gdr.dropin_f64(*(inp[n] for n in ("query", "key", "value", "g", "beta", "initial_state")),
                                     do=inp["do"], dsT=dsT, use_qk_l2norm_in_kernel=False)
        o, sT, g = run_dropin(inp, dsT=dsT, l2norm=False)
        errs = {"o": gdr.rel(o, ro), "sT": gdr.rel(sT, rsT)}
        errs.update({n: gdr.rel(x, rg[n]) for n, x in g.items()})
        ref = torch_path_errors(inp, ro, rsT, rg, dsT, False)
        for n in errs:
            worst[n] = max(worst.get(n, 0.0), errs[n])
            anchor[n] = max(anchor.get(n, 0.0), ref[n])
    if dtype == torch.float32:
        _say("torch-path fp32 errors (largest over the seeds):", {k: f"{v:.2e}" for k, v in anchor.items()})
        _parity.check(worst, {n: 2 * anchor[n] for n in worst}, recompute=op.RECOMPUTE_STATES)


def test_golden_fixture():
    """The committed fixture (autograd through the recurrence in float64): the bf16 drop-in within 1e-2."""
    import os

    import numpy as np
    z = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dropin_small.npz"))
    t = {n: torch.from_numpy(z[n]) for n in z.files}
    inp = {n: t[n].to(torch.bfloat16) for n in ("query", "key", "value", "do")}
    inp.update(g=t["g"], beta=t["beta"], initial_state=t["initial_state"])
    o, sT, g = run_dropin(inp, dsT=t["dsT"])
    errs = {"o": gdr.rel(o, t["o"]), "sT": gdr.rel(sT, t["sT"])}
    errs.update({n: gdr.rel(x, t[n]) for n, x in g.items()})
    _parity.check(errs, BF16_BAR)


# ---- the GatedDeltaRule contract on the reference harness cases ------------------------------------------------------
def check_rule(xs64, rtol, dtype=torch.float32):
    gen = torch.Generator().manual_seed(9)
    xs = [x.to(dtype if i < 3 else torch.float32).to(DEV).requires_grad_(True) for i, x in enumerate(xs64)]
    o, sT = GatedDeltaRule.apply(*xs, True)
    ref = [x.to(dtype if i < 3 else torch.float32).double() for i, x in enumerate(xs64)]
    w_o = torch.randn(o.shape, generator=gen, dtype=torch.float64)
    w_s = torch.randn(sT.shape, generator=gen, dtype=torch.float64)
    torch.autograd.backward([o, sT], [w_o.to(DEV, o.dtype), w_s.float().to(DEV)])
    ro, rsT, P = gdr.chunked_forward(*ref)
    rg, _ = gdr.chunked_backward(*ref, w_o.to(o.dtype).double(), w_s.float().double(), P=P)
    errs = {"o": gdr.rel(o.cpu(), ro), "sT": gdr.rel(sT.cpu(), rsT)}
    for n, a, r in zip(("dq", "dk", "dv", "dg", "dbeta", "ds0"), xs, rg):
        errs[n] = gdr.rel(a.grad.cpu(), r)
    _parity.check(errs, rtol, recompute=op.RECOMPUTE_STATES)


@pytest.mark.parametrize("shape", [(1, 1, 1, 128, 128), (1, 2, 1, 128, 128), (2, 7, 3, 128, 128), (1, 8, 2, 128, 128),
                                   (1, 9, 2, 128, 128), (3, 63, 2, 128, 128), (1, 64, 1, 128, 128), (2, 65, 2, 128, 64),
                                   (1, 100, 5, 64, 64), (1, 31, 2, 64, 32)])
def test_rule_shapes(shape):
    _say(f"case rule_shapes {shape}")
    check_rule(gdr.harness_inputs(*shape), 2e-4)


def test_rule_no_starting_state():
    _say("case rule_no_state")
    check_rule(gdr.harness_inputs(2, 40, 2, 128, 128, state=False), 2e-4)


@pytest.mark.parametrize("beta,g", [(0.0, None), (1.0 - 1e-6, None), (None, 0.0), (None, -20.0), (1.0 - 1e-6, 0.0)])
def test_rule_stress(beta, g):
    _say(f"case rule_stress beta={beta} g={g}")
    check_rule(gdr.harness_inputs(1, 48, 2, 128, 128, beta=beta, g=g), 5e-4)


@pytest.mark.parametrize("beta,g", [(None, None), (1.0 - 1e-6, 0.0), (1.0 - 1e-6, None)])
def test_rule_correlated_keys(beta, g):
    _say(f"case rule_corr beta={beta} g={g}")
    xs = gdr.harness_inputs(1, 96, 2, 128, 128, beta=beta, g=g, corr=0.9, seed=6)
    assert (xs[1][0, 1:, 0] * xs[1][0, :-1, 0]).sum(-1).min() > 0.95
    check_rule(xs, 5e-4)


@pytest.mark.parametrize("T", [2048, 4096])
def test_rule_long_sequence(T):
    _say(f"case rule_long T={T}")
    check_rule(gdr.harness_inputs(1, T, 1, 128, 128, seed=3), 1e-3)


@pytest.mark.parametrize("shape", [(1, 33, 2, 256, 128), (2, 150, 3, 256, 64)])
def test_rule_wide_keys(shape):
    """Key heads of 256 (reference tests/test_harness.py:214-230, make(1, 33, 2, 256, 128)): forward and the chunked
    backward, at the harness bar.  The float32 kernels stage key columns in two passes (prep) and read the chunk
    tiles from memory where a stage does not fit LDS (the state passes)."""
    _say(f"case rule_wide {shape}")
    check_rule(gdr.harness_inputs(*shape, seed=2), 2e-4)


@pytest.mark.parametrize("split", [2, 4, 8])
def test_wide_keys_every_split(split):
    """Key width 256 at each value split (4, 2 and 1 column waves a workgroup) and in both backward modes: the same
    bits as the default launch."""
    _say(f"case wide split={split}")
    inp = gdr.make_inputs(1, 100, 2, 2, 256, 128, torch.float32, s0=True, seed=3)
    ref = _grads_once(inp, dsT_width=256)
    old = op.RECOMPUTE_STATES
    try:
        for mode in (True, False):
            op.RECOMPUTE_STATES = mode
            got = _grads_once(inp, split, dsT_width=256)
            assert all(torch.equal(a, b) for a, b in zip(ref, got))
    finally:
        op.RECOMPUTE_STATES = old


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dropin_wide_keys_2byte(dtype):
    """bf16 / fp16 drop-in at key width 256: upcast exactly and computed by the float32 kernels, output and the q, k,
    v gradients returned in the input dtype; within the 2-byte bar."""
    _say(f"case dropin_wide {dtype}")
    inp = gdr.make_inputs(2, 70, 2, 2, 256, 128, dtype, s0=True, seed=7)
    dsT = torch.randn(2, 2, 256, 128, generator=torch.Generator().manual_seed(9))
    check_dropin(inp, bar=5e-3, dsT=dsT)


def test_rule_bf16_operands():
    """The contract with bf16 q/k/v (bf16 MFMA operands, fp32 accumulation): within 1e-2."""
    _say("case rule_bf16")
    check_rule(gdr.harness_inputs(2, 100, 2, 128, 128, seed=4), BF16_BAR, dtype=torch.bfloat16)


def test_bf16_inputs_on_the_float32_kernels(monkeypatch):
    """BF16_OPERANDS = False: bf16 inputs upcast exactly and run on the float32 kernels, the reference's own
    precision for every input (op.py:276-285, 297).  On the smoke's draw with a final-state gradient (the bf16
    attribution case) the float32 outputs and gradients (sT, dg,
    dbeta, ds0) come within 1e-4 of float64, at least 10x closer than the bf16 operands (their backward with the final
    state's gradient kept on them: op.BF16_STATE_GRAD), and the bf16 outputs and gradients within their own rounding
    (1e-2)."""
    _say("case bf16 inputs on float32 kernels")
    monkeypatch.setattr(op, "BF16_STATE_GRAD", True)
    inp = gdr.make_inputs(1, 100, 2, 2, 128, 128, torch.bfloat16, s0=True, seed=7)
    dsT = torch.randn(1, 2, 128, 128, generator=torch.Generator().manual_seed(11))
    ro, rsT, rg = gdr.dropin_f64(*(inp[n] for n in ("query", "key", "value", "g", "beta", "initial_state")),
                                 do=inp["do"], dsT=dsT)

    def errors():
        o, sT, g = run_dropin(inp, dsT=dsT)
        e = {"o": gdr.rel(o, ro), "sT": gdr.rel(sT, rsT)}
        e.update({n: gdr.rel(x, rg[n]) for n, x in g.items()})
        return e, o.dtype, {n: x.dtype for n, x in g.items()}

    fast, _, _ = errors()
    old = op.BF16_OPERANDS
    try:
        op.BF16_OPERANDS = False
        exact, odt, gdt = errors()
    finally:
        op.BF16_OPERANDS = old
    _say("bf16 operands:", {k: f"{v:.2e}" for k, v in fast.items()})
    assert odt == torch.bfloat16 and gdt["dquery"] == gdt["dkey"] == gdt["dvalue"] == torch.bfloat16
    f32 = ("sT", "dg", "dbeta", "dstate")
    bars = {n: (1e-4 if n in f32 else BF16_BAR) for n in exact}
    _parity.check(exact, bars, bf16_operands=False)
    for n in f32:
        assert exact[n] * 10 <= fast[n], (n, exact[n], fast[n])


# ---- determinism and launch-policy invariance ------------------------------------------------------------------------
def _grads_once(inp, split=None, dsT_width=128):
    old = op.VALUE_SPLIT
    try:
        if split is not None:
            op.VALUE_SPLIT = split
        o, sT, g = run_dropin(inp, dsT=torch.ones(inp["value"].shape[0], inp["value"].shape[2], dsT_width,
                                                  inp["value"].shape[-1]))
    finally:
        op.VALUE_SPLIT = old
    return [o, sT] + [g[n] for n in sorted(g)]


@pytest.fixture
def bf16_state_grad(monkeypatch):
    """op.BF16_STATE_GRAD on: a backward with a final-state gradient stays on the bf16 kernels, whose invariances the
    tests below pin (by default such a backward runs the float32 kernels)."""
    monkeypatch.setattr(op, "BF16_STATE_GRAD", True)


def test_backward_is_bitwise_deterministic(bf16_state_grad):
    """One writer per gradient element, no atomics: three runs give identical bits (reference test_harness.py:196-211)."""
    _say("case determinism")
    inp = gdr.make_inputs(2, 100, 2, 2, 128, 128, torch.bfloat16, s0=True, seed=5)
    runs = [_grads_once(inp) for _ in range(3)]
    assert all(torch.equal(a, b) for r in runs[1:] for a, b in zip(runs[0], r))


@pytest.mark.parametrize("B,T,Hk,Hv,D", [(8, 1000, 16, 16, 128), (8, 1000, 16, 16, 64), (4, 700, 8, 16, 128)])
def test_persistent_chunk_backward_equals_per_row_runs(B, T, Hk, Hv, D):
    """With more chunk-heads than CUs the bf16 chunk backward runs persistent workgroups, each over a strided run of
    chunk-heads whose reads are issued during the previous one's compute (rotating LDS arrays, the state registers
    refilled early); one batch row alone has at most 256 chunk-heads and runs one chunk-head a workgroup.  Every row
    is independent, so the batch run must equal the rows run one at a time bit for bit (ragged last chunks, grouped
    value heads, D = 64 and 128)."""
    _say(f"case persistent chunk backward B={B} T={T} Hk={Hk} Hv={Hv} D={D}")
    inp = gdr.make_inputs(B, T, Hk, Hv, D, D, torch.bfloat16, s0=True, seed=21)
    o, sT, g = run_dropin(inp, dsT=None)
    for b in range(B):
        row = {n: (None if x is None else x[b:b + 1]) for n, x in inp.items()}
        ob, sTb, gb = run_dropin(row, dsT=None)
        assert torch.equal(o[b:b + 1], ob) and torch.equal(sT[b:b + 1], sTb), b
        for n in NAMES:
            assert torch.equal(g[n][b:b + 1], gb[n]), (b, n)


def test_value_split_changes_no_bits(bf16_state_grad):
    """Splitting a head-row's value columns over 1, 2, 4 or 8 workgroups changes no arithmetic: identical bits
    (reference test_chunking.py:108-128)."""
    _say("case split bits")
    inp = gdr.make_inputs(1, 150, 3, 3, 128, 128, torch.bfloat16, s0=True, seed=6)
    runs = [_grads_once(inp, s) for s in (1, 2, 4, 8)]
    assert all(torch.equal(a, b) for r in runs[1:] for a, b in zip(runs[0], r))


@pytest.mark.parametrize("D", [64, 128])
def test_float32_key_split_changes_no_bits(D):
    """The float32 state passes carry a 16-column slice on two waves, each holding half the state's rows, where a
    workgroup has at most two slices (value splits 4 and 8 at DV = 128), and on one wave a slice otherwise (splits 1,
    2); both forms add the halves' products in the same order, so every split, both backward modes and the recompute
    pair in one launch or two give identical bits."""
    _say(f"case float32 key split bits D={D}")
    inp = gdr.make_inputs(2, 150, 2, 2, D, 128, torch.float32, s0=True, seed=31)
    ref = _grads_once(inp, 1, dsT_width=D)
    old = op.RECOMPUTE_STATES, op.OVERLAP
    try:
        for split in (2, 4, 8):
            for recompute, overlap in ((True, True), (True, False), (False, False)):
                op.RECOMPUTE_STATES, op.OVERLAP = recompute, overlap
                got = _grads_once(inp, split, dsT_width=D)
                assert all(torch.equal(a, b) for a, b in zip(ref, got)), (split, recompute, overlap)
    finally:
        op.RECOMPUTE_STATES, op.OVERLAP = old


@pytest.mark.parametrize("split", [2, 4])
def test_overlapped_passes_change_no_bits(split, bf16_state_grad):
    """In the recompute mode (the default) the backward's recompute and reverse passes run in one launch
    (op.OVERLAP, macai_gdr_state_pair) or as two launches: identical bits, several times in a row.  split 2 gives
    four column waves a workgroup (config 1's pair pass), split 4 two."""
    _say(f"case overlap bits split={split}")
    inp = gdr.make_inputs(2, 200, 4, 4, 128, 128, torch.bfloat16, s0=True, seed=8)
    old = op.OVERLAP, op.RECOMPUTE_STATES, op.VALUE_SPLIT
    before = dict(op.CALLS)
    try:
        op.RECOMPUTE_STATES, op.VALUE_SPLIT = True, split
        op.OVERLAP = False
        ref = _grads_once(inp, split)
        op.OVERLAP = True
        runs = [_grads_once(inp, split) for _ in range(3)]
    finally:
        op.OVERLAP, op.RECOMPUTE_STATES, op.VALUE_SPLIT = old
    ran = {k: v - before.get(k, 0) for k, v in op.CALLS.items() if v != before.get(k, 0)}
    assert ran == {f"fwd s{split}": 4, f"bwd recompute+reverse s{split}": 1, f"bwd pair s{split}": 3}, ran
    assert all(torch.equal(a, b) for r in runs for a, b in zip(ref, r))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_kept_prep_operands_change_no_bits(dtype, bf16_state_grad):
    """The training forward keeping prep's operands (with A) and the chunk states for the backward
    (op.RECOMPUTE_STATES = False), only prep's operands (op.KEEP_PREP: the backward recomputes the states), or nothing
    (the reference's default, op.py:27-33, the backward rerunning prep): the same output and gradient bits (the
    reference's claim for its switch, tests/test_memory.py), and each mode runs the passes it should (the recompute
    modes pair their two state passes in one launch for bf16 operands, two launches for float32, op.OVERLAP)."""
    _say("case recompute bits", dtype)
    inp = gdr.make_inputs(2, 150, 2, 4, 128, 128, dtype, s0=True, seed=9)
    old = op.RECOMPUTE_STATES, op.KEEP_PREP
    both = "pair" if dtype == torch.bfloat16 else "recompute+reverse"
    try:
        outs = []
        for recompute, keep_prep, state_pass in ((True, False, both), (False, False, "reverse"), (True, True, both)):
            op.RECOMPUTE_STATES, op.KEEP_PREP = recompute, keep_prep
            p = op.plan(2, 150, 4, 128, 128, True, Hk=2, dtype=dtype)
            assert (p["bwd_state_passes"], p["bwd_prep"]) == (state_pass, "rerun" if recompute and not keep_prep
                                                              else "kept"), p
            events, op.EVENTS = op.EVENTS, []
            try:
                o, sT, grads = run_dropin(inp, dsT=torch.ones(2, 4, 128, 128))
                ran = [name for name, _, _ in op.EVENTS]
            finally:
                op.EVENTS = events
            assert ran.count("prep_bwd") == (1 if recompute and not keep_prep else 0), ran
            assert ("state_pair" in ran) == (state_pass == "pair") and ("state_bwd" in ran) == (state_pass != "pair")
            assert ("state_fwd_store" in ran) == (state_pass == "recompute+reverse")
            outs.append([o, sT] + [grads[n] for n in sorted(grads)])
    finally:
        op.RECOMPUTE_STATES, op.KEEP_PREP = old
    assert all(torch.equal(a, b) for other in outs[1:] for a, b in zip(outs[0], other))


def test_unfused_prologue_switch():
    """op.FUSED_NORM = False (the reference's switch, op.py:19-21): the query / key normalisation runs as float32
    PyTorch operations (autograd through them) and the kernels apply only the scale, on the float32 kernels with the
    normalised values kept in float32; outputs and gradients within the bf16 bar of float64 (rounding the normalised
    keys to bf16 for the bf16 kernels put dg at 9.4e-3 on this draw, and the oracle's model over 1e-2 on others)."""
    _say("case fused_norm off")
    inp = gdr.make_inputs(2, 150, 3, 3, 128, 128, torch.bfloat16, s0=True, seed=31)
    dsT = torch.randn(2, 3, 128, 128, generator=torch.Generator().manual_seed(32))
    old = op.FUSED_NORM
    try:
        op.FUSED_NORM = False
        assert op.plan(2, 150, 3, 128, 128, True)["operands"] == "f32"
        check_dropin(inp, bar=BF16_BAR, dsT=dsT)
    finally:
        op.FUSED_NORM = old


def test_misaligned_inputs_give_the_aligned_bits():
    """q, k, v, g, beta, the initial state and dO as contiguous views whose start is not 16-byte aligned (one element
    into a larger buffer): the drop-in copies them to aligned buffers and returns the bits of aligned inputs, gradients
    included (the reference's _even, op.py:58-60)."""
    _say("case misaligned inputs")
    inp = gdr.make_inputs(1, 100, 2, 2, 128, 128, torch.bfloat16, s0=True, seed=33)
    dsT = torch.randn(1, 2, 128, 128, generator=torch.Generator().manual_seed(34))
    names = ("query", "key", "value", "g", "beta", "initial_state")

    def run(shift):
        bases, leaves = [], []
        for n in names:
            x = inp[n].to(DEV)
            base = torch.zeros(x.numel() + shift, device=DEV, dtype=x.dtype)
            base[shift:] = x.reshape(-1)
            base.requires_grad_(True)
            bases.append(base)
            leaves.append(base[shift:].view(x.shape))
        assert shift == 0 or all(t.data_ptr() % 16 for t in leaves)
        do = torch.zeros(inp["do"].numel() + shift, device=DEV, dtype=inp["do"].dtype)
        do[shift:] = inp["do"].to(DEV).reshape(-1)
        o, sT = chunk_gated_delta_rule(*leaves[:5], initial_state=leaves[5], output_final_state=True,
                                       use_qk_l2norm_in_kernel=True)
        torch.autograd.backward([o, sT], [do[shift:].view(inp["do"].shape), dsT.to(DEV)])
        torch.cuda.synchronize()
        return [o.detach().cpu(), sT.detach().cpu()] + [b.grad[shift:].cpu() for b in bases]

    ref, got = run(0), run(1)
    assert all(torch.equal(a, b) for a, b in zip(ref, got))


# ---- head widths beyond the bf16 kernels' (the reference takes any multiple of 32: op.py:124-125) --------------------
@pytest.mark.parametrize("shape", [(1, 100, 2, 96, 64), (1, 77, 2, 160, 128), (2, 70, 2, 192, 96), (1, 130, 1, 224, 160),
                                   (1, 90, 2, 128, 256), (1, 65, 2, 64, 192), (1, 100, 1, 256, 224), (1, 40, 2, 32, 256)])
def test_rule_widths(shape):
    """Key widths 96, 160, 192, 224 and value widths 160-256 through the backward, on the float32 kernels (key columns
    staged in one pass up to 192, in passes of 32 at 224; the value width taken at run time by the per-chunk
    backward): the contract at the harness bar 2e-4, ragged lengths, with a starting state."""
    _say(f"case rule_widths {shape}")
    check_rule(gdr.harness_inputs(*shape, seed=2), 2e-4)


@pytest.mark.parametrize("DK,DV", [(96, 128), (128, 256), (160, 64)])
def test_dropin_widths_bf16(DK, DV):
    """bf16 drop-in at widths the bf16 kernels do not take in the backward: upcast exactly and computed by the float32
    kernels (outputs and q, k, v gradients returned in bf16), within the 2-byte bar; the forward alone at a value width
    of 256 stays on the bf16 kernels, within the bf16 bar."""
    _say(f"case dropin_widths_bf16 DK={DK} DV={DV}")
    inp = gdr.make_inputs(2, 80, 2, 2, DK, DV, torch.bfloat16, s0=True, seed=17)
    dsT = torch.randn(2, 2, DK, DV, generator=torch.Generator().manual_seed(18))
    check_dropin(inp, bar=5e-3, dsT=dsT)
    if DV > 128:
        ro, rsT, _ = gdr.dropin_f64(*(inp[n] for n in ("query", "key", "value", "g", "beta", "initial_state")))
        with torch.no_grad():
            o, sT, _ = run_dropin(inp, grads=False)
        _parity.check({"o": gdr.rel(o, ro), "sT": gdr.rel(sT, rsT)}, BF16_BAR)


def test_recompute_keeps_only_inputs():
    """What the training forward keeps for its backward (the reference's tests/test_memory.py:239-250): with
    op.RECOMPUTE_STATES (the default) exactly the six inputs, nothing a chunk; with it off, the inputs and one buffer
    holding prep's operands with A and the chunk states (2,816 bytes a token-head at D = 128 in bf16); with
    op.KEEP_PREP, the inputs and prep's operands with A alone (1,536 bytes a token-head)."""
    _say("case saved tensors")
    B, T, H, D = 2, 650, 4, 128
    xs = [x.to(DEV).requires_grad_(True) for x in gdr.harness_inputs(B, T, H, D, D, seed=3)]
    xs = [x.to(torch.bfloat16 if i < 3 else torch.float32).detach().requires_grad_(True) for i, x in enumerate(xs)]
    NT = -(-T // 64)
    old = op.RECOMPUTE_STATES, op.KEEP_PREP
    try:
        op.RECOMPUTE_STATES = True
        o, sT = GatedDeltaRule.apply(*xs, True)
        saved = [t for t in o.grad_fn.saved_tensors if t is not None]
        assert len(saved) == 6 and all(s.data_ptr() == x.data_ptr() for s, x in zip(saved, xs))
        for recompute, keep_prep, size in ((False, False, 2816), (True, True, 1536)):
            op.RECOMPUTE_STATES, op.KEEP_PREP = recompute, keep_prep
            o, sT = GatedDeltaRule.apply(*xs, True)
            saved = [t for t in o.grad_fn.saved_tensors if t is not None]
            assert len(saved) == 7 and all(s.data_ptr() == x.data_ptr() for s, x in zip(saved, xs))
            per_token_head = saved[6].numel() / (B * H * NT * 64)
            assert size <= per_token_head < size + 64, per_token_head    # plus the parts' 256-byte alignment
    finally:
        op.RECOMPUTE_STATES, op.KEEP_PREP = old


def test_strided_views_give_contiguous_bits():
    """q, k, v as strided views of one projection output (the model splits its conv output; the reference's layout
    cases in tests/test_memory.py): the drop-in makes them contiguous itself and returns the bits of contiguous
    inputs, gradients included."""
    _say("case strided views")
    inp = gdr.make_inputs(2, 90, 3, 3, 128, 128, torch.bfloat16, s0=True, seed=35)
    dsT = torch.randn(2, 3, 128, 128, generator=torch.Generator().manual_seed(36))
    ref = run_dropin(inp, dsT=dsT)
    packed = torch.stack([inp["query"], inp["key"], inp["value"]], 2).to(DEV).requires_grad_(True)   # [B, T, 3, H, D]
    q, k, v = packed[:, :, 0], packed[:, :, 1], packed[:, :, 2]
    assert not q.is_contiguous()
    rest = [inp[n].to(DEV).requires_grad_(True) for n in ("g", "beta", "initial_state")]
    o, sT = chunk_gated_delta_rule(q, k, v, rest[0], rest[1], initial_state=rest[2], output_final_state=True,
                                   use_qk_l2norm_in_kernel=True)
    torch.autograd.backward([o, sT], [inp["do"].to(DEV), dsT.to(DEV)])
    torch.cuda.synchronize()
    assert torch.equal(o.detach().cpu(), ref[0]) and torch.equal(sT.detach().cpu(), ref[1])
    grads = [packed.grad[:, :, i].cpu() for i in range(3)] + [x.grad.cpu() for x in rest]
    for n, x in zip(NAMES, grads):
        assert torch.equal(x, ref[2][n]), n

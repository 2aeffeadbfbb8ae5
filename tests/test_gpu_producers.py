"""GPU parity of the rule's producers, the linear-attention layer's convolution path and gates (macai.layer; the
reference's tests/test_layer.py:216-316 and its parity helper 48-99).

Reference values: the float64 oracle (oracle/producers.py, pinned in tests/test_oracle_producers.py) and autograd
through it, on inputs drawn as float64 values exactly representable in the tested dtype.  The bar, per output and per
needed input gradient: the HIP path's error against float64 at most twice that of the PyTorch path in the same dtype
on the same device (conv1d with groups = channels + silu, sigmoid / softplus: transformers' torch path).
"""
import pytest
import torch

import _parity
import torch.nn.functional as F

from macai.layer import conv_qkv, gates
from oracle import producers as P
from oracle.gdr import rel

pytestmark = pytest.mark.gpu
DEV = "cuda"
F64 = torch.float64
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
DT = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}
# the real widths (reference tests/test_layer.py:36-37): key_dim, value_dim, head widths, repeat, value heads
LIN = {"0.8b": dict(kd=2048, vd=2048, dk=128, rep=1, dv=128, hv=16),
       "9b": dict(kd=2048, vd=4096, dk=128, rep=2, dv=128, hv=32)}


def _say(*a):
    print(*a, flush=True)


def draw(shape, dtype, scale=1.0, seed=0):
    """float64 values exactly representable in dtype (reference tests/test_layer.py:52-55)."""
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=gen, dtype=F64) * scale).to(dtype).double()


def run(fn, xs, dtypes, needs, gouts, device):
    leaves = [x.detach().to(device, d).clone().requires_grad_(n) for x, d, n in zip(xs, dtypes, needs)]
    outs = fn(*leaves)
    outs = outs if isinstance(outs, tuple) else (outs,)
    torch.autograd.backward(outs, [g.to(device, o.dtype) for g, o in zip(gouts, outs)])
    if device != "cpu":
        torch.cuda.synchronize()
    return ([o.detach().cpu().double() for o in outs],
            [x.grad.detach().cpu().double() if n else None for x, n in zip(leaves, needs)])


def parity(case, ref_fn, torch_fn, fused_fn, xs, dtypes, needs, out_names, in_names, gdtype):
    _say("case", case)
    with torch.no_grad():
        shapes = [o.shape for o in ref_fn(*xs)]
    gouts = [draw(s, gdtype, seed=100 + i) for i, s in enumerate(shapes)]
    ro, rg = run(ref_fn, xs, [F64] * len(xs), needs, gouts, "cpu")
    to, tg = run(torch_fn, xs, dtypes, needs, gouts, DEV)
    fo, fg = run(fused_fn, xs, dtypes, needs, gouts, DEV)
    rows = {n: (rel(t, r), rel(f, r)) for n, r, t, f in zip(out_names, ro, to, fo)}
    rows.update({"d" + n: (rel(t, r), rel(f, r)) for n, r, t, f, need in zip(in_names, rg, tg, fg, needs) if need})
    _say("  (pytorch, fused):", {k: f"{v[0]:.1e}/{v[1]:.1e}" for k, v in rows.items()})
    _parity.check({k: v[1] for k, v in rows.items()}, {k: 2 * v[0] for k, v in rows.items()}, case=case)


# ---- the convolution path ---------------------------------------------------------------------------------------------
def check_conv(model, bt, dtype, trained):
    c = LIN[model]
    B, T = bt
    C = 2 * c["kd"] + c["vd"]
    x = draw((B, T, C), dtype, seed=11)
    w = draw((C, 1, 4), dtype, scale=0.3, seed=12)

    def ref(x_, w_):
        return P.conv_qkv(x_, w_, c["kd"], c["dk"], c["rep"], c["dv"])

    def torch_path(x_, w_):
        y = F.silu(F.conv1d(x_.transpose(1, 2), w_, padding=3, groups=C)[:, :, :T]).transpose(1, 2)
        q, k, v = torch.split(y, [c["kd"], c["kd"], c["vd"]], dim=-1)
        q, k, v = q.reshape(B, T, -1, c["dk"]), k.reshape(B, T, -1, c["dk"]), v.reshape(B, T, -1, c["dv"])
        if c["rep"] > 1:
            q, k = q.repeat_interleave(c["rep"], 2), k.repeat_interleave(c["rep"], 2)
        return q, k, v.float()

    def fused(x_, w_):
        return conv_qkv(x_, w_, c["kd"], c["dk"], c["rep"], c["dv"])
    parity(f"conv {model} {bt} {DT[dtype]}{' trained' if trained else ''}", ref, torch_path, fused, [x, w],
           [dtype, dtype], [True, trained], ["q", "k", "v"], ["x", "w"], dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=DT.get)
@pytest.mark.parametrize("bt", [(1, 1), (2, 3), (2, 33), (3, 100)], ids=str)
@pytest.mark.parametrize("model", ["0.8b", "9b"])
def test_conv_path(model, bt, dtype):
    check_conv(model, bt, dtype, False)


@pytest.mark.parametrize("dtype", DTYPES, ids=DT.get)
@pytest.mark.parametrize("model", ["0.8b", "9b"])
def test_conv_path_trained_weight(model, dtype):
    """The taps' gradient when the weight trains (partials a tile, fixed-order sum)."""
    check_conv(model, (2, 33), dtype, True)


def test_conv_key_heads_layout():
    """repeat=False (key heads only) with v in x's dtype, the layout the rule reads natively: q, k are every rep-th
    head of the repeated layout and v its float32 v rounded to bf16, bit for bit; dx through both layouts agrees
    (the repeated copies' gradients are summed in the kernel in either case)."""
    c = LIN["9b"]
    B, T = 2, 50
    C = 2 * c["kd"] + c["vd"]
    x = draw((B, T, C), torch.bfloat16, seed=21).to(DEV, torch.bfloat16)
    w = draw((C, 1, 4), torch.bfloat16, scale=0.3, seed=22).to(DEV, torch.bfloat16)
    q1, k1, v1 = conv_qkv(x, w, c["kd"], c["dk"], c["rep"], c["dv"])
    q2, k2, v2 = conv_qkv(x, w, c["kd"], c["dk"], c["rep"], c["dv"], repeat=False, v_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert q2.shape == (B, T, c["kd"] // c["dk"], c["dk"]) and v2.dtype == torch.bfloat16
    assert torch.equal(q1[:, :, ::c["rep"]], q2) and torch.equal(k1[:, :, ::c["rep"]], k2)
    assert torch.equal(v1.to(torch.bfloat16), v2)


def test_conv_empty_and_rejects_cpu():
    c = LIN["0.8b"]
    C = 2 * c["kd"] + c["vd"]
    x = torch.zeros(2, 0, C, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    w = torch.zeros(C, 1, 4, device=DEV, dtype=torch.bfloat16)
    q, k, v = conv_qkv(x, w, c["kd"], c["dk"], c["rep"], c["dv"])
    assert q.shape == (2, 0, 16, 128) and v.shape == (2, 0, 16, 128)
    with pytest.raises(RuntimeError, match="HIP device"):
        conv_qkv(torch.zeros(1, 4, C), torch.zeros(C, 1, 4), c["kd"], c["dk"], c["rep"], c["dv"])


# ---- beta and g ---------------------------------------------------------------------------------------------------------
def check_gates(model, bt, dtype, trained):
    hv = LIN[model]["hv"]
    b = draw((*bt, hv), dtype, scale=2.0, seed=13)
    a = draw((*bt, hv), dtype, scale=3.0, seed=14)
    gen = torch.Generator().manual_seed(15)
    A_log = torch.log(torch.rand(hv, generator=gen, dtype=F64) * 15.99 + 0.01).to(dtype).double()
    dt_bias = draw((hv,), dtype, seed=16)

    def torch_path(b_, a_, A_, d_):
        return b_.sigmoid().float(), -A_.float().exp() * F.softplus(a_.float() + d_.float())
    parity(f"gates {model} {bt} {DT[dtype]}{' trained' if trained else ''}", P.gates, torch_path, gates,
           [b, a, A_log, dt_bias], [dtype] * 4, [True, True, trained, trained], ["beta", "g"],
           ["b", "a", "A_log", "dt_bias"], torch.float32)


@pytest.mark.parametrize("dtype", DTYPES, ids=DT.get)
@pytest.mark.parametrize("bt", [(1, 1), (2, 7), (3, 33), (2, 129)], ids=str)
@pytest.mark.parametrize("model", ["0.8b", "9b"])
def test_gates(model, bt, dtype):
    check_gates(model, bt, dtype, False)


@pytest.mark.parametrize("dtype", DTYPES, ids=DT.get)
@pytest.mark.parametrize("model", ["0.8b", "9b"])
def test_gates_trained(model, dtype):
    """A_log's and dt_bias's gradients when they train."""
    check_gates(model, (3, 33), dtype, True)


def test_gates_softplus_threshold():
    """Past softplus's threshold (a + dt_bias > 20) the input itself; deep in the negative range, log1p (the
    reference's case, tests/test_layer.py:306-316)."""
    a = torch.tensor([[-80.0, -30.0, -5.0, 0.0, 19.5, 20.5, 40.0, 3.0]], dtype=torch.float32)
    z = torch.zeros(8)
    beta, g = gates(*(t.to(DEV) for t in (torch.zeros_like(a), a, z, z)))
    ref = -F.softplus(a.double())
    assert ((g.cpu().double() - ref).abs() / ref.abs()).max() < 1e-6
    assert torch.equal(beta.cpu(), torch.full_like(a, 0.5))


def test_producers_feed_the_rule():
    """x -> conv (key heads, bf16 v) and gates -> the drop-in rule with grouped heads -> backward into x, a, b: the
    same gradients, within the bf16 bar, as through the repeated layout with float32 v (the reference's)."""
    from macai.gated_delta import chunk_gated_delta_rule
    c = LIN["9b"]
    B, T = 1, 130
    C = 2 * c["kd"] + c["vd"]
    xs = draw((B, T, C), torch.bfloat16, seed=31)
    w = draw((C, 1, 4), torch.bfloat16, scale=0.3, seed=32).to(DEV, torch.bfloat16)
    bs, as_ = draw((B, T, c["hv"]), torch.bfloat16, seed=33), draw((B, T, c["hv"]), torch.bfloat16, seed=34)
    A_log = torch.zeros(c["hv"], device=DEV)
    dt = torch.zeros(c["hv"], device=DEV)
    do = draw((B, T, c["hv"], c["dv"]), torch.bfloat16, seed=35).to(DEV, torch.bfloat16)
    grads = []
    for native in (False, True):
        x = xs.to(DEV, torch.bfloat16).requires_grad_(True)
        b = bs.to(DEV, torch.bfloat16).requires_grad_(True)
        a = as_.to(DEV, torch.bfloat16).requires_grad_(True)
        kw = dict(repeat=False, v_dtype=torch.bfloat16) if native else {}
        q, k, v = conv_qkv(x, w, c["kd"], c["dk"], c["rep"], c["dv"], **kw)
        beta, g = gates(b, a, A_log, dt)
        o, _ = chunk_gated_delta_rule(q, k, v, g, beta, use_qk_l2norm_in_kernel=True)
        torch.autograd.backward(o, do)
        torch.cuda.synchronize()
        grads.append([t.grad.cpu().double() for t in (x, b, a)])
    errs = [rel(n, r) for n, r in zip(grads[1], grads[0])]
    _say("native vs repeated layout, dx db da:", errs)
    assert max(errs) < 1e-2

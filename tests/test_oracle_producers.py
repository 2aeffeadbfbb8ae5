"""The producers' oracle (oracle/producers.py) pinned on the CPU: the convolution path against torch's conv1d with
groups = channels (the form of transformers' torch path, modeling_qwen3_5.py causal_conv1d fallback; reference
tests/test_layer.py:236-240) and silu; the gates against sigmoid and softplus (threshold 20), including the
reference's threshold values (tests/test_layer.py:306-316)."""
import torch
import torch.nn.functional as F

from oracle import producers as P

F64 = torch.float64


def test_conv_matches_conv1d_and_silu():
    gen = torch.Generator().manual_seed(0)
    B, T, kd, vd, dk, dv = 2, 37, 32, 64, 16, 16
    C = 2 * kd + vd
    x = torch.randn(B, T, C, generator=gen, dtype=F64)
    w = torch.randn(C, 1, 4, generator=gen, dtype=F64) * 0.3
    u = F.conv1d(x.transpose(1, 2), w, padding=3, groups=C)[:, :, :T].transpose(1, 2)
    y = F.silu(u)
    for rep in (1, 2):
        q, k, v = P.conv_qkv(x, w, kd, dk, rep, dv, repeat=True)
        rq = y[..., :kd].reshape(B, T, -1, dk).repeat_interleave(rep, 2)
        rk = y[..., kd:2 * kd].reshape(B, T, -1, dk).repeat_interleave(rep, 2)
        assert torch.allclose(q, rq, rtol=0, atol=1e-13) and torch.allclose(k, rk, rtol=0, atol=1e-13)
        assert torch.allclose(v, y[..., 2 * kd:].reshape(B, T, -1, dv), rtol=0, atol=1e-13)
    # a plausible slip -- the taps applied in reverse order (a correlation instead of the causal convolution) -- fails
    u_rev = P.conv_u(x, w.reshape(C, 4).flip(-1))
    assert (u_rev - u).abs().max() > 1e-2


def test_conv_is_causal():
    """An input at time t changes no output before t."""
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(1, 20, 16, generator=gen, dtype=F64)
    w = torch.randn(16, 4, generator=gen, dtype=F64)
    x2 = x.clone()
    x2[:, 11] += 1.0
    d = (P.conv_u(x2, w) - P.conv_u(x, w)).abs().amax((0, 2))
    assert d[:11].max() == 0 and d[11:15].min() > 0 and d[15:].max() == 0


def test_gates_match_torch():
    gen = torch.Generator().manual_seed(2)
    b = torch.randn(3, 33, 8, generator=gen, dtype=F64) * 2
    a = torch.randn(3, 33, 8, generator=gen, dtype=F64) * 3
    A_log = torch.log(torch.rand(8, generator=gen, dtype=F64) * 15.99 + 0.01)
    dt = torch.randn(8, generator=gen, dtype=F64)
    beta, g = P.gates(b, a, A_log, dt)
    assert torch.allclose(beta, torch.sigmoid(b), rtol=0, atol=1e-15)
    assert torch.allclose(g, -A_log.exp() * F.softplus(a + dt, threshold=20), rtol=1e-14, atol=0)


def test_softplus_threshold_values():
    """The reference's threshold test inputs (tests/test_layer.py:307-316): the input itself past 20, log1p deep in
    the negative range."""
    a = torch.tensor([[-80.0, -30.0, -5.0, 0.0, 19.5, 20.5, 40.0, 3.0]], dtype=F64)
    z = torch.zeros(8, dtype=F64)
    _, g = P.gates(torch.zeros_like(a), a, z, z)
    ref = -F.softplus(a)
    assert ((g - ref).abs() / ref.abs()).max() < 1e-15
    assert g[0, 6] == -40.0 and g[0, 5] == -20.5


def test_gradients_flow():
    """The oracle is differentiable (the GPU tests take their reference gradients from autograd through it)."""
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(1, 9, 48, generator=gen, dtype=F64, requires_grad=True)
    w = torch.randn(48, 4, generator=gen, dtype=F64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda x_, w_: P.conv_qkv(x_, w_, 16, 8, 1, 8), (x, w))

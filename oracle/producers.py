"""Float64 CPU restatement of the rule's producers, the linear-attention layer's convolution path and gates (test
infrastructure only; see oracle/__init__.py).  Differentiable through autograd, so the backward's reference values
are the autograd gradients of these functions.

Pinned in tests/test_oracle_producers.py against torch's own routines (conv1d with groups = channels, silu,
softplus with threshold 20, sigmoid) and against the reference's softplus-threshold values
(tests/test_layer.py:306-316).
"""
import torch

F64 = torch.float64
K = 4


def conv_u(x, w):
    """u[b, t, c] = sum_j w[c, j] x[b, t - 3 + j, c], zero before the start (reference layer/_conv.py:4, 73).
    x [B, T, C], w [C, 4]."""
    B, T, C = x.shape
    xp = torch.cat([x.new_zeros(B, K - 1, C), x], 1)
    return sum(w[:, j] * xp[:, j:j + T] for j in range(K))


def conv_qkv(x, w, kd, dk, rep, dv, repeat=True):
    """The convolution path (layer/_conv.py:1-24): y = u sigmoid(u); q, k = y's first two kd-channel blocks as
    [B, T, kd / dk, dk], each key head repeated rep times when repeat (transformers' repeat_interleave); v = the rest
    as [B, T, ., dv]."""
    B, T, C = x.shape
    u = conv_u(x, w.reshape(C, K))
    y = u * torch.sigmoid(u)
    q, k, v = y[..., :kd], y[..., kd:2 * kd], y[..., 2 * kd:]
    q, k, v = q.reshape(B, T, -1, dk), k.reshape(B, T, -1, dk), v.reshape(B, T, -1, dv)
    if repeat and rep > 1:
        q, k = q.repeat_interleave(rep, 2), k.repeat_interleave(rep, 2)
    return q, k, v


def softplus20(x):
    """PyTorch's softplus with threshold 20: x itself above it, log(1 + e^x) below (layer/_gates.py:3-5, 31)."""
    return torch.where(x > 20, x, torch.log1p(torch.exp(torch.clamp(x, max=20))))


def gates(b, a, A_log, dt_bias):
    """(beta, g) = (sigmoid(b), -exp(A_log) softplus(a + dt_bias)) (layer/_gates.py:1-5); b, a [..., H]; A_log,
    dt_bias [H]."""
    return torch.sigmoid(b), -torch.exp(A_log) * softplus20(a + dt_bias)

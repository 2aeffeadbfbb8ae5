"""The linear-attention layer's gates, one HIP launch each way (entry points macai_gdr_gates_fwd /
macai_gdr_gates_bwd of include/macai_gdr.h; the function of the reference's layer/_gates.py:1-13):

    beta = sigmoid(b)
    g    = -exp(A_log) softplus(a + dt_bias)      softplus with PyTorch's threshold of 20

b and a are the [..., H] outputs of in_proj_b and in_proj_a (float32, bfloat16 or float16); A_log and dt_bias are
[H].  beta and g come out in float32, the dtype the rule reads them in.  Gradients: db and da in the inputs' dtype;
A_log's and dt_bias's only when they train, each head's rows summed on the device in a fixed order (deterministic).
"""
import torch

from ..gated_delta import _native as N
from ..gated_delta.op import _on


def _dense(t):
    """t contiguous and 16-byte aligned, as the kernels' vector accesses need (a copy only when it is not)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _f32(t):
    """t as a dense, aligned float32 tensor (t itself when it already is)."""
    return _dense(t if t.dtype == torch.float32 else t.to(torch.float32))


class Gates(torch.autograd.Function):
    """(beta, g) = (sigmoid(b), -exp(A_log) softplus(a + dt_bias)), both float32."""

    @staticmethod
    def forward(ctx, b, a, A_log, dt_bias):
        if not b.is_cuda:
            raise RuntimeError("macai's gates run on a HIP device (MI355X); got " + str(b.device))
        heads = A_log.shape[0]
        pre_b, pre_a = _dense(b), _dense(a)
        rate_log, bias = _f32(A_log), _f32(dt_bias)
        beta = torch.empty(pre_b.shape, dtype=torch.float32, device=b.device)
        g = torch.empty_like(beta)
        if pre_b.numel():
            with _on(b.device):
                N.call("macai_gdr_gates_fwd", N.ptr(pre_b), N.ptr(pre_a), N.ptr(rate_log), N.ptr(bias), N.ptr(beta),
                       N.ptr(g), pre_b.numel(), heads, N.dtype_code(b.dtype, True), N.stream_of(pre_b))
        ctx.save_for_backward(pre_b, pre_a, rate_log, bias)
        ctx.param_dtypes = (A_log.dtype, dt_bias.dtype)
        return beta, g

    @staticmethod
    def backward(ctx, grad_beta, grad_g):
        pre_b, pre_a, rate_log, bias = ctx.saved_tensors
        heads, dev = rate_log.shape[0], pre_b.device
        gb = torch.zeros(pre_b.shape, dtype=torch.float32, device=dev) if grad_beta is None else _f32(grad_beta)
        gg = torch.zeros(pre_b.shape, dtype=torch.float32, device=dev) if grad_g is None else _f32(grad_g)
        d_b, d_a = torch.empty_like(pre_b), torch.empty_like(pre_a)
        need_rate, need_bias = ctx.needs_input_grad[2], ctx.needs_input_grad[3]
        d_rate = d_bias = None
        if need_rate or need_bias:
            d_rate = torch.zeros(heads, dtype=torch.float32, device=dev)
            d_bias = torch.zeros(heads, dtype=torch.float32, device=dev)
        if pre_b.numel():
            with _on(dev):
                N.call("macai_gdr_gates_bwd", N.ptr(pre_b), N.ptr(pre_a), N.ptr(rate_log), N.ptr(bias), N.ptr(gb),
                       N.ptr(gg), N.ptr(d_b), N.ptr(d_a), N.ptr(d_rate), N.ptr(d_bias), pre_b.numel(), heads,
                       N.dtype_code(pre_b.dtype, True), N.stream_of(pre_b))
        rate_dt, bias_dt = ctx.param_dtypes
        return (d_b, d_a, d_rate.to(rate_dt) if need_rate else None, d_bias.to(bias_dt) if need_bias else None)


def gates(b: torch.Tensor, a: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    """(beta, g) with the reference's arguments (layer/_gates.py:120-121)."""
    return Gates.apply(b, a, A_log, dt_bias)

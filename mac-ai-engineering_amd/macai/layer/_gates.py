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


DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _unfit(b, a, A_log, dt_bias):
    """Why the gates cannot take these arguments, or None.  The kernels index b and a by one count n = b.numel() and
    take the head of element i as i mod H, so b and a must agree in shape and dtype and end in the H heads of A_log
    and dt_bias."""
    if not all(isinstance(t, torch.Tensor) for t in (b, a, A_log, dt_bias)):
        return "b, a, A_log and dt_bias must be tensors"
    if b.dtype not in DTYPES or a.dtype != b.dtype:
        return f"b and a must share a dtype among float32, bfloat16, float16 (got {b.dtype}, {a.dtype})"
    if A_log.dtype not in DTYPES or dt_bias.dtype not in DTYPES:
        return f"A_log and dt_bias must be float32, bfloat16 or float16 (got {A_log.dtype}, {dt_bias.dtype})"
    if b.shape != a.shape or b.dim() < 1:
        return f"b and a must have one shape [..., H] (got {tuple(b.shape)}, {tuple(a.shape)})"
    if A_log.dim() != 1 or dt_bias.shape != A_log.shape or b.shape[-1] != A_log.shape[0]:
        return (f"A_log and dt_bias must be [H] with H = b.shape[-1] (got {tuple(A_log.shape)}, "
                f"{tuple(dt_bias.shape)} for b {tuple(b.shape)})")
    if b.numel() >= 2 ** 31:
        return "b and a past 2^31 elements are not supported"
    devs = {t.device for t in (b, a, A_log, dt_bias)}
    if len(devs) != 1:
        return f"b, a, A_log and dt_bias must be on one device (got {sorted(map(str, devs))})"
    return None


def supported(b, a, A_log, dt_bias) -> bool:
    """Whether the HIP gates take these arguments (the reference's test of the same name and signature,
    layer/_gates.py:75): on a HIP device, b and a of one shape [..., H] and dtype, A_log and dt_bias [H]."""
    return isinstance(b, torch.Tensor) and b.is_cuda and _unfit(b, a, A_log, dt_bias) is None


class Gates(torch.autograd.Function):
    """The layer's two gates in one launch: the write strength beta = sigmoid(b) and the log decay
    g = -exp(A_log) softplus(a + dt_bias), both returned in float32."""

    @staticmethod
    def forward(ctx, b, a, A_log, dt_bias):
        why = _unfit(b, a, A_log, dt_bias)
        if why is not None:
            raise ValueError("macai gates: " + why)
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

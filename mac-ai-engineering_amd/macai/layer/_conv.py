"""The linear-attention layer's convolution path as one HIP pass each way (the reference's layer/_conv.py:1-24, 167-241;
entry points macai_gdr_conv_fwd / macai_gdr_conv_bwd of include/macai_gdr.h).

Forward, from the input projection's output x [B, T, C] (C = 2 key_dim + value_dim) and the depthwise taps w [C, 1, 4]:

    u[t, c] = sum_j w[c, j] x[t - 3 + j, c]     (causal, zero before the start; float32)
    y = u sigmoid(u)                             (one rounding)
    q, k = y's first two key_dim channel blocks as [B, T, heads, dk]; v = the last value_dim channels [B, T, ., dv]

With repeat=True (the reference's layout) each key head is written `rep` times, as transformers' repeat_interleave
over the value heads would, and v comes out in float32 (v_dtype); the MI355X rule reads grouped heads natively, so
repeat=False (key heads only) with v in x's dtype is the layout that feeds it without copies.

Backward: dx [B, T, C] in x's dtype (u recomputed from x, dq and dk summed over the copies); the taps' gradient only
when the weight trains (float32 partial sums a tile of 16 time steps, then a fixed-order sum: deterministic).
"""
import torch

from ..gated_delta import _native as N
from ..gated_delta.op import _on

K = 4


def supported(x: torch.Tensor, w: torch.Tensor, kd: int, dk: int, rep: int, dv: int) -> bool:
    """Shapes the kernels take (the reference's rule, layer/_conv.py:174-181, with 8-channel groups)."""
    if x.dim() != 3 or not x.is_cuda or x.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        return False
    C = x.shape[-1]
    vd = C - 2 * kd
    return (w.numel() == C * K and w.shape[-1] == K and C % 8 == 0 and kd % dk == 0 and dk % 8 == 0 and vd > 0
            and dv % 8 == 0 and vd % dv == 0 and (kd // dk) * rep == vd // dv and x.numel() < 2 ** 31
            and x.numel() // C * kd * rep < 2 ** 31)


class ConvQKV(torch.autograd.Function):
    """(q, k, v) = the convolution path of x [B, T, C] (see the module's docstring)."""

    @staticmethod
    def forward(ctx, x, weight, kd: int, dk: int, rep: int, dv: int, repeat: bool = True, v_dtype=torch.float32):
        if not x.is_cuda:
            raise RuntimeError("macai's convolution path runs on a HIP device (MI355X); got " + str(x.device))
        B, T, C = x.shape
        copies = rep if repeat else 1
        xc = x.contiguous()
        w = weight.reshape(C, K).to(torch.float32).contiguous()
        heads = kd // dk * copies
        q = torch.empty((B, T, heads, dk), dtype=x.dtype, device=x.device)
        k = torch.empty((B, T, heads, dk), dtype=x.dtype, device=x.device)
        v = torch.empty((B, T, (C - 2 * kd) // dv, dv), dtype=v_dtype, device=x.device)
        if B * T:
            with _on(x.device):
                N.call("macai_gdr_conv_fwd", N.ptr(xc), N.ptr(w), N.ptr(q), N.ptr(k), N.ptr(v), B, T, C, kd, dk,
                       copies, dv, N.dtype_code(x.dtype, True), N.dtype_code(v_dtype, True), N.stream_of(xc))
        ctx.save_for_backward(xc, w)
        ctx.dims = (kd, dk, copies, dv)
        ctx.wshape, ctx.wdtype, ctx.vdtype = weight.shape, weight.dtype, v_dtype
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk_, dv_):
        xc, w = ctx.saved_tensors
        kd, dk, copies, dv = ctx.dims
        B, T, C = xc.shape
        heads = kd // dk * copies
        dev, dt = xc.device, xc.dtype
        want_dw = ctx.needs_input_grad[1]
        dq = torch.zeros((B, T, heads, dk), dtype=dt, device=dev) if dq is None else dq.to(dt).contiguous()
        dk_ = torch.zeros((B, T, heads, dk), dtype=dt, device=dev) if dk_ is None else dk_.to(dt).contiguous()
        dv_ = (torch.zeros((B, T, (C - 2 * kd) // dv, dv), dtype=ctx.vdtype, device=dev) if dv_ is None
               else dv_.to(ctx.vdtype).contiguous())
        dx = torch.empty_like(xc)
        dwp = dw = None
        if want_dw:
            dwp = torch.empty(N.lib().macai_gdr_conv_partials(B, T, C), dtype=torch.float32, device=dev)
            dw = torch.zeros(C, K, dtype=torch.float32, device=dev)
        if B * T:
            with _on(dev):
                N.call("macai_gdr_conv_bwd", N.ptr(xc), N.ptr(w), N.ptr(dq), N.ptr(dk_), N.ptr(dv_), N.ptr(dx),
                       N.ptr(dwp), N.ptr(dw), B, T, C, kd, dk, copies, dv, N.dtype_code(dt, True),
                       N.dtype_code(ctx.vdtype, True), N.stream_of(xc))
        dwo = dw.view(ctx.wshape).to(ctx.wdtype) if want_dw else None
        return (dx if ctx.needs_input_grad[0] else None), dwo, None, None, None, None, None, None


def conv_qkv(x: torch.Tensor, weight: torch.Tensor, kd: int, dk: int, rep: int, dv: int, repeat: bool = True,
             v_dtype=torch.float32):
    """(q, k, v) of the convolution path: the reference's conv_qkv (layer/_conv.py:240-241) with the same defaults;
    repeat=False and v_dtype=x.dtype give the layout the MI355X rule reads without copies."""
    return ConvQKV.apply(x, weight, kd, dk, rep, dv, repeat, v_dtype)

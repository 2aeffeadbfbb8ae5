"""The linear-attention layer's convolution path, one HIP launch each way (entry points macai_gdr_conv_fwd /
macai_gdr_conv_bwd of include/macai_gdr.h; the function of the reference's layer/_conv.py:1-24).

From the input projection's output x [B, T, C], C = 2 key_dim + value_dim, and depthwise taps w [C, 1, 4]:

    u[t, c] = sum_j w[c, j] x[t - 3 + j, c]      causal, zero before the start, float32
    y       = u sigmoid(u)                        rounded once to the output dtype
    q, k    = y[..., :key_dim], y[..., key_dim:2 key_dim] as heads of dk;  v = y[..., 2 key_dim:] as heads of dv

`repeat=True` (the default) writes every key head `rep` times, the layout transformers' repeat_interleave over the
value heads produces, and v in float32 (`v_dtype`): the reference's outputs.  `repeat=False` keeps the key heads only,
which the MI355X rule reads natively (grouped value heads), and `v_dtype=x.dtype` skips the float32 copy of v.

The backward returns dx in x's dtype (the gradients of a key head's copies summed inside the kernel) and, when the
weight trains, its gradient from per-tile partial sums added in tile order (deterministic).
"""
import torch

from ..gated_delta import _native as N
from ..gated_delta.op import _on

TAPS = 4


class _Split:
    """How the C channels of x split into the outputs, and the output shapes."""

    def __init__(self, shape, kd: int, dk: int, rep: int, dv: int, repeat: bool):
        self.B, self.T, self.C = shape
        self.kd, self.dk, self.dv = kd, dk, dv
        self.copies = rep if repeat else 1        # writes of each key head
        self.qk_shape = (self.B, self.T, kd // dk * self.copies, dk)
        self.v_shape = (self.B, self.T, (self.C - 2 * kd) // dv, dv)

    def dims(self):
        """The size arguments of the two entry points."""
        return self.B, self.T, self.C, self.kd, self.dk, self.copies, self.dv


def _dense(t):
    """t contiguous and 16-byte aligned, as the kernels' vector accesses need (a copy only when it is not)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _upstream(grad, shape, dtype, device):
    """An output's gradient as the kernel reads it: dense, in the output's dtype; zeros when autograd passes None."""
    if grad is None:
        return torch.zeros(shape, dtype=dtype, device=device)
    return _dense(grad if grad.dtype == dtype else grad.to(dtype))


DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _unfit(x, w, kd: int, dk: int, rep: int, dv: int):
    """Why the convolution path cannot take these arguments, or None: x [B, T, C] in one of DTYPES with C = 2 kd +
    value_dim, w of C x 4 taps, kd a whole number of key heads of dk and value_dim of value heads of dv, each value head
    group rep value heads a key head, every width a multiple of 8 (the kernels move 16-byte channel vectors)."""
    if not isinstance(x, torch.Tensor) or not isinstance(w, torch.Tensor):
        return "x and the weight must be tensors"
    if x.dim() != 3:
        return f"x must be [B, T, C] (got {tuple(x.shape)})"
    if x.dtype not in DTYPES:
        return f"x must be float32, bfloat16 or float16 (got {x.dtype})"
    C = x.shape[-1]
    vd = C - 2 * kd
    if w.numel() != C * TAPS or w.shape[-1] != TAPS:
        return f"the weight must hold {TAPS} taps a channel, [C, 1, {TAPS}] (got {tuple(w.shape)} for C = {C})"
    if min(kd, dk, dv, rep) < 1 or vd < 1 or kd % dk or vd % dv or (kd // dk) * rep != vd // dv:
        return (f"need C = 2 key_dim + value_dim with key_dim = key heads x {dk}, value_dim = key heads x rep x {dv} "
                f"(got C {C}, key_dim {kd}, rep {rep})")
    if C % 8 or kd % 8 or dk % 8 or dv % 8:
        return f"C, key_dim and the head widths must be multiples of 8 (got {C}, {kd}, {dk}, {dv})"
    if x.numel() >= 2 ** 31 or x.numel() // C * kd * rep >= 2 ** 31:
        return "tensors past 2^31 elements are not supported"
    if w.device != x.device:
        return f"x and the weight must be on one device (got {x.device}, {w.device})"
    return None


def supported(x: torch.Tensor, w: torch.Tensor, kd: int, dk: int, rep: int, dv: int) -> bool:
    """Whether the HIP convolution path takes these arguments (the reference's test of the same name and signature,
    layer/_conv.py:178): x on a HIP device and the widths the kernels take."""
    return isinstance(x, torch.Tensor) and x.is_cuda and _unfit(x, w, kd, dk, rep, dv) is None


class ConvQKV(torch.autograd.Function):
    """(q, k, v) = the convolution path of x (see the module's docstring)."""

    @staticmethod
    def forward(ctx, x, weight, kd: int, dk: int, rep: int, dv: int, repeat: bool = True, v_dtype=torch.float32):
        why = _unfit(x, weight, kd, dk, rep, dv)
        if why is not None:
            raise ValueError("macai conv_qkv: " + why)
        if not x.is_cuda:
            raise RuntimeError("macai's convolution path runs on a HIP device (MI355X); got " + str(x.device))
        sp = _Split(x.shape, kd, dk, rep, dv, repeat)
        src = _dense(x)
        taps = weight.detach().reshape(sp.C, TAPS).to(torch.float32).contiguous()
        q = torch.empty(sp.qk_shape, dtype=x.dtype, device=x.device)
        k = torch.empty_like(q)
        v = torch.empty(sp.v_shape, dtype=v_dtype, device=x.device)
        if src.numel():
            with _on(x.device):
                N.call("macai_gdr_conv_fwd", N.ptr(src), N.ptr(taps), N.ptr(q), N.ptr(k), N.ptr(v), *sp.dims(),
                       N.dtype_code(x.dtype, True), N.dtype_code(v_dtype, True), N.stream_of(src))
        ctx.save_for_backward(src, taps)
        ctx.split, ctx.v_dtype = sp, v_dtype
        ctx.w_meta = (weight.shape, weight.dtype)
        return q, k, v

    @staticmethod
    def backward(ctx, grad_q, grad_k, grad_v):
        src, taps = ctx.saved_tensors
        sp = ctx.split
        dev = src.device
        gq = _upstream(grad_q, sp.qk_shape, src.dtype, dev)
        gk = _upstream(grad_k, sp.qk_shape, src.dtype, dev)
        gv = _upstream(grad_v, sp.v_shape, ctx.v_dtype, dev)
        dx = torch.empty_like(src)
        train_w = ctx.needs_input_grad[1]
        partials = dw = None
        if train_w:
            partials = torch.empty(N.lib().macai_gdr_conv_partials(sp.B, sp.T, sp.C), dtype=torch.float32, device=dev)
            dw = torch.zeros(sp.C, TAPS, dtype=torch.float32, device=dev)
        if src.numel():
            with _on(dev):
                N.call("macai_gdr_conv_bwd", N.ptr(src), N.ptr(taps), N.ptr(gq), N.ptr(gk), N.ptr(gv), N.ptr(dx),
                       N.ptr(partials), N.ptr(dw), *sp.dims(), N.dtype_code(src.dtype, True),
                       N.dtype_code(ctx.v_dtype, True), N.stream_of(src))
        w_shape, w_dtype = ctx.w_meta
        grad_w = dw.view(w_shape).to(w_dtype) if train_w else None
        return (dx if ctx.needs_input_grad[0] else None), grad_w, None, None, None, None, None, None


def conv_qkv(x: torch.Tensor, weight: torch.Tensor, kd: int, dk: int, rep: int, dv: int, repeat: bool = True,
             v_dtype=torch.float32):
    """(q, k, v) of the convolution path, with the reference's arguments and defaults (layer/_conv.py:240-241);
    repeat=False and v_dtype=x.dtype give the layout the MI355X rule reads without copies."""
    return ConvQKV.apply(x, weight, kd, dk, rep, dv, repeat, v_dtype)

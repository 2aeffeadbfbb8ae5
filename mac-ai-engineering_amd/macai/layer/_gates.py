"""The linear-attention layer's gates as one HIP pass each way (the reference's layer/_gates.py:1-13, 83-121; entry
points macai_gdr_gates_fwd / macai_gdr_gates_bwd of include/macai_gdr.h):

    beta = sigmoid(b)                             (float32)
    g    = -exp(A_log) softplus(a + dt_bias)      (float32; softplus with PyTorch's threshold of 20)

from the [B, T, H] outputs of in_proj_b and in_proj_a (float32, bfloat16 or float16) and A_log, dt_bias [H], written
in float32, the dtype the rule reads them in.  The backward: db = dbeta beta (1 - beta), da = dg (-exp(A_log))
sigmoid(a + dt_bias) (1 above the threshold), in the inputs' dtype; A_log's and dt_bias's gradients only when they
train, summed over the rows by one workgroup a head in a fixed order (the reference uses PyTorch reductions there).
"""
import torch

from ..gated_delta import _native as N
from ..gated_delta.op import _on


def supported(b, a, A_log, dt_bias) -> bool:
    """Shapes the kernels take (the reference's rule, layer/_gates.py:77-79)."""
    return (b.is_cuda and b.dtype == a.dtype and b.shape == a.shape and b.dtype in (torch.float32, torch.bfloat16,
            torch.float16) and A_log.dim() == 1 and dt_bias.shape == A_log.shape and b.shape[-1] == A_log.shape[0]
            and b.numel() < 2 ** 31)


class Gates(torch.autograd.Function):
    """(beta, g) = (sigmoid(b), -exp(A_log) softplus(a + dt_bias)), both float32."""

    @staticmethod
    def forward(ctx, b, a, A_log, dt_bias):
        if not b.is_cuda:
            raise RuntimeError("macai's gates run on a HIP device (MI355X); got " + str(b.device))
        bc, ac = b.contiguous(), a.contiguous()
        al, dtb = A_log.to(torch.float32).contiguous(), dt_bias.to(torch.float32).contiguous()
        n, H = bc.numel(), A_log.shape[0]
        beta = torch.empty(bc.shape, dtype=torch.float32, device=b.device)
        g = torch.empty(bc.shape, dtype=torch.float32, device=b.device)
        if n:
            with _on(b.device):
                N.call("macai_gdr_gates_fwd", N.ptr(bc), N.ptr(ac), N.ptr(al), N.ptr(dtb), N.ptr(beta), N.ptr(g), n,
                       H, N.dtype_code(b.dtype, True), N.stream_of(bc))
        ctx.save_for_backward(bc, ac, al, dtb)
        ctx.pdtypes = (A_log.dtype, dt_bias.dtype)
        return beta, g

    @staticmethod
    def backward(ctx, dbeta, dg):
        bc, ac, al, dtb = ctx.saved_tensors
        n, H = bc.numel(), al.shape[0]
        dev = bc.device
        dbeta = torch.zeros(bc.shape, dtype=torch.float32, device=dev) if dbeta is None else dbeta.float().contiguous()
        dg = torch.zeros(bc.shape, dtype=torch.float32, device=dev) if dg is None else dg.float().contiguous()
        db, da = torch.empty_like(bc), torch.empty_like(ac)
        trained = ctx.needs_input_grad[2] or ctx.needs_input_grad[3]
        dA = ddt = None
        if trained:
            dA = torch.zeros(H, dtype=torch.float32, device=dev)
            ddt = torch.zeros(H, dtype=torch.float32, device=dev)
        if n:
            with _on(dev):
                N.call("macai_gdr_gates_bwd", N.ptr(bc), N.ptr(ac), N.ptr(al), N.ptr(dtb), N.ptr(dbeta), N.ptr(dg),
                       N.ptr(db), N.ptr(da), N.ptr(dA), N.ptr(ddt), n, H, N.dtype_code(bc.dtype, True),
                       N.stream_of(bc))
        dA = dA.to(ctx.pdtypes[0]) if ctx.needs_input_grad[2] else None
        ddt = ddt.to(ctx.pdtypes[1]) if ctx.needs_input_grad[3] else None
        return db, da, dA, ddt


def gates(b: torch.Tensor, a: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    """(beta, g): the reference's gates (layer/_gates.py:120-121)."""
    return Gates.apply(b, a, A_log, dt_bias)

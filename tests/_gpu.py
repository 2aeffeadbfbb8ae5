"""Helpers of the GPU parity tests: run the C-ABI passes one by one and the drop-in, on seeded inputs."""
import math

import torch

from macai.gated_delta import _native as N

C = 64


def passes(q, k, v, g, beta, s0, do, dsT, l2norm=False, q_scale=1.0, split=0):
    """Every pass of a training step through the C ABI; returns a dict of all intermediates and outputs."""
    B, T, H, DK = q.shape
    DV = v.shape[-1]
    NT = math.ceil(T / C)
    dev, dt = q.device, q.dtype
    f32 = torch.float32
    code, st = N.dtype_code(dt), N.stream_of(q)
    r = {}
    e = lambda *s, d=f32: torch.full(s, float("nan"), device=dev, dtype=d)
    r["W"], r["U"], r["M"] = e(B, H, NT, C, DK, d=dt), e(B, H, NT, C, DV), e(B, H, NT, C, C, d=dt)
    N.call("macai_gdr_prep", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g), N.ptr(beta), N.ptr(r["W"]), N.ptr(r["U"]),
           N.ptr(r["M"]), None, None, None, B, T, H, DK, DV, code, int(l2norm), q_scale, st)
    r["Mt"], r["A"], r["At"] = e(B, H, NT, C, C, d=dt), e(B, H, NT, C, C), e(B, H, NT, C, C)
    W2, U2 = e(B, H, NT, C, DK, d=dt), e(B, H, NT, C, DV)
    N.call("macai_gdr_prep", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g), N.ptr(beta), N.ptr(W2), N.ptr(U2), None,
           N.ptr(r["Mt"]), N.ptr(r["A"]), N.ptr(r["At"]), B, T, H, DK, DV, code, int(l2norm), q_scale, st)
    r["o"], r["sT"] = e(B, T, H, DV, d=dt), e(B, H, DK, DV)
    N.call("macai_gdr_state_fwd", N.ptr(q), N.ptr(k), N.ptr(g), N.ptr(r["W"]), N.ptr(r["U"]), N.ptr(r["M"]), N.ptr(s0),
           N.ptr(r["o"]), N.ptr(r["sT"]), None, None, B, T, H, DK, DV, code, int(l2norm), q_scale, 0, split, st)
    r["Sc"], r["Vn"] = e(B, H, NT, DK, DV), e(B, H, NT, C, DV)
    N.call("macai_gdr_state_fwd", N.ptr(q), N.ptr(k), N.ptr(g), N.ptr(W2), N.ptr(U2), None, N.ptr(s0), None, None,
           N.ptr(r["Sc"]), N.ptr(r["Vn"]), B, T, H, DK, DV, code, int(l2norm), q_scale, N.STORE_STATES | N.NO_OUTPUT,
           split, st)
    r["dSn"], r["dVn"], r["ds0"] = e(B, H, NT, DK, DV), e(B, H, NT, C, DV), e(B, H, DK, DV)
    N.call("macai_gdr_state_bwd", N.ptr(q), N.ptr(k), N.ptr(g), N.ptr(W2), N.ptr(r["Mt"]), N.ptr(do), N.ptr(dsT),
           N.ptr(r["dSn"]), N.ptr(r["dVn"]), N.ptr(r["ds0"]), B, T, H, DK, DV, code, int(l2norm), q_scale, split, st)
    r["dq"], r["dk"], r["dv"] = e(B, T, H, DK, d=dt), e(B, T, H, DK, d=dt), e(B, T, H, DV, d=dt)
    r["dg"], r["dbeta"] = e(B, T, H), e(B, T, H)
    N.call("macai_gdr_chunk_bwd", N.ptr(q), N.ptr(k), N.ptr(v), N.ptr(g), N.ptr(beta), N.ptr(do), N.ptr(r["A"]),
           N.ptr(r["At"]), N.ptr(r["Sc"]), N.ptr(r["dSn"]), N.ptr(r["Vn"]), N.ptr(r["dVn"]), N.ptr(r["dq"]),
           N.ptr(r["dk"]), N.ptr(r["dv"]), N.ptr(r["dg"]), N.ptr(r["dbeta"]), B, T, H, DK, DV, code, int(l2norm),
           q_scale, st)
    torch.cuda.synchronize()
    return {k_: x.cpu() for k_, x in r.items()}

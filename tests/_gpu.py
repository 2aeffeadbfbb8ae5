"""Helpers of the GPU parity tests: run the C-ABI passes one by one on seeded inputs."""
import math

import torch

from macai.gated_delta import _native as N
from macai.gated_delta import op

C = 64


def passes(q, k, v, g, beta, s0, do, dsT, l2norm=False, q_scale=1.0, split=0):
    """Every pass of a training step through the C ABI; returns a dict of all intermediates and outputs (CPU)."""
    B, T, H, DK = q.shape
    DV = v.shape[-1]
    NT = math.ceil(T / C)
    dev, dt = q.device, q.dtype
    f32 = torch.float32
    code, st = N.dtype_code(dt), N.stream_of(q)
    split = split or op.split_for(B * H, T, DV)
    P = N.ptr
    r = {}
    e = lambda *s, d=f32: torch.full(s, float("nan"), device=dev, dtype=d)
    # forward-mode prep, then the output pass
    for n_, shape, d in (("W", (B, H, NT, C, DK), dt), ("U", (B, H, NT, C, DV), f32), ("Ke", (B, H, NT, C, DK), dt),
                         ("GL", (B, H, NT), f32), ("Qg", (B, H, NT, C, DK), dt), ("M", (B, H, NT, C, C), dt)):
        r[n_] = e(*shape, d=d)
    N.call("macai_gdr_prep", P(q), P(k), P(v), P(g), P(beta), P(r["W"]), P(r["U"]), P(r["Ke"]), P(r["GL"]),
           P(r["Qg"]), P(r["M"]), None, B, T, H, H, DK, DV, code, int(l2norm), q_scale, None, 0, st)
    r["o"], r["sT"] = e(B, T, H, DV, d=dt), e(B, H, DK, DV)
    N.call("macai_gdr_state_fwd", P(r["W"]), P(r["U"]), P(r["Ke"]), P(r["GL"]), P(r["Qg"]), P(r["M"]), P(s0),
           P(r["o"]), P(r["sT"]), None, None, B, T, H, DK, DV, code, 0, split, None, 0, st)
    # backward-mode prep (adds A), recompute, reverse pass, per-chunk backward
    b2 = {n_: e(*x.shape, d=x.dtype) for n_, x in r.items() if n_ in ("W", "U", "Ke", "GL", "Qg", "M")}
    r["A"] = e(B, H, NT, C, C, d=dt)
    N.call("macai_gdr_prep", P(q), P(k), P(v), P(g), P(beta), P(b2["W"]), P(b2["U"]), P(b2["Ke"]), P(b2["GL"]),
           P(b2["Qg"]), P(b2["M"]), P(r["A"]), B, T, H, H, DK, DV, code, int(l2norm), q_scale, None, 0, st)
    r["Sc"], r["Vn"] = e(B, H, NT, DK, DV), e(B, H, NT, C, DV, d=dt)
    N.call("macai_gdr_state_fwd", P(b2["W"]), P(b2["U"]), P(b2["Ke"]), P(b2["GL"]), None, None, P(s0), None, None,
           P(r["Sc"]), P(r["Vn"]), B, T, H, DK, DV, code, N.STORE_STATES | N.NO_OUTPUT, split, None, 0, st)
    # the training forward's form: output and states in one pass (flags STORE_STATES)
    k2 = {"o": e(B, T, H, DV, d=dt), "sT": e(B, H, DK, DV), "Sc": e(B, H, NT, DK, DV),
          "Vn": e(B, H, NT, C, DV, d=dt)}
    N.call("macai_gdr_state_fwd", P(b2["W"]), P(b2["U"]), P(b2["Ke"]), P(b2["GL"]), P(b2["Qg"]), P(b2["M"]), P(s0),
           P(k2["o"]), P(k2["sT"]), P(k2["Sc"]), P(k2["Vn"]), B, T, H, DK, DV, code, N.STORE_STATES, split, None, 0,
           st)
    r["dSn"], r["dVn"], r["ds0"] = e(B, H, NT, DK, DV), e(B, H, NT, C, DV, d=dt), e(B, H, DK, DV)
    N.call("macai_gdr_state_bwd", P(b2["Ke"]), P(b2["Qg"]), P(b2["W"]), P(b2["M"]), P(b2["GL"]), P(do), P(dsT),
           P(r["dSn"]), P(r["dVn"]), P(r["ds0"]), B, T, H, DK, DV, code, split, None, 0, st)
    r["dq"], r["dk"], r["dv"] = e(B, T, H, DK, d=dt), e(B, T, H, DK, d=dt), e(B, T, H, DV, d=dt)
    r["dg"], r["dbeta"] = e(B, T, H), e(B, T, H)
    N.call("macai_gdr_chunk_bwd", P(q), P(k), P(v), P(g), P(beta), P(do), P(r["A"]), P(r["Sc"]), P(r["dSn"]),
           P(r["Vn"]), P(r["dVn"]), P(r["dq"]), P(r["dk"]), P(r["dv"]), P(r["dg"]), P(r["dbeta"]),
           B, T, H, H, DK, DV, code, int(l2norm), q_scale, None, 0, st)
    torch.cuda.synchronize()
    out = {k_: x.cpu() for k_, x in r.items()}
    out["W2_equal"] = all(torch.equal(b2[n_].cpu(), out[n_]) for n_ in b2)
    # the one-pass output + states must equal the output pass and the recompute pass bit for bit
    out["store_equal"] = all(torch.equal(k2[n_].cpu(), out[n_]) for n_ in k2)
    return out

"""Float64 CPU restatement of the chunked gated delta rule (test infrastructure only; see oracle/__init__.py).

Tensor convention (the reference's, /root/reference/src/macai/gated_delta/op.py:266-269): q, k [B, T, H, DK];
v [B, T, H, DV]; g (log decay, <= 0) and beta [B, T, H]; states [B, H, DK, DV].  q is already l2-normalised and
scaled by DK^-1/2 where a function says "q already normalised" (op.py:117).
"""
import math

import torch

F64 = torch.float64
EPS = 1e-6


def l2norm(x, eps=EPS):
    """y = x * rsqrt(sum(x^2) + eps) over the last dim (op.py:260-261; transformers modeling_qwen3_5.py l2norm)."""
    return x * torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)


def rel(a, r):
    """The reference's error metric: max|a - r| / max|r| (tests/test_harness.py:45-54, tests/test_layer.py:48-49)."""
    a = a.detach().to(F64)
    r = r.detach().to(F64)
    return ((a - r).abs().max() / r.abs().max().clamp_min(1e-300)).item()


# ---------------------------------------------------------------------------------------------------------------------
# the token recurrence (op.py:301-314; _metal.py:5-10; tools/check_chunk_equations.py:11-19)
# ---------------------------------------------------------------------------------------------------------------------
def recurrence(q, k, v, g, beta, s0):
    """S~ = e^{g_t} S; d = beta_t (v_t - S~^T k_t); S = S~ + k_t d^T; o_t = S^T q_t.  Differentiable (autograd)."""
    B, T, H, DK = q.shape
    s = s0
    outs = []
    for t in range(T):
        st = s * g[:, t].exp()[..., None, None]
        u = torch.einsum("bhkv,bhk->bhv", st, k[:, t])
        d = beta[:, t, :, None] * (v[:, t] - u)
        s = st + k[:, t, :, :, None] * d[:, :, None, :]
        outs.append(torch.einsum("bhkv,bhk->bhv", s, q[:, t]))
    return torch.stack(outs, 1), s


def decode_step(q, k, v, g, beta, s):
    """One recurrent step (T = 1; config 4): q, k [B, H, DK] (q normalised and scaled), v [B, H, DV], g, beta [B, H].
    Returns (o [B, H, DV], S').  Follows op.py:308-313 with T = 1 (transformers modeling_qwen3_5.py:365-372)."""
    st = s * g.exp()[..., None, None]
    u = torch.einsum("bhkv,bhk->bhv", st, k)
    d = beta[..., None] * (v - u)
    s2 = st + k[..., :, None] * d[..., None, :]
    return torch.einsum("bhkv,bhk->bhv", s2, q), s2


# ---------------------------------------------------------------------------------------------------------------------
# the chunked forward F1-F5 and backward B1-B6 (_chunked.py:1-35; docs/prior_art_gated_delta.md:132-195;
# tools/check_chunk_equations.py:22-78), batched over (B, H, chunks)
# ---------------------------------------------------------------------------------------------------------------------
def _chunks(x, C):
    """[B, T, H, ...] -> [B, H, NT, C, ...] with zero padding rows (padding carries q = k = v = 0, g = 0, beta = 0)."""
    B, T = x.shape[:2]
    nt = -(-T // C)
    x = x.transpose(1, 2)
    pad = nt * C - T
    if pad:
        x = torch.cat([x, x.new_zeros((x.shape[0], x.shape[1], pad) + tuple(x.shape[3:]))], 2)
    return x.reshape(x.shape[0], x.shape[1], nt, C, *x.shape[3:])


def _unchunk(x, T):
    """[B, H, NT, C, ...] -> [B, T, H, ...]."""
    B, H, nt, C = x.shape[:4]
    x = x.reshape(B, H, nt * C, *x.shape[4:])[:, :, :T]
    return x.transpose(1, 2).contiguous()


def chunk_prep(k, v, g, beta, q=None, C=64):
    """F1-F3 (+ M of F5) for every chunk independently: returns dict with G, gam, e, Gam, KK, L, A, W, U (and M)."""
    K, V, gc, bc = _chunks(k, C), _chunks(v, C), _chunks(g, C), _chunks(beta, C)
    G = torch.cumsum(gc, -1)                                                 # F1
    gam = torch.exp(G)
    e = torch.exp(G[..., -1:] - G)
    diff = G[..., :, None] - G[..., None, :]
    lowi = torch.ones(C, C, dtype=torch.bool).tril(0)
    low = torch.ones(C, C, dtype=torch.bool).tril(-1)
    Gam = torch.where(lowi, torch.exp(torch.where(lowi, diff, torch.zeros_like(diff))), torch.zeros_like(diff))
    KK = K @ K.transpose(-1, -2)                                             # F2
    L = torch.where(low, bc[..., :, None] * KK * Gam, torch.zeros_like(KK))
    eye = torch.eye(C, dtype=K.dtype)
    A = torch.linalg.solve_triangular(eye + L, eye.expand_as(L), upper=False, unitriangular=True)
    W = A @ ((bc * gam)[..., None] * K)                                      # F3
    U = A @ (bc[..., None] * V)
    out = dict(G=G, gam=gam, e=e, Gam=Gam, KK=KK, L=L, A=A, W=W, U=U, low=low, K=K, V=V, beta=bc)
    if q is not None:
        Q = _chunks(q, C)
        out["Q"] = Q
        out["M"] = Gam * (Q @ K.transpose(-1, -2))                           # F5 (lower with the diagonal)
    return out


# Planted mistakes (test infrastructure: tests/test_oracle.py checks that the GPU chain tests' inputs and bars catch
# each one).  "fwd_gamma_sq" / "bwd_gamma_sq": the carried state (forward) or state gradient (reverse pass) decays by
# gamma_last^2 instead of gamma_last; "fwd_glast_off" / "bwd_glast_off": the chain takes G_last from the row before the
# chunk's last (both the carried decay gamma_last and e_r = exp(G_last - G_r)).
PLANTS = ("fwd_gamma_sq", "fwd_glast_off", "bwd_gamma_sq", "bwd_glast_off")
# Operand classes a bf16 MFMA product can take rounded (the rest is fp32): prep's stored W, Ke = diag(e) K,
# Qg = diag(gamma) Q, M and A; the state S and its gradient dS as product operands; Vn and dVn; the per-chunk
# backward's chunk state in dO S_c^T ("Sc") and in dW = -dVn S_c^T ("ScW"), its normalised q, k ("QK") and the
# intermediates it forms and feeds to further products ("CC": dM, dW, dA, dA A^T and the decayed dL).  `rnd` rounds
# the named classes to bf16 where they enter a product (the precision model of the bf16 path; no rounding by default).
ROUNDABLE = ("W", "Ke", "Qg", "M", "A", "S", "dS", "Vn", "dVn", "Sc", "ScW", "QK", "CC")
# The classes the bf16 kernels round: all but QK (they take the raw bf16 q, k, exact, and apply the norms in fp32) and
# Sc (the per-chunk backward takes the fp32 chunk state into dO S_c^T as a hi + lo pair of bf16 fragments).  With
# these the model gives the kernels' outputs and gradients to about three digits on the draws compared (the smoke's,
# draws with large starting states and draws with a final-state gradient over the bar).
BF16_PATH = tuple(c for c in ROUNDABLE if c not in ("QK", "Sc"))
# A class the bf16 kernels do NOT round, for design analysis: "ScDot" rounds Sc in the last-row dg term <Sc, dSn> too,
# as storing the chunk states in bf16 would (tests/test_oracle.py::test_chunk_states_stay_float32 shows the cost).
NOT_ROUNDED = ("ScDot",)


def bf16(x):
    """x rounded to bfloat16 (round to nearest even) and back to its dtype."""
    return x.to(torch.bfloat16).to(x.dtype)


def _rounder(rnd):
    bad = set(rnd) - set(ROUNDABLE) - set(NOT_ROUNDED)
    assert not bad, bad
    return lambda name, x: bf16(x) if name in rnd else x


def _chain_decays(P, c, plant, side):
    """(gamma_last [B,H,1,1], e [B,H,C,1]) the forward (side "fwd") or reverse ("bwd") chain uses at chunk c."""
    G = P["G"][:, :, c]
    gl, e = P["gam"][:, :, c, -1], P["e"][:, :, c]
    if plant == side + "_glast_off":
        gl, e = torch.exp(G[..., -2]), torch.exp(G[..., -2:-1] - G)
    if plant == side + "_gamma_sq":
        gl = gl * gl
    return gl[..., None, None], e[..., :, None]


def chunked_forward(q, k, v, g, beta, s0, C=64, plant=None, rnd=()):
    """F1-F5 (q already normalised and scaled).  Returns (o [B,T,H,DV], sT [B,H,DK,DV], P) where P holds the per-chunk
    intermediates: everything of chunk_prep plus Sc [B,H,NT,DK,DV] (state entering each chunk) and Vn [B,H,NT,C,DV].
    plant: one of PLANTS (a deliberate mistake, for the tests' teeth); rnd: operand classes of ROUNDABLE rounded to
    bf16 where they enter a product."""
    assert plant is None or plant in PLANTS, plant
    R = _rounder(rnd)
    T = q.shape[1]
    P = chunk_prep(k, v, g, beta, q, C)
    nt = P["G"].shape[2]
    S = s0.clone()
    Sc, Vn, O = [], [], []
    for c in range(nt):
        Sc.append(S)
        Sop = R("S", S)
        vn = P["U"][:, :, c] - R("W", P["W"][:, :, c]) @ Sop                   # F4
        vop = R("Vn", vn)
        if "Qg" in rnd:
            qs = R("Qg", P["gam"][:, :, c, :, None] * P["Q"][:, :, c]) @ Sop
        else:
            qs = P["gam"][:, :, c, :, None] * (P["Q"][:, :, c] @ Sop)
        O.append(qs + R("M", P["M"][:, :, c]) @ vop)                             # F5
        Vn.append(vn)
        gl, e = _chain_decays(P, c, plant, "fwd")
        if "Ke" in rnd:
            S = gl * S + R("Ke", e * P["K"][:, :, c]).transpose(-1, -2) @ vop
        else:
            S = gl * S + P["K"][:, :, c].transpose(-1, -2) @ (e * vop)
    P["Sc"] = torch.stack(Sc, 2)
    P["Vn"] = torch.stack(Vn, 2)
    return _unchunk(torch.stack(O, 2), T), S, P


def chunked_forward_segments(q, k, v, g, beta, s0, C=64, seg=4096, plant=None):
    """chunked_forward over segments of `seg` tokens (a multiple of C), the state carried between them: the same
    arithmetic chunk by chunk with bounded memory, for long sequences.  Returns (o, sT).  plant: as chunked_forward."""
    assert seg % C == 0
    S, outs = s0, []
    for t0 in range(0, q.shape[1], seg):
        sl = slice(t0, t0 + seg)
        o, S, _ = chunked_forward(q[:, sl], k[:, sl], v[:, sl], g[:, sl], beta[:, sl], S, C, plant=plant)
        outs.append(o)
    return torch.cat(outs, 1), S


def segment_map(q, k, v, g, beta, C=64):
    """The chunked state pass (F3-F4) as an affine map of its starting state: (A [B,H,DK,DK], Bm [B,H,DK,DV]) with
    S_end = A S_0 + Bm, composed chunk by chunk: S <- (gamma_last I - K^T diag(e) W) S + K^T diag(e) U.  The product's
    sequence-parallel forward splits a row into segments by this map (no reference counterpart: the reference walks
    a row in one chain); pinned in tests/test_oracle.py against chunked_forward."""
    P = chunk_prep(k, v, g, beta, None, C)
    B, H, nt = P["G"].shape[:3]
    DK, DV = k.shape[-1], v.shape[-1]
    eye = torch.eye(DK, dtype=k.dtype)
    A = eye.expand(B, H, DK, DK).clone()
    Bm = torch.zeros(B, H, DK, DV, dtype=k.dtype)
    for c in range(nt):
        KeT = (P["e"][:, :, c, :, None] * P["K"][:, :, c]).transpose(-1, -2)
        Ac = P["gam"][:, :, c, -1, None, None] * eye - KeT @ P["W"][:, :, c]
        A, Bm = Ac @ A, Ac @ Bm + KeT @ P["U"][:, :, c]
    return A, Bm


def chunked_backward(q, k, v, g, beta, s0, do, dsT, C=64, P=None, plant=None, rnd=()):
    """B1-B6 (q already normalised and scaled), dg in the reference's no-cancellation form (_chunked.py:1138-1176).
    Returns (dq, dk, dv, dg, dbeta, ds0) and the intermediates dict (adds dSn = dS_{c+1} per chunk and dVn).  plant and
    rnd as for chunked_forward (a forward plant or rounding applies to the forward that P comes from)."""
    assert plant is None or plant in PLANTS, plant
    R = _rounder(rnd)
    T = q.shape[1]
    if P is None:
        _, _, P = chunked_forward(q, k, v, g, beta, s0, C, plant=plant, rnd=rnd)
    dO = _chunks(do, C)
    nt = P["G"].shape[2]
    gam, e, Gam, A, W, M, K, V, Q, bc = (P[n] for n in ("gam", "e", "Gam", "A", "W", "M", "K", "V", "Q", "beta"))
    low = P["low"]
    dS = dsT.clone()
    dSn, dVn = [None] * nt, [None] * nt
    for c in reversed(range(nt)):
        dSn[c] = dS
        gl, ec = _chain_decays(P, c, plant, "bwd")
        dop = R("dS", dS)
        if "Ke" in rnd:
            kds = R("Ke", ec * K[:, :, c]) @ dop
        else:
            kds = ec * (K[:, :, c] @ dop)
        dvn = R("M", M[:, :, c]).transpose(-1, -2) @ dO[:, :, c] + kds                                    # B1
        if "Qg" in rnd:
            qdo = R("Qg", gam[:, :, c, :, None] * Q[:, :, c]).transpose(-1, -2) @ dO[:, :, c]
        else:
            qdo = (gam[:, :, c, :, None] * Q[:, :, c]).transpose(-1, -2) @ dO[:, :, c]
        dS = gl * dS + qdo - R("W", W[:, :, c]).transpose(-1, -2) @ R("dVn", dvn)                           # B2
        dVn[c] = dvn
    dSn = torch.stack(dSn, 2)
    dVn = torch.stack(dVn, 2)
    Sc, Vn = P["Sc"], P["Vn"]
    tr = lambda x: x.transpose(-1, -2)
    Ar, Scr, Vnr, dVnr, Kr, Qr = R("A", A), R("Sc", Sc), R("Vn", Vn), R("dVn", dVn), R("QK", K), R("QK", Q)
    dOVt = dO @ tr(Vnr)                                                    # B3
    dM = Gam * dOVt
    dMr = R("CC", dM)
    dOSt = dO @ tr(Scr)
    dQ = gam[..., None] * dOSt + dMr @ Kr
    VndSt = Vnr @ tr(dSn)
    dK = tr(dMr) @ Qr + e[..., None] * VndSt
    dW = -dVnr @ tr(R("ScW", Sc))
    dWr = R("CC", dW)
    X, Y = tr(Ar) @ dWr, tr(Ar) @ dVnr                                     # B5
    bg = bc * gam
    dK = dK + bg[..., None] * X
    dV = bc[..., None] * Y
    dA = torch.where(low, dWr @ tr(bg[..., None] * Kr) + dVnr @ tr(bc[..., None] * V), torch.zeros_like(A))
    dL = torch.where(low, -tr(Ar) @ R("CC", R("CC", dA) @ tr(Ar)), torch.zeros_like(A))
    Pm = dL * Gam
    Pr = R("CC", Pm)
    dK = dK + bc[..., None] * (Pr @ Kr) + tr(Pr) @ (bc[..., None] * Kr)
    KG = P["KK"] * Gam
    R2 = dL * KG
    kx = (K * X).sum(-1)
    dbeta = gam * kx + (V * Y).sum(-1) + R2.sum(-1)
    # dG: the terms through gamma (Q S_c and W), the decays of M and L (row sum minus column sum of their strictly lower
    # parts), gamma_last's own term on the last row; then dg_t = sum_{s>=t} dG_s + sum_{r<t} e_r k_r.(Vn dSn^T)_r
    dG = gam * (Q * dOSt).sum(-1) + bg * kx
    R1 = torch.where(low, dOVt * M, torch.zeros_like(M))
    dG = dG + R1.sum(-1) - R1.sum(-2)
    dG = dG + bc * R2.sum(-1) - (bc[..., :, None] * R2).sum(-2)
    dG[..., -1] = dG[..., -1] + gam[..., -1] * (R("ScDot", Sc) * dSn).sum((-1, -2))
    E = e * (K * VndSt).sum(-1)
    # exclusive prefix by shifting first: cumsum(E) - E would cancel E_t (O(1) on the last row) against the O(e^g)
    # earlier terms under strong decay
    Ex = torch.cat([torch.zeros_like(E[..., :1]), E[..., :-1]], -1)
    dg = torch.flip(torch.cumsum(torch.flip(dG, [-1]), -1), [-1]) + torch.cumsum(Ex, -1)
    P = dict(P, dSn=dSn, dVn=dVn)
    return (_unchunk(dQ, T), _unchunk(dK, T), _unchunk(dV, T), _unchunk(dg, T), _unchunk(dbeta, T), dS), P


# ---------------------------------------------------------------------------------------------------------------------
# the drop-in in float64 (op.py:264-298): prologue + rule, outputs and gradients w.r.t. the raw inputs
# ---------------------------------------------------------------------------------------------------------------------
def prologue(query, key, use_qk_l2norm_in_kernel=True):
    """q = l2norm(query) * DK^-1/2, k = l2norm(key) (op.py:276-283; _norm.py:1-10)."""
    q, k = query, key
    if use_qk_l2norm_in_kernel:
        q, k = l2norm(q), l2norm(k)
    return q * q.shape[-1] ** -0.5, k


def dropin_f64(query, key, value, g, beta, initial_state=None, do=None, dsT=None, use_qk_l2norm_in_kernel=True,
               C=64, plant=None, rnd=()):
    """The drop-in in float64 from the given (dtype-representable) values: returns (o, sT, grads) with grads a dict of
    dquery, dkey, dvalue, dg, dbeta, dstate (None without do / dsT).  Chunked F/B equations; the prologue's gradient by
    autograd.  Every tensor is upcast to float64 first.  plant, rnd: as for chunked_forward (test infrastructure)."""
    query, key, value, g, beta = (x.detach().to(F64) for x in (query, key, value, g, beta))
    B, T, H, DK = query.shape
    DV = value.shape[-1]
    s0 = torch.zeros(B, H, DK, DV, dtype=F64) if initial_state is None else initial_state.detach().to(F64)
    qr = query.clone().requires_grad_(True)
    kr = key.clone().requires_grad_(True)
    q, k = prologue(qr, kr, use_qk_l2norm_in_kernel)
    o, sT, P = chunked_forward(q.detach(), k.detach(), value, g, beta, s0, C, plant=plant, rnd=rnd)
    if do is None and dsT is None:
        return o, sT, None
    do = torch.zeros_like(o) if do is None else do.detach().to(F64)
    dsT = torch.zeros_like(sT) if dsT is None else dsT.detach().to(F64)
    (dq, dk, dv, dg, db, ds0), _ = chunked_backward(q.detach(), k.detach(), value, g, beta, s0, do, dsT, C, P,
                                                    plant=plant, rnd=rnd)
    torch.autograd.backward([q, k], [dq, dk])
    grads = dict(dquery=qr.grad, dkey=kr.grad, dvalue=dv, dg=dg, dbeta=db, dstate=ds0)
    return o, sT, grads


# ---------------------------------------------------------------------------------------------------------------------
# transformers' torch_chunk_gated_delta_rule, restated (the reference torch path; error anchor of the parity bar).
# Installed transformers 5.15.0 modeling_qwen3_5.py:248-327; the reference pins 5.22.1, which casts to float32 before the
# l2norm and inverts with solve_triangular (bench/profile_gated_delta.py:37-86; docs/prior_art_gated_delta.md:319-327).
# ---------------------------------------------------------------------------------------------------------------------
def torch_chunk_gated_delta_rule(query, key, value, g, beta, chunk_size=64, initial_state=None,
                                 output_final_state=False, use_qk_l2norm_in_kernel=False, cast_first=True,
                                 compute_dtype=torch.float32, inverse="rowloop"):
    """cast_first=True: cast to compute_dtype, then l2norm (5.22.1 and macai's prologue order); False: l2norm in the
    input dtype first (5.15.0).  inverse: "rowloop" (5.15.0's in-place row recursion) or "solve" (5.22.1)."""
    initial_dtype = query.dtype
    if not cast_first and use_qk_l2norm_in_kernel:
        query, key = l2norm(query), l2norm(key)
    query, key, value, beta, g = (x.transpose(1, 2).contiguous().to(compute_dtype) for x in (query, key, value, beta, g))
    if cast_first and use_qk_l2norm_in_kernel:
        query, key = l2norm(query), l2norm(key)
    B, H, T, DK = key.shape
    DV = value.shape[-1]
    C = chunk_size
    pad = (C - T % C) % C
    query, key, value = (torch.nn.functional.pad(x, (0, 0, 0, pad)) for x in (query, key, value))
    beta, g = torch.nn.functional.pad(beta, (0, pad)), torch.nn.functional.pad(g, (0, pad))
    Tp = T + pad
    query = query * (1 / (DK ** 0.5))
    v_beta = value * beta.unsqueeze(-1)
    k_beta = key * beta.unsqueeze(-1)
    query, key, value, k_beta, v_beta = (x.reshape(B, H, -1, C, x.shape[-1]) for x in (query, key, value, k_beta, v_beta))
    g = g.reshape(B, H, -1, C)
    upper0 = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=0)
    g = g.cumsum(dim=-1)
    decay = ((g.unsqueeze(-1) - g.unsqueeze(-2)).tril().exp()).tril()   # transformers' .float() is a no-op here
    attn = -((k_beta @ key.transpose(-1, -2)) * decay).masked_fill(upper0, 0)
    if inverse == "rowloop":
        for i in range(1, C):
            row = attn[..., i, :i].clone()
            sub = attn[..., :i, :i].clone()
            attn[..., i, :i] = row + (row.unsqueeze(-1) * sub).sum(-2)
        attn = attn + torch.eye(C, dtype=attn.dtype)
    else:
        eye = torch.eye(C, dtype=attn.dtype)
        attn = torch.linalg.solve_triangular(eye - attn, eye.expand_as(attn), upper=False, unitriangular=True)
    value = attn @ v_beta
    k_cumdecay = attn @ (k_beta * g.exp().unsqueeze(-1))
    S = (torch.zeros(B, H, DK, DV, dtype=compute_dtype) if initial_state is None else initial_state.to(compute_dtype))
    out = torch.zeros_like(value)
    upper1 = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=1)
    for i in range(Tp // C):
        q_i, k_i, v_i = query[:, :, i], key[:, :, i], value[:, :, i]
        attn_i = (q_i @ k_i.transpose(-1, -2) * decay[:, :, i]).masked_fill_(upper1, 0)
        v_new = v_i - k_cumdecay[:, :, i] @ S
        out_i = (q_i * g[:, :, i, :, None].exp()) @ S + attn_i @ v_new
        out = out.clone()
        out[:, :, i] = out_i
        S = S * g[:, :, i, -1, None, None].exp() + (k_i * (g[:, :, i, -1, None] - g[:, :, i]).exp()[..., None]).transpose(-1, -2) @ v_new
    out = out.reshape(B, H, -1, DV)[:, :, :T].transpose(1, 2).contiguous().to(initial_dtype)
    return out, (S if output_final_state else None)


# ---------------------------------------------------------------------------------------------------------------------
# seeded synthetic inputs (the draw order of the measurement plan: q, k, v, u_g, x_g, x_beta, s0, dO)
# ---------------------------------------------------------------------------------------------------------------------
CONFIGS = {
    0: dict(B=1, T=256, Hk=4, Hv=4, DK=64, DV=64, dtype=torch.float32, s0=False, grads=False),
    1: dict(B=4, T=1024, Hk=16, Hv=16, DK=128, DV=128, dtype=torch.bfloat16, s0=False, grads=True),
    2: dict(B=2, T=1024, Hk=16, Hv=32, DK=128, DV=128, dtype=torch.bfloat16, s0=True, grads=True),
    3: dict(B=1, T=32768, Hk=16, Hv=16, DK=128, DV=128, dtype=torch.bfloat16, s0=False, grads=False),
    4: dict(B=64, T=1, Hk=16, Hv=32, DK=128, DV=128, dtype=torch.bfloat16, s0=True, grads=False),
}


def make_inputs(B, T, Hk, Hv, DK, DV, dtype=torch.float32, s0=False, seed=0, dsT=False):
    """q, k, v ~ N(0,1) (q, k drawn per key head and repeated over the Hv / Hk value heads of each); beta =
    sigmoid(N(0,1)); g = -exp(u) softplus(x), u ~ U(0, ln 16) per value head (the model's A_log), x ~ N(0,1) per token;
    s0 ~ N(0, 0.02); dO ~ N(0,1).  Drawn in float64 from a seeded CPU generator, q/k/v/dO cast to dtype, g/beta/s0
    float32.  Returns a dict of CPU tensors."""
    gen = torch.Generator().manual_seed(seed)
    rep = Hv // Hk
    q = torch.randn(B, T, Hk, DK, generator=gen, dtype=F64).repeat_interleave(rep, 2)
    k = torch.randn(B, T, Hk, DK, generator=gen, dtype=F64).repeat_interleave(rep, 2)
    v = torch.randn(B, T, Hv, DV, generator=gen, dtype=F64)
    u = torch.rand(Hv, generator=gen, dtype=F64) * math.log(16.0)
    xg = torch.randn(B, T, Hv, generator=gen, dtype=F64)
    xb = torch.randn(B, T, Hv, generator=gen, dtype=F64)
    g = -torch.exp(u) * torch.nn.functional.softplus(xg)
    beta = torch.sigmoid(xb)
    st = (torch.randn(B, Hv, DK, DV, generator=gen, dtype=F64) * 0.02) if s0 else None
    do = torch.randn(B, T, Hv, DV, generator=gen, dtype=F64)
    out = dict(query=q.to(dtype), key=k.to(dtype), value=v.to(dtype), g=g.float(), beta=beta.float(),
               initial_state=None if st is None else st.float(), do=do.to(dtype))
    if dsT:
        out["dsT"] = torch.randn(B, Hv, DK, DV, generator=gen, dtype=F64).float()
    return out


def config_inputs(cfg, seed=None, **over):
    """Inputs of BASELINE config `cfg` (seed 1000 + cfg unless given); keyword overrides replace config fields."""
    c = dict(CONFIGS[cfg], **over)
    return make_inputs(c["B"], c["T"], c["Hk"], c["Hv"], c["DK"], c["DV"], c["dtype"], c["s0"],
                       1000 + cfg if seed is None else seed)


def harness_inputs(B, T, H, DK, DV, seed=0, beta=None, g=None, state=True, corr=0.0):
    """The reference harness's generator (tests/test_harness.py:19-31), restated: float64, q normalised and scaled, k
    normalised (corr > 0: keys share a direction, k_i . k_j -> 1), g = -U(0,1) or constant, beta = U(0,1) or constant,
    s0 ~ 0.1 N(0,1) or zeros."""
    gen = torch.Generator().manual_seed(seed)
    q = l2norm(torch.randn(B, T, H, DK, generator=gen, dtype=F64)) * DK ** -0.5
    k = torch.randn(B, T, H, DK, generator=gen, dtype=F64)
    if corr:
        k = corr * torch.randn(B, 1, H, DK, generator=gen, dtype=F64) + (1 - corr) * k
    k = l2norm(k)
    v = torch.randn(B, T, H, DV, generator=gen, dtype=F64)
    gg = -torch.rand(B, T, H, generator=gen, dtype=F64) if g is None else torch.full((B, T, H), float(g), dtype=F64)
    bb = torch.rand(B, T, H, generator=gen, dtype=F64) if beta is None else torch.full((B, T, H), float(beta), dtype=F64)
    s0 = (torch.randn(B, H, DK, DV, generator=gen, dtype=F64) * 0.1) if state else torch.zeros(B, H, DK, DV, dtype=F64)
    return q, k, v, gg, bb, s0

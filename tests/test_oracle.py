"""The CPU oracle pinned (no GPU): the chunked equations against autograd through the recurrence, closed forms that a
dropped term, a wrong sign or a transposed operand would break, the transformers restatement against the installed
transformers function, and the golden fixture (tests/golden/dropin_small.npz)."""
import os

import numpy as np
import pytest
import torch

import _chain
from oracle import gdr

F64 = torch.float64
HERE = os.path.dirname(os.path.abspath(__file__))


def _grads_autograd(q, k, v, g, b, s0, do, dsT):
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, g, b, s0)]
    o, sT = gdr.recurrence(*leaves)
    grads = torch.autograd.grad((o * do).sum() + (sT * dsT).sum(), leaves)
    return o.detach(), sT.detach(), grads


@pytest.mark.parametrize("shape,C,gconst", [((1, 21, 1, 6, 5), 8, None),       # tools/check_chunk_equations.py:8
                                            ((2, 37, 3, 16, 8), 8, None),
                                            ((1, 21, 1, 6, 5), 8, -20.0),       # strong decay (test_harness.py:79)
                                            ((1, 70, 2, 8, 8), 64, None),       # the kernels' chunk, ragged tail
                                            ((1, 130, 1, 8, 4), 64, 0.0)])      # no decay, three chunks
def test_chunked_equations_match_the_recurrence(shape, C, gconst):
    """F1-F5 and B1-B6 (no-cancellation dg) vs autograd through the token recurrence, float64: < 1e-12 relative
    (reference tests/test_chunk_equations.py:13-14)."""
    q, k, v, g, b, s0 = gdr.harness_inputs(*shape, seed=1, g=gconst)
    gen = torch.Generator().manual_seed(5)
    do = torch.randn(q.shape[:3] + (v.shape[-1],), generator=gen, dtype=F64)
    dsT = torch.randn(s0.shape, generator=gen, dtype=F64)
    o, sT, grads = _grads_autograd(q, k, v, g, b, s0, do, dsT)
    oc, sc, P = gdr.chunked_forward(q, k, v, g, b, s0, C)
    mine, _ = gdr.chunked_backward(q, k, v, g, b, s0, do, dsT, C, P)
    errs = [gdr.rel(oc, o), gdr.rel(sc, sT)] + [gdr.rel(a, r) for a, r in zip(mine, grads)]
    assert len(errs) == 8 and max(errs) < 1e-12, errs


def test_dg_keeps_relative_precision_under_strong_decay():
    """With g = -20 every dg is ~1e-9 of the other gradients; the no-cancellation form keeps it to ~1e-8 relative,
    where the naive q.dQ - k.dK form loses it entirely (the reference's docs/series_phase3.md:65-66)."""
    q, k, v, g, b, s0 = gdr.harness_inputs(1, 40, 1, 8, 8, seed=2, g=-20.0)
    gen = torch.Generator().manual_seed(3)
    do = torch.randn(1, 40, 1, 8, generator=gen, dtype=F64)
    dsT = torch.randn(1, 1, 8, 8, generator=gen, dtype=F64)
    _, _, grads = _grads_autograd(q, k, v, g, b, s0, do, dsT)
    (_, _, _, dg, _, _), _ = gdr.chunked_backward(q, k, v, g, b, s0, do, dsT, 8)
    assert grads[3].abs().max() < 1e-7
    assert gdr.rel(dg, grads[3]) < 1e-6


def test_beta_zero_is_pure_decay():
    """beta = 0: S_T = exp(sum g) S_0 and o_t = exp(G_t) S_0^T q_t, by hand."""
    q, k, v, g, b, s0 = gdr.harness_inputs(2, 50, 2, 16, 8, seed=4, beta=0.0)
    o, sT, _ = gdr.chunked_forward(q, k, v, g, b, s0, 64)
    G = g.cumsum(1)
    o_hand = torch.einsum("bth,bhkv,bthk->bthv", G.exp(), s0, q)
    sT_hand = s0 * G[:, -1].exp()[..., None, None]
    assert gdr.rel(o, o_hand) < 1e-13 and gdr.rel(sT, sT_hand) < 1e-13
    o2, sT2 = gdr.recurrence(q, k, v, g, b, s0)
    assert gdr.rel(o2, o_hand) < 1e-13 and gdr.rel(sT2, sT_hand) < 1e-13


def test_orthonormal_keys_recall_exactly():
    """g = 0, beta = 1, keys = distinct basis vectors: the delta rule overwrites row k_t of S with v_t, so S_t^T k_t =
    v_t after every token and S_T's untouched rows keep S_0."""
    T, DK, DV = 12, 16, 5
    q, _, v, _, _, s0 = gdr.harness_inputs(1, T, 1, DK, DV, seed=6)
    k = torch.zeros(1, T, 1, DK, dtype=F64)
    perm = torch.randperm(DK, generator=torch.Generator().manual_seed(1))[:T]
    k[0, torch.arange(T), 0, perm] = 1.0
    g = torch.zeros(1, T, 1, dtype=F64)
    b = torch.ones(1, T, 1, dtype=F64)
    for run in (lambda: gdr.recurrence(q, k, v, g, b, s0)[1], lambda: gdr.chunked_forward(q, k, v, g, b, s0, 8)[1]):
        sT = run()
        expect = s0.clone()
        expect[0, 0, perm] = v[0, :, 0]
        assert gdr.rel(sT, expect) < 1e-14


def test_one_step_by_hand():
    """T = 1 (the decode step): S' = e^g S + beta k (v - e^g S^T k)^T, o = S'^T q, written out element by element."""
    gen = torch.Generator().manual_seed(8)
    DK, DV = 3, 2
    q, k = torch.randn(DK, generator=gen, dtype=F64), torch.randn(DK, generator=gen, dtype=F64)
    v, S = torch.randn(DV, generator=gen, dtype=F64), torch.randn(DK, DV, generator=gen, dtype=F64)
    g, b = -0.7, 0.3
    a = np.exp(g)
    Sh = np.zeros((DK, DV))
    oh = np.zeros(DV)
    for j in range(DV):
        u = sum(a * S[i, j].item() * k[i].item() for i in range(DK))
        d = b * (v[j].item() - u)
        for i in range(DK):
            Sh[i, j] = a * S[i, j].item() + k[i].item() * d
        oh[j] = sum(Sh[i, j] * q[i].item() for i in range(DK))
    o1, S1 = gdr.decode_step(q[None, None], k[None, None], v[None, None], torch.tensor([[g]], dtype=F64),
                             torch.tensor([[b]], dtype=F64), S[None, None])
    assert np.abs(S1[0, 0].numpy() - Sh).max() < 1e-14 and np.abs(o1[0, 0].numpy() - oh).max() < 1e-14
    o2, S2 = gdr.recurrence(q[None, None, None], k[None, None, None], v[None, None, None],
                            torch.tensor([[[g]]], dtype=F64), torch.tensor([[[b]]], dtype=F64), S[None, None])
    assert torch.equal(o2[:, 0], o1) and torch.equal(S2, S1)


def test_strong_decay_resets_the_state():
    """g = -20: the state keeps ~2e-9 of its past each token, so S_t = beta_t k_t v_t^T to ~1e-8."""
    q, k, v, _, b, s0 = gdr.harness_inputs(1, 9, 1, 8, 8, seed=9)
    g = torch.full((1, 9, 1), -20.0, dtype=F64)
    _, sT = gdr.recurrence(q, k, v, g, b, s0)
    expect = b[0, -1, 0] * torch.outer(k[0, -1, 0], v[0, -1, 0])
    assert (sT[0, 0] - expect).abs().max() < 1e-7


def test_inverse_is_unit_lower_and_inverts():
    """A (I + L) = I with A unit lower triangular, also for nearly parallel keys (test_harness.py:86-91)."""
    q, k, v, g, b, s0 = gdr.harness_inputs(1, 96, 2, 32, 8, seed=6, corr=0.9, beta=1 - 1e-6, g=0.0)
    P = gdr.chunk_prep(k, v, g, b, q, 64)
    I = torch.eye(64, dtype=F64)
    assert (P["A"] @ (I + P["L"]) - I).abs().max() < 1e-9
    assert torch.equal(P["A"].triu(1), torch.zeros_like(P["A"]))
    assert torch.equal(P["A"].diagonal(dim1=-2, dim2=-1), torch.ones(1, 2, 2, 64, dtype=F64))


def test_chunk_size_invariance():
    """In exact arithmetic the chunking changes nothing (docs/series_layer.md:1643): C in {8, 16, 64}, float64."""
    xs = gdr.harness_inputs(2, 150, 2, 16, 16, seed=10)
    outs = [gdr.chunked_forward(*xs, C)[:2] for C in (8, 16, 64)]
    for o, sT in outs[1:]:
        assert gdr.rel(o, outs[0][0]) < 1e-12 and gdr.rel(sT, outs[0][1]) < 1e-12


def test_recurrence_gradcheck():
    """torch.autograd.gradcheck (float64 finite differences) of the recurrence on a tiny shape: the truth the chunked
    backward is compared with is the true derivative."""
    xs = [x.requires_grad_(True) for x in gdr.harness_inputs(1, 5, 1, 3, 2, seed=11)]
    assert torch.autograd.gradcheck(lambda *a: gdr.recurrence(*a), xs, eps=1e-6, atol=1e-8)


def _tf():
    m = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
    return getattr(m.torch_chunk_gated_delta_rule, "__wrapped__", m.torch_chunk_gated_delta_rule)


@pytest.mark.parametrize("T,s0", [(100, True), (64, False), (1, True)])
@pytest.mark.parametrize("in_dtype", [torch.float32, torch.bfloat16, F64])
def test_transformers_restatement_matches_installed_transformers(T, s0, in_dtype):
    """oracle.torch_chunk_gated_delta_rule (l2norm in the input dtype before the float32 cast, row-loop inverse: the
    installed 5.15.0 order) against the installed function, which always computes in float32."""
    tf = _tf()
    inp = gdr.make_inputs(2, T, 3, 3, 32, 32, in_dtype, s0=s0, seed=12)
    args = [inp[n] for n in ("query", "key", "value", "g", "beta")]
    kw = dict(initial_state=inp["initial_state"], output_final_state=True, use_qk_l2norm_in_kernel=True)
    ro, rs = tf(*args, **kw)
    mo, ms = gdr.torch_chunk_gated_delta_rule(*args, cast_first=False, **kw)
    assert mo.dtype == ro.dtype == in_dtype
    assert gdr.rel(mo, ro) < 1e-6 and gdr.rel(ms, rs) < 1e-6
    if in_dtype == torch.float32:
        # float32 inputs: the two cast orders are one computation (the cast is the identity), bit for bit; the 5.22.1
        # form the GPU tests' 2x anchor uses (cast first, solve_triangular inverse) sits within float32 error of the
        # installed row-loop function
        co, cs = gdr.torch_chunk_gated_delta_rule(*args, cast_first=True, **kw)
        assert torch.equal(co, mo) and torch.equal(cs, ms)
        so, ss = gdr.torch_chunk_gated_delta_rule(*args, cast_first=True, inverse="solve", **kw)
        assert gdr.rel(so, ro) < 1e-5 and gdr.rel(ss, rs) < 1e-5


def test_transformers_algorithm_is_the_recurrence():
    """The transformers algorithm (restated, run in float64) equals the token recurrence to rounding, and the installed
    float32 function sits within float32 error of it: the reference torch path computes the rule the recurrence
    defines."""
    tf = _tf()
    inp = gdr.make_inputs(1, 90, 2, 2, 16, 16, F64, s0=True, seed=13)
    inp = {n: (None if x is None else x.double()) for n, x in inp.items()}
    args = [inp[n] for n in ("query", "key", "value", "g", "beta")]
    kw = dict(initial_state=inp["initial_state"], output_final_state=True, use_qk_l2norm_in_kernel=True)
    q, k = gdr.prologue(inp["query"], inp["key"])
    o, sT = gdr.recurrence(q, k, inp["value"], inp["g"], inp["beta"], inp["initial_state"])
    for inverse in ("rowloop", "solve"):
        mo, ms = gdr.torch_chunk_gated_delta_rule(*args, compute_dtype=F64, inverse=inverse, **kw)
        assert gdr.rel(mo, o) < 1e-12 and gdr.rel(ms, sT) < 1e-12
    ro, rs = tf(*args, **kw)
    assert gdr.rel(ro, o) < 1e-5 and gdr.rel(rs, sT) < 1e-5


def test_dropin_oracle_against_golden_fixture():
    """oracle.dropin_f64 (chunked equations + autograd through the prologue) reproduces the committed fixture's
    float64 outputs and gradients (autograd through the recurrence); transformers' stored float32 output sits within
    its own fp32 error."""
    z = np.load(os.path.join(HERE, "golden", "dropin_small.npz"))
    t = {n: torch.from_numpy(z[n]) for n in z.files}
    o, sT, grads = gdr.dropin_f64(t["query"], t["key"], t["value"], t["g"], t["beta"], t["initial_state"],
                                  do=t["do"], dsT=t["dsT"])
    assert gdr.rel(o, t["o"]) < 1e-12 and gdr.rel(sT, t["sT"]) < 1e-12
    for n, x in grads.items():
        assert gdr.rel(x, t[n]) < 1e-11, n
    assert gdr.rel(t["tf_o"], t["o"]) < 1e-5 and gdr.rel(t["tf_sT"], t["sT"]) < 1e-5


def test_planted_mistakes_are_caught():
    """A dropped term, a transposed operand or a wrong sign in the oracle's backward fails the recurrence check (the
    tests above would catch such a slip): here planted into copies of the equations on the CPU."""
    q, k, v, g, b, s0 = gdr.harness_inputs(1, 21, 1, 6, 5, seed=1)
    gen = torch.Generator().manual_seed(5)
    do = torch.randn(1, 21, 1, 5, generator=gen, dtype=F64)
    dsT = torch.randn(1, 1, 6, 5, generator=gen, dtype=F64)
    _, _, grads = _grads_autograd(q, k, v, g, b, s0, do, dsT)
    _, _, P = gdr.chunked_forward(q, k, v, g, b, s0, 8)
    bad = dict(P, A=P["A"].transpose(-1, -2))            # transposed operand
    mine, _ = gdr.chunked_backward(q, k, v, g, b, s0, do, dsT, 8, bad)
    assert max(gdr.rel(a, r) for a, r in zip(mine, grads)) > 1e-3
    bad = dict(P, e=torch.ones_like(P["e"]))             # dropped decay term
    mine, _ = gdr.chunked_backward(q, k, v, g, b, s0, do, dsT, 8, bad)
    assert max(gdr.rel(a, r) for a, r in zip(mine, grads)) > 1e-3
    bad = dict(P, W=-P["W"])                             # wrong sign (of W's term in B2 and of dW)
    mine, _ = gdr.chunked_backward(q, k, v, g, b, s0, do, dsT, 8, bad)
    assert max(gdr.rel(a, r) for a, r in zip(mine, grads)) > 1e-3


def test_segmented_forward_is_the_same_computation():
    """Cutting the sequence at chunk boundaries and carrying the state changes nothing (bitwise)."""
    xs = gdr.harness_inputs(1, 300, 2, 16, 8, seed=14)
    o, sT, _ = gdr.chunked_forward(*xs, 64)
    o2, sT2 = gdr.chunked_forward_segments(*xs, 64, seg=128)
    assert gdr.rel(o2, o) < 1e-14 and gdr.rel(sT2, sT) < 1e-14


def test_segment_map_composes_the_state_pass():
    """segment_map: A S_0 + B is the final state of chunked_forward from any S_0 (< 1e-12), composing two halves' maps
    in order gives the whole row's, and the composition in the wrong order does not (a planted mistake)."""
    gen = torch.Generator().manual_seed(21)
    B, T, H, DK, DV = 1, 200, 2, 32, 16
    q = gdr.l2norm(torch.randn(B, T, H, DK, generator=gen, dtype=F64)) * DK ** -0.5
    k = gdr.l2norm(torch.randn(B, T, H, DK, generator=gen, dtype=F64))
    v = torch.randn(B, T, H, DV, generator=gen, dtype=F64)
    g = -torch.rand(B, T, H, generator=gen, dtype=F64) * 0.1
    b = torch.rand(B, T, H, generator=gen, dtype=F64)
    s0 = torch.randn(B, H, DK, DV, generator=gen, dtype=F64)
    A, Bm = gdr.segment_map(q, k, v, g, b)
    _, sT, _ = gdr.chunked_forward(q, k, v, g, b, s0)
    assert (A @ s0 + Bm - sT).abs().max() < 1e-12
    h = 128                                  # two segments of whole chunks
    A1, B1 = gdr.segment_map(q[:, :h], k[:, :h], v[:, :h], g[:, :h], b[:, :h])
    A2, B2 = gdr.segment_map(q[:, h:], k[:, h:], v[:, h:], g[:, h:], b[:, h:])
    assert (A2 @ (A1 @ s0 + B1) + B2 - sT).abs().max() < 1e-12
    assert (A1 @ (A2 @ s0 + B2) + B1 - sT).abs().max() > 1e-3


@pytest.mark.parametrize("name", list(_chain.CASES))
def test_chain_cases_catch_planted_mistakes(name):
    """The many-chunk chain cases of tests/test_gpu_chain.py have teeth: on exactly their inputs, a carried decay of
    gamma_last^2 instead of gamma_last, and G_last taken from the row before the chunk's last, each planted in the
    forward chain and (for the cases with a backward) in the reverse chain, move some output or gradient by more than
    twice the largest bar those tests apply (1e-2 for bf16; the float32 bars are 2x a float32 error, far smaller).  So
    a kernel with such a mistake fails them even with its own rounding (a few 1e-3) on top."""
    plants = gdr.PLANTS if _chain.CASES[name]["kind"] != "prefill" else ("fwd_gamma_sq", "fwd_glast_off")
    for seed in _chain.seeds(name):
        inp = _chain.inputs(name, seed)
        ref = _chain.oracle(name, inp)
        for plant in plants:
            errs = _chain.errors(_chain.oracle(name, inp, plant), ref)
            worst = max(errs, key=errs.get)
            print(name, seed, plant, worst, f"{errs[worst]:.2e}", flush=True)
            assert errs[worst] > 2 * _chain.BF16_BAR, (name, seed, plant, errs)


def test_bf16_rounding_model_is_off_by_default():
    """The precision model (rnd) rounds nothing unless asked, and rounding to bf16 is torch's round-to-nearest-even:
    with rnd=() the forward and backward are the pinned equations bit for bit."""
    xs = gdr.harness_inputs(1, 90, 2, 16, 8, seed=3)
    gen = torch.Generator().manual_seed(4)
    do = torch.randn(1, 90, 2, 8, generator=gen, dtype=F64)
    dsT = torch.randn(1, 2, 16, 8, generator=gen, dtype=F64)
    a, _ = gdr.chunked_backward(*xs, do, dsT, 64)
    b, _ = gdr.chunked_backward(*xs, do, dsT, 64, rnd=())
    assert all(torch.equal(x, y) for x, y in zip(a, b))
    x = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -3.14159], dtype=F64)
    assert torch.equal(gdr.bf16(x), torch.tensor([1.0, 1.0 + 2 ** -6, -3.140625], dtype=F64))
    c, _ = gdr.chunked_backward(*xs, do, dsT, 64, rnd=gdr.ROUNDABLE)
    assert 1e-5 < max(gdr.rel(u, v) for u, v in zip(c, a)) < 3e-2


def test_chunk_states_stay_float32():
    """Why the chunk states S_c are stored in fp32 although the per-chunk backward feeds them to its products in bf16:
    its last-row dg term <S_c, dS_{c+1}> is a dot over DK x DV products that can cancel.  On the inputs of
    test_gpu_dropin.py::test_dropin_bf16_small's (1, 1, 2, 64) case the bf16 path's rounding model moves dg by 1.9e-3,
    and S_c rounded in that dot as well ("ScDot", what bf16 storage would do) by 2.0e-2, twice the bf16 bar: a build
    that stored S_c in bf16 failed that case on the GPU with exactly dg 2.00e-2.  Over 50 tokens the other terms of dg
    dominate and the dot's rounding does not show."""
    names = ("query", "key", "value", "g", "beta", "initial_state")
    model = gdr.BF16_PATH
    for shape, lo, hi in (((1, 1, 2, 64), 1.5e-2, 2.5e-2), ((2, 50, 3, 128), 0.0, 1e-2)):
        B, T, H, D = shape
        inp = gdr.make_inputs(B, T, H, H, D, D, torch.bfloat16, s0=True, seed=8)
        dsT = torch.randn(B, H, D, D, generator=torch.Generator().manual_seed(9))
        args = [inp[n] for n in names]
        exact = gdr.dropin_f64(*args, do=inp["do"], dsT=dsT)[2]["dg"]
        path = gdr.dropin_f64(*args, do=inp["do"], dsT=dsT, rnd=model)[2]["dg"]
        dot = gdr.dropin_f64(*args, do=inp["do"], dsT=dsT, rnd=model + ("ScDot",))[2]["dg"]
        assert gdr.rel(path, exact) < 2.5e-3, shape
        assert lo <= gdr.rel(dot, exact) < hi, shape


def test_chunk_state_enters_dq_and_dg_as_a_pair():
    """Why the per-chunk backward takes S_c into dO S_c^T as a hi + lo pair of bf16 fragments: gamma q . (S_c dO^T) in
    dg cancels when the state is large against the output's gradient.  On a draw with an N(0, 1) starting state
    (B=1, T=150, H=2, DK=32, DV=128, seed 8073; tests/test_gpu_dropin.py::test_large_starting_state runs it on the GPU)
    the bf16 path's rounding model gives dg 3.1e-3 from float64, and 1.5e-2 with S_c rounded once there ("Sc")."""
    names = ("query", "key", "value", "g", "beta", "initial_state")
    inp = gdr.make_inputs(1, 150, 2, 2, 32, 128, torch.bfloat16, s0=True, seed=8073)
    inp["initial_state"] = inp["initial_state"] * 50.0
    args = [inp[n] for n in names]
    exact = gdr.dropin_f64(*args, do=inp["do"])[2]["dg"]
    path = gdr.dropin_f64(*args, do=inp["do"], rnd=gdr.BF16_PATH)[2]["dg"]
    once = gdr.dropin_f64(*args, do=inp["do"], rnd=gdr.BF16_PATH + ("Sc",))[2]["dg"]
    assert gdr.rel(path, exact) < 5e-3 and gdr.rel(once, exact) > 1e-2

"""GPU tests of packed rows (transformers' cu_seqlens): several sequences in one row, each run on its own from its own
initial state.  The reference refuses cu_seqlens (op.py:270-273); the varlen form is what transformers passes for
packed batches (modeling_qwen3_5.py:519-530).

A sequence inside a packed row is chunked from its own start, so every chunk sees the same tokens and the same
arithmetic as when the sequence runs alone (and the value split changes no bits): outputs, final states and every
gradient must equal the per-sequence runs bit for bit.  The per-sequence runs are the drop-in's ordinary path, held to
the float64 oracle by test_gpu_dropin.py; one fp32 case is also checked against the oracle here.
"""
import pytest
import torch

import _parity

from macai.gated_delta import chunk_gated_delta_rule, op
from oracle import gdr

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _same_kernels_alone(monkeypatch):
    """A packed row runs on the bf16 kernels whatever its sequences' lengths; a bf16 sequence shorter than a chunk run
    alone would take the float32 kernels (op.BF16_MIN_TOKENS).  The comparisons here run it on the bf16 kernels too,
    and keep the backward with the final states' gradient on them (op.BF16_STATE_GRAD): these tests pin the bf16
    kernels' packed-row forms."""
    monkeypatch.setattr(op, "BF16_MIN_TOKENS", 0)
    monkeypatch.setattr(op, "BF16_STATE_GRAD", True)


def _say(*a):
    print(*a, flush=True)


def _inputs(lens, Hk, Hv, DK, DV, dtype, seed):
    """One packed row of the sequences (each drawn with gdr.make_inputs), their initial states, dO and dsT."""
    parts = [gdr.make_inputs(1, max(n, 1), Hk, Hv, DK, DV, dtype, s0=True, seed=seed + i) for i, n in enumerate(lens)]
    cat = lambda name: torch.cat([p[name][:, :n] for p, n in zip(parts, lens)], 1)
    row = {n: cat(n) for n in ("query", "key", "value", "g", "beta", "do")}
    row["query"], row["key"] = row["query"][:, :, ::Hv // Hk].contiguous(), row["key"][:, :, ::Hv // Hk].contiguous()
    s0 = torch.cat([p["initial_state"] for p in parts], 0)
    dsT = torch.randn(len(lens), Hv, DK, DV, generator=torch.Generator().manual_seed(seed + 99))
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32)
    return row, s0, dsT, cu


def _run(row, s0, dsT, cu=None):
    names = ("query", "key", "value", "g", "beta")
    leaves = [row[n].to(DEV).requires_grad_(True) for n in names]
    s0 = s0.to(DEV).requires_grad_(True)
    kw = {} if cu is None else {"cu_seqlens": cu.to(DEV)}
    o, sT = chunk_gated_delta_rule(*leaves, initial_state=s0, output_final_state=True, use_qk_l2norm_in_kernel=True,
                                   **kw)
    torch.autograd.backward([o, sT], [row["do"].to(DEV), dsT.to(DEV)])
    torch.cuda.synchronize()
    return o.detach().cpu(), sT.detach().cpu(), [x.grad.cpu() for x in leaves + [s0]]


@pytest.mark.parametrize("lens,Hk,Hv,DK,DV,dtype", [
    ([130, 0, 64, 6, 200], 2, 2, 128, 128, torch.bfloat16),
    ([1, 63, 65, 128], 1, 3, 64, 64, torch.bfloat16),
    ([77, 150], 2, 4, 128, 64, torch.bfloat16),
    ([40, 0, 90], 2, 2, 64, 128, torch.float32),
    # 51 chunks x 16 heads: more chunk-heads than CUs, so the persistent chunk backward runs over packed chunks
    ([1000, 0, 700, 65, 1300, 3], 16, 16, 128, 128, torch.bfloat16),
])
def test_packed_rows_equal_separate_sequences(lens, Hk, Hv, DK, DV, dtype):
    _say("case", lens, Hk, Hv, DK, DV, dtype)
    row, s0, dsT, cu = _inputs(lens, Hk, Hv, DK, DV, dtype, seed=40)
    o, sT, g = _run(row, s0, dsT, cu)
    assert o.shape == row["value"].shape and sT.shape == s0.shape
    t = 0
    for n, L in enumerate(lens):
        if L == 0:                           # an empty sequence: its state passes through, its gradient too
            assert torch.equal(sT[n], s0[n]) and torch.equal(g[5][n], dsT[n])
            continue
        seq = {k: v[:, t:t + L].contiguous() for k, v in row.items()}
        o1, sT1, g1 = _run(seq, s0[n:n + 1], dsT[n:n + 1])
        assert torch.equal(o[:, t:t + L], o1) and torch.equal(sT[n:n + 1], sT1), f"sequence {n}"
        for i in range(5):
            assert torch.equal(g[i][:, t:t + L], g1[i]), f"sequence {n}, gradient {i}"
        assert torch.equal(g[5][n:n + 1], g1[5]), f"sequence {n}, initial-state gradient"
        t += L


def test_packed_rows_mixed_io_changes_no_bits(monkeypatch):
    """bf16 packed rows on the float32 kernels (op.BF16_OPERANDS off): the bf16 tensors handed to them as they are
    (op.MIXED_IO: read exactly, o and dq, dk, dv rounded once) or upcast and the results cast back -- the same bits."""
    _say("case packed mixed io")
    monkeypatch.setattr(op, "BF16_OPERANDS", False)
    row, s0, dsT, cu = _inputs([70, 0, 130, 5], 2, 2, 128, 128, torch.bfloat16, seed=46)
    runs = []
    for mixed in (True, False):
        monkeypatch.setattr(op, "MIXED_IO", mixed)
        runs.append(_run(row, s0, dsT, cu))
    (o, sT, g), (o2, sT2, g2) = runs
    assert o.dtype == torch.bfloat16 and torch.equal(o, o2) and torch.equal(sT, sT2)
    assert all(a.dtype == b.dtype and torch.equal(a, b) for a, b in zip(g, g2))


def test_packed_rows_against_the_oracle():
    """fp32, three sequences: outputs, final states and gradients within the fp32 harness bar of the float64 oracle
    run on each sequence."""
    lens = [100, 37, 64]
    row, s0, dsT, cu = _inputs(lens, 2, 2, 64, 64, torch.float32, seed=50)
    o, sT, g = _run(row, s0, dsT, cu)
    t, errs = 0, {}
    for n, L in enumerate(lens):
        ro, rsT, rg = gdr.dropin_f64(*(row[k][:, t:t + L] for k in ("query", "key", "value", "g", "beta")),
                                     initial_state=s0[n:n + 1], do=row["do"][:, t:t + L], dsT=dsT[n:n + 1])
        errs[f"o{n}"], errs[f"sT{n}"] = gdr.rel(o[:, t:t + L], ro), gdr.rel(sT[n:n + 1], rsT)
        for i, name in enumerate(("dquery", "dkey", "dvalue", "dg", "dbeta")):
            errs[f"{name}{n}"] = gdr.rel(g[i][:, t:t + L], rg[name])
        errs[f"dstate{n}"] = gdr.rel(g[5][n:n + 1], rg["dstate"])
        t += L
    _parity.check(errs, 2e-4)


@pytest.mark.parametrize("lens,Hk,Hv,dtype", [([130, 0, 64, 6, 200], 2, 2, torch.bfloat16),
                                              ([300, 1, 700], 1, 2, torch.bfloat16),
                                              ([40, 0, 90], 2, 2, torch.float32)])
def test_packed_rows_forward_only(lens, Hk, Hv, dtype):
    """Inference (no_grad: the state pass with the output only, which prefetches its next tiles into L2) on packed
    rows: the same bits as each sequence run alone and as the training forward's output (the state pass that also
    stores the chunk states forms the same products in the same order)."""
    _say("case forward only", lens, Hk, Hv, dtype)
    row, s0, dsT, cu = _inputs(lens, Hk, Hv, 128, 128, dtype, seed=60)
    names = ("query", "key", "value", "g", "beta")

    def fwd(r, s, c=None):
        kw = {} if c is None else {"cu_seqlens": c.to(DEV)}
        with torch.no_grad():
            o, sT = chunk_gated_delta_rule(*(r[n].to(DEV) for n in names), initial_state=s.to(DEV),
                                           output_final_state=True, use_qk_l2norm_in_kernel=True, **kw)
        torch.cuda.synchronize()
        return o.cpu(), sT.cpu()
    o, sT = fwd(row, s0, cu)
    to, tsT, _ = _run(row, s0, dsT, cu)
    assert torch.equal(o, to) and torch.equal(sT, tsT), "no_grad and training forwards differ"
    t = 0
    for n, L in enumerate(lens):
        if L == 0:
            assert torch.equal(sT[n], s0[n])
            continue
        o1, sT1 = fwd({k: v[:, t:t + L].contiguous() for k, v in row.items()}, s0[n:n + 1])
        assert torch.equal(o[:, t:t + L], o1) and torch.equal(sT[n:n + 1], sT1), f"sequence {n}"
        t += L

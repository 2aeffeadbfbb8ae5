"""The many-chunk state-chain cases: inputs and their float64 oracle, shared by the GPU parity tests
(tests/test_gpu_chain.py) and the CPU check that those very inputs catch a planted chain mistake
(tests/test_oracle.py::test_chain_cases_catch_planted_mistakes).

Why a weaker decay: under the BASELINE generator's decay (g = -exp(u) softplus(x), a chunk's log decay about -260) the
state carried into a chunk is multiplied by e^-30 or less per chunk, so a wrong exp(G_last) on the carried state S_c
(forward, reference _chunked.py:643-653) or on the carried gradient dS_{c+1} (reverse pass, _chunked.py:886-898)
moves no output.  Here g is the generator's draw times DECAY (mean log decay about -1.6 a chunk over the generator's
mix of per-head rates), every case runs at least 16 chunks a sequence with a starting state and an upstream gradient
of the final state, so each chunk's output and each gradient depends on the chain through many chunks.
"""
import torch

from oracle import gdr

DECAY = 0.005
BF16_BAR = 1e-2
NAMES = ("query", "key", "value", "g", "beta")
GRADS = ("dquery", "dkey", "dvalue", "dg", "dbeta", "dstate")
bf16, f32 = torch.bfloat16, torch.float32

# name -> case.  kind "dense": B rows of T tokens (q, k at Hk key heads, Hv value heads), forward + backward;
# seeds: several draws of the case (the float32 case: one draw's float32 error, the anchor of its bar, varies a few
# times between seeds, so the bar compares the largest over the draws);
# "packed": one row of sequences of the given lengths (cu_seqlens), one starting state each, forward + backward;
# "prefill": BASELINE config 3's single row, forward only (no starting state, the final state returned).
CASES = {
    # config 1's shape: the recompute backward's pair pass runs at split 2 with four column waves a workgroup
    "config1_bf16": dict(kind="dense", B=4, T=1024, Hk=16, Hv=16, D=128, dtype=bf16, seed=1201),
    "fp32": dict(kind="dense", B=2, T=1024, Hk=4, Hv=4, D=128, dtype=f32, seed=1202, seeds=(1202, 1212, 1222, 1232)),
    "grouped_bf16": dict(kind="dense", B=2, T=1024, Hk=4, Hv=8, D=128, dtype=bf16, seed=1203),
    "packed_bf16": dict(kind="packed", lens=(1030, 1070, 1400), Hk=4, Hv=4, D=128, dtype=bf16, seed=1210),
    "config3_bf16": dict(kind="prefill", T=32768, Hk=16, Hv=16, D=128, dtype=bf16, seed=1205),
}


def seeds(name):
    """The draws of a case."""
    return CASES[name].get("seeds", (CASES[name]["seed"],))


def inputs(name, seed=None):
    """The case's CPU inputs (draw `seed`, the case's first by default): query, key (at the key heads), value, g, beta,
    initial_state, do, dsT, cu (or None)."""
    c = CASES[name]
    seed = c["seed"] if seed is None else seed
    D, Hk, Hv, dt = c["D"], c["Hk"], c["Hv"], c["dtype"]
    gen = torch.Generator().manual_seed(seed + 7)
    if c["kind"] == "prefill":
        inp = gdr.make_inputs(1, c["T"], Hk, Hv, D, D, dt, s0=False, seed=seed)
        inp.update(dsT=None, cu=None)
    elif c["kind"] == "packed":
        lens = c["lens"]
        inp = gdr.make_inputs(1, sum(lens), Hk, Hv, D, D, dt, s0=False, seed=seed)
        inp["initial_state"] = (torch.randn(len(lens), Hv, D, D, generator=gen, dtype=torch.float64) * 0.02).float()
        inp["dsT"] = torch.randn(len(lens), Hv, D, D, generator=gen)
        inp["cu"] = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    else:
        inp = gdr.make_inputs(c["B"], c["T"], Hk, Hv, D, D, dt, s0=True, seed=seed)
        inp["dsT"] = torch.randn(c["B"], Hv, D, D, generator=gen)
        inp["cu"] = None
    inp["g"] = inp["g"] * DECAY
    rep = Hv // Hk
    inp["query"], inp["key"] = inp["query"][:, :, ::rep].contiguous(), inp["key"][:, :, ::rep].contiguous()
    return inp


def _repeat(x, rep):
    return x if rep == 1 else x.repeat_interleave(rep, 2)


def _fold(x, rep):
    """The gradient of repeat_interleave over the heads: each key head's value heads summed."""
    return x if rep == 1 else x.reshape(*x.shape[:2], -1, rep, x.shape[-1]).sum(3)


def oracle(name, inp, plant=None):
    """{o, sT, and for the backward cases the six gradients} in float64 from the case's inputs (the drop-in's
    semantics: fused l2norm prologue, q scaled by D^-1/2); plant: one of gdr.PLANTS, a deliberate chain mistake."""
    c = CASES[name]
    rep = c["Hv"] // c["Hk"]
    if c["kind"] == "prefill":
        q, k = gdr.prologue(_repeat(inp["query"], rep).double(), _repeat(inp["key"], rep).double())
        s0 = torch.zeros(1, c["Hv"], c["D"], c["D"], dtype=torch.float64)
        o, sT = gdr.chunked_forward_segments(q, k, inp["value"].double(), inp["g"].double(), inp["beta"].double(), s0,
                                             plant=plant)
        return {"o": o, "sT": sT}
    cu = [0, inp["query"].shape[1]] if inp["cu"] is None else inp["cu"].tolist()
    parts = []
    for n, (t0, t1) in enumerate(zip(cu, cu[1:])):
        sl = (slice(None), slice(t0, t1))
        rows = slice(None) if inp["cu"] is None else slice(n, n + 1)
        o, sT, gr = gdr.dropin_f64(*(_repeat(inp[x][sl], rep) if x in ("query", "key") else inp[x][sl]
                                     for x in NAMES),
                                   initial_state=inp["initial_state"][rows], do=inp["do"][sl], dsT=inp["dsT"][rows],
                                   plant=plant)
        gr["dquery"], gr["dkey"] = _fold(gr["dquery"], rep), _fold(gr["dkey"], rep)
        parts.append(dict(o=o, sT=sT, **gr))
    if len(parts) == 1:
        return parts[0]
    out = {}
    for x in parts[0]:
        out[x] = torch.cat([p[x] for p in parts], 0 if x in ("sT", "dstate") else 1)
    return out


def errors(got, ref):
    """The reference harness's metric, max|a - r| / max|r|, per tensor of ref."""
    return {n: gdr.rel(got[n], ref[n]) for n in ref}

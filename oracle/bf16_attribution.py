"""Where the bf16 path's error comes from: the float64 oracle with one operand class at a time rounded to bf16 where
a bf16 MFMA product would take it (oracle.gdr.ROUNDABLE), then the classes the kernels round (oracle.gdr.BF16_PATH)
and combinations of them kept at full precision (the cost of hi + lo bf16 pairs for them), against float64 of the
same inputs.  Test infrastructure / design analysis only (CPU): `python oracle/bf16_attribution.py` prints the table
in markdown.

Cases: the smoke's draw (B=1, T=100, H=2, D=128, bf16, a starting state) with an N(0, 1) gradient of the final state
(on the bf16 kernels only with op.BF16_STATE_GRAD), and the same draw at 1024 tokens with g x 0.005 (the many-chunk
chain cases' decay).  Every run also rounds the bf16 outputs (o, dq, dk, dv) once, as the kernels do.  "QK" (the
normalised q, k as operands) is not in the path, since the kernels take the raw bf16 q, k (exact) and apply the norms
in fp32, nor is "Sc" (the per-chunk backward takes the chunk state as a hi + lo pair); its row shows what rounding it
once would add.
"""
import os
import sys

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
from oracle import gdr  # noqa: E402

NAMES = ("query", "key", "value", "g", "beta", "initial_state")
OUTS = ("o", "sT", "dquery", "dkey", "dvalue", "dg", "dbeta", "dstate")
MODEL = gdr.BF16_PATH
CLASSES = tuple(c for c in gdr.ROUNDABLE if c != "QK")   # one row each (Sc: what rounding S_c once would add)


def case(T, scale):
    inp = gdr.make_inputs(1, T, 2, 2, 128, 128, torch.bfloat16, s0=True, seed=7)
    inp["g"] = inp["g"] * scale
    return inp, torch.randn(1, 2, 128, 128, generator=torch.Generator().manual_seed(11))


def errors(inp, dsT, rnd, exact):
    o, sT, gr = gdr.dropin_f64(*(inp[n] for n in NAMES), do=inp["do"], dsT=dsT, rnd=rnd)
    got = dict(o=o, sT=sT, **gr)
    for n in ("o", "dquery", "dkey", "dvalue"):
        got[n] = gdr.bf16(got[n].float()).double()
    return {n: gdr.rel(got[n], exact[n]) for n in OUTS}


def main():
    combos = {"all classes (the bf16 path)": MODEL,
              "hi+lo S, dS": tuple(c for c in MODEL if c not in ("S", "dS")),
              "hi+lo Vn, dVn, dS": tuple(c for c in MODEL if c not in ("Vn", "dVn", "dS")),
              "hi+lo Vn, dVn, dS, Ke": tuple(c for c in MODEL if c not in ("Vn", "dVn", "dS", "Ke")),
              "no operand rounding": ()}
    for tag, (T, scale) in {"smoke (T=100)": (100, 1.0), "chain (T=1024, g x 0.005)": (1024, 0.005)}.items():
        inp, dsT = case(T, scale)
        o, sT, gr = gdr.dropin_f64(*(inp[n] for n in NAMES), do=inp["do"], dsT=dsT)
        exact = dict(o=o, sT=sT, **gr)
        print(f"## {tag}")
        print("| rounded to bf16 | " + " | ".join(OUTS) + " |")
        print("|---" * (len(OUTS) + 1) + "|")
        rows = [(f"only {c}", (c,)) for c in CLASSES] + list(combos.items())
        for name, rnd in rows:
            e = errors(inp, dsT, rnd, exact)
            print(f"| {name} | " + " | ".join(f"{e[n]:.1e}" for n in OUTS) + " |", flush=True)


if __name__ == "__main__":
    main()

"""Writes tests/golden/dropin_small.npz: a small drop-in case (bf16-representable inputs stored as float32) with its
float64 outputs and gradients computed by torch.autograd through the token recurrence and the l2norm prologue -- an
independent truth, not the chunked oracle -- plus installed transformers' torch_chunk_gated_delta_rule output in float32
(the reference torch path; transformers 5.15.0 in this image).  The reference ships no vectors of its own (its tests
regenerate inputs from seeds), so this fixture is derived from the mathematics.  Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import gdr  # noqa: E402

B, T, H, D = 1, 77, 2, 64


def main():
    inp = gdr.make_inputs(B, T, H, H, D, D, torch.bfloat16, s0=True, seed=2024, dsT=True)
    names = ("query", "key", "value", "g", "beta", "initial_state")
    x64 = [inp[n].double().requires_grad_(True) for n in names]
    q, k = gdr.prologue(x64[0], x64[1], True)
    o, sT = gdr.recurrence(q, k, *x64[2:])
    do, dsT = inp["do"].double(), inp["dsT"].double()
    torch.autograd.backward([o, sT], [do, dsT])
    import transformers.models.qwen3_5.modeling_qwen3_5 as m
    tf = getattr(m.torch_chunk_gated_delta_rule, "__wrapped__", m.torch_chunk_gated_delta_rule)
    with torch.no_grad():
        to, tsT = tf(*(inp[n].float() for n in names[:5]), initial_state=inp["initial_state"],
                     output_final_state=True, use_qk_l2norm_in_kernel=True)
    out = {n: inp[n].float().numpy() for n in names}
    out.update(do=do.float().numpy(), dsT=dsT.float().numpy(), o=o.detach().numpy(), sT=sT.detach().numpy(),
               tf_o=to.numpy(), tf_sT=tsT.numpy())
    for n, x in zip(("dquery", "dkey", "dvalue", "dg", "dbeta", "dstate"), x64):
        out[n] = x.grad.numpy()
    np.savez_compressed(os.path.join(HERE, "dropin_small.npz"), **out)
    print({n: v.shape for n, v in out.items()})


if __name__ == "__main__":
    main()

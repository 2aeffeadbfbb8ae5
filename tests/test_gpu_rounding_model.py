"""The bf16 kernels against the oracle's rounding model of the bf16 path (oracle.gdr.BF16_PATH: the float64 rule with
the operand classes the kernels round to bf16 rounded where they enter a product, and the bf16 outputs rounded once).
The routing rules (op.BF16_MIN_TOKENS, BF16_UNNORMALIZED, BF16_STATE_GRAD) and the precision figures quoted for them
rest on random sweeps of that model on the CPU; these cases check that the kernels' errors against float64 are the
model's, draw by draw, including draws where both miss the 1e-2 bar (a final-state gradient kept on the bf16 kernels).
dq is left out: the kernels fold the norm scales into dM before rounding it, which the model does not."""
import pytest
import torch

from macai.gated_delta import chunk_gated_delta_rule, op
from oracle import gdr

pytestmark = pytest.mark.gpu
NAMES = ("query", "key", "value", "g", "beta", "initial_state")
OUTS = ("o", "sT", "dkey", "dvalue", "dg", "dbeta", "dstate")


@pytest.mark.parametrize("T,DK,DV,seed,s0scale,dseed", [
    (100, 128, 128, 7, 1.0, None),      # the smoke's draw
    (100, 128, 128, 7, 1.0, 11),        # with a final-state gradient (the attribution case)
    (150, 128, 128, 209, 1.0, 216),     # a final-state gradient on which dg misses the bar
    (150, 32, 128, 8073, 50.0, None),   # an N(0, 1) starting state
    (64, 128, 64, 8070, 1.0, None),     # one chunk, the default state scale
])
def test_kernels_follow_the_rounding_model(T, DK, DV, seed, s0scale, dseed, monkeypatch):
    print(f"case rounding model T={T} DK={DK} DV={DV} seed={seed} s0x{s0scale} dsT={dseed}", flush=True)
    monkeypatch.setattr(op, "BF16_STATE_GRAD", True)      # the bf16 kernels throughout, as the model
    monkeypatch.setattr(op, "BF16_MIN_TOKENS", 0)
    inp = gdr.make_inputs(1, T, 2, 2, DK, DV, torch.bfloat16, s0=True, seed=seed)
    inp["initial_state"] = inp["initial_state"] * s0scale
    dsT = None if dseed is None else torch.randn(1, 2, DK, DV, generator=torch.Generator().manual_seed(dseed))
    args = [inp[n] for n in NAMES]
    eo, esT, eg = gdr.dropin_f64(*args, do=inp["do"], dsT=dsT)
    mo, msT, mg = gdr.dropin_f64(*args, do=inp["do"], dsT=dsT, rnd=gdr.BF16_PATH)
    exact = dict(o=eo, sT=esT, **eg)
    model = dict(o=gdr.bf16(mo.float()).double(), sT=msT, **mg)
    for n in ("dkey", "dvalue"):
        model[n] = gdr.bf16(model[n].float()).double()
    leaves = [x.cuda().requires_grad_(True) for x in args]
    o, sT = chunk_gated_delta_rule(*leaves[:5], initial_state=leaves[5], output_final_state=True,
                                   use_qk_l2norm_in_kernel=True)
    outs, ups = [o], [inp["do"].cuda()]
    if dsT is not None:
        outs.append(sT)
        ups.append(dsT.cuda())
    grads = torch.autograd.grad(outs, leaves, ups)
    torch.cuda.synchronize()
    kern = dict(o=o.detach().cpu(), sT=sT.detach().cpu(), **{("dg" if n == "g" else "dstate" if n == "initial_state"
                                                               else "d" + n): x.cpu() for n, x in zip(NAMES, grads)})
    ek = {n: gdr.rel(kern[n], exact[n]) for n in OUTS}
    em = {n: gdr.rel(model[n], exact[n]) for n in OUTS}
    print("kernel", {n: f"{v:.2e}" for n, v in ek.items()}, flush=True)
    print("model ", {n: f"{v:.2e}" for n, v in em.items()}, flush=True)
    # the kernel's error is the model's to within 15% (or 2e-4 where both are small)
    off = {n: (ek[n], em[n]) for n in OUTS if abs(ek[n] - em[n]) > max(0.15 * em[n], 2e-4)}
    assert not off, off

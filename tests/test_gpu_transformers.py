"""The drop-in inside transformers' own linear-attention module: Qwen3_5GatedDeltaNet (a small config with seeded random
weights) forward and backward on the GPU with the rule's name swapped by macai.patch.installed(), against the same
module in float64 on the CPU (reference tests/test_gated_delta.py:37-56, tests/test_layer.py:578-635).

The float64 run keeps transformers' code for everything but the rule, whose own float32 casts would otherwise cap it
at float32: there the module's name points at the oracle's float64 restatement of transformers' function.  Bars
(error = max|a - r| / max|r| per tensor: the output, the input's gradient and every parameter's gradient):
  * float32: <= 2 x the error of the unpatched module (transformers' own rule, float32) on the same GPU -- the
    pattern of the reference's layer test;
  * bfloat16 weights and activations: <= max(2 x the unpatched module's error in bfloat16 on the CPU, 1e-2).
"""
import copy

import pytest
import torch

import _parity
from oracle import gdr

pytestmark = pytest.mark.gpu
M = pytest.importorskip("transformers.models.qwen3_5.modeling_qwen3_5")
DEV = "cuda"


def _module(Hk, Hv):
    from transformers.models.qwen3_5.configuration_qwen3_5 import Qwen3_5TextConfig
    cfg = Qwen3_5TextConfig(hidden_size=256, linear_num_key_heads=Hk, linear_num_value_heads=Hv,
                            linear_key_head_dim=128, linear_value_head_dim=128, linear_conv_kernel_dim=4,
                            hidden_act="silu", rms_norm_eps=1e-6, num_hidden_layers=1,
                            layer_types=["linear_attention"], num_attention_heads=2, num_key_value_heads=1,
                            intermediate_size=512)
    torch.manual_seed(21)
    m = M.Qwen3_5GatedDeltaNet(cfg, 0)
    with torch.no_grad():
        for n, p in m.named_parameters():
            if n == "norm.weight":
                p.normal_(1.0, 0.1)
            elif n.endswith("weight"):
                p.normal_(0.0, 0.05 if "proj" in n else 0.3)
    return m


def _run(m, x, gy, device, dtype):
    """Forward + backward of a copy of m in dtype on device: (y, dx, {parameter: gradient}) on the CPU in float64."""
    m = copy.deepcopy(m).to(device, dtype)
    xx = x.to(device, dtype).clone().requires_grad_(True)
    y = m(xx)
    y.backward(gy.to(device, y.dtype))
    if device != "cpu":
        torch.cuda.synchronize()
    grads = {n: p.grad.detach().cpu().double() for n, p in m.named_parameters()}
    return y.detach().cpu().double(), xx.grad.detach().cpu().double(), grads


def _f64_rule(query, key, value, g, beta, chunk_size=64, initial_state=None, output_final_state=False,
              use_qk_l2norm_in_kernel=False, **kwargs):
    return gdr.torch_chunk_gated_delta_rule(query, key, value, g, beta, chunk_size, initial_state, output_final_state,
                                            use_qk_l2norm_in_kernel, compute_dtype=torch.float64, inverse="solve")


def _errors(got, ref):
    (y, dx, gr), (ry, rdx, rgr) = got, ref
    e = {"y": gdr.rel(y, ry), "dx": gdr.rel(dx, rdx)}
    e.update({"d " + n: gdr.rel(gr[n], rgr[n]) for n in rgr})
    return e


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("Hk,Hv", [(2, 2), (2, 4)])
def test_module_under_the_patch(Hk, Hv, dtype):
    import macai.patch as patch
    from macai.gated_delta import chunk_gated_delta_rule
    print(f"case transformers module Hk={Hk} Hv={Hv} {dtype}", flush=True)
    m = _module(Hk, Hv)
    gen = torch.Generator().manual_seed(22)
    B, T = 2, 150
    x = torch.randn(B, T, 256, generator=gen).to(dtype)
    gy = (torch.randn(B, T, 256, generator=gen) * 0.1).to(dtype)
    if dtype == torch.bfloat16:         # the bf16 model's values, held exactly by every run below
        m = m.to(torch.bfloat16).float()
    saved = M.torch_chunk_gated_delta_rule
    M.torch_chunk_gated_delta_rule = _f64_rule
    try:
        ref = _run(m, x.double(), gy.double(), "cpu", torch.float64)
    finally:
        M.torch_chunk_gated_delta_rule = saved
    if dtype == torch.float32:
        anchor = _errors(_run(m, x, gy, DEV, dtype), ref)
    else:
        anchor = _errors(_run(m, x, gy, "cpu", dtype), ref)
    with patch.installed(layer=False, training=False, lora=False):
        assert M.torch_chunk_gated_delta_rule is chunk_gated_delta_rule
        errs = _errors(_run(m, x, gy, DEV, dtype), ref)
    assert M.torch_chunk_gated_delta_rule is saved
    print("unpatched module's errors:", {k: f"{v:.2e}" for k, v in anchor.items()}, flush=True)
    bars = {n: 2 * anchor[n] if dtype == torch.float32 else max(2 * anchor[n], 1e-2) for n in errs}
    _parity.check(errs, bars)

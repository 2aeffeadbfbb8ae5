"""Install the MI355X gated delta rule into transformers' Qwen3.5-family models, so existing training and inference
code runs the HIP kernels without changes: the models call the module-level function torch_chunk_gated_delta_rule by
name, and install() swaps that name in the Qwen3.5, Qwen3.5-MoE and Qwen3-Next modeling modules (reference
src/macai/patch.py:27-56, 77-98; the layer / training / LoRA hooks of the reference are outside this build).  With
decode=True it also swaps torch_recurrent_gated_delta_rule, which the reference leaves unpatched.

    import macai.patch
    macai.patch.install()          # every loaded or later-loaded Qwen3.5 / Qwen3.5-MoE / Qwen3-Next model
    with macai.patch.installed():  # or only inside a block
        ...
"""
import contextlib
import importlib

from .gated_delta import chunk_gated_delta_rule, recurrent_gated_delta_rule

MODULES = ("transformers.models.qwen3_5.modeling_qwen3_5", "transformers.models.qwen3_5_moe.modeling_qwen3_5_moe",
           "transformers.models.qwen3_next.modeling_qwen3_next")
NAME = "torch_chunk_gated_delta_rule"
DECODE_NAME = "torch_recurrent_gated_delta_rule"
_saved = {}


def install(decode: bool = False) -> list:
    """Swap the rule in every module that has it; returns the (module, name) pairs patched."""
    done = []
    swaps = [(NAME, chunk_gated_delta_rule)] + ([(DECODE_NAME, recurrent_gated_delta_rule)] if decode else [])
    for path in MODULES:
        try:
            mod = importlib.import_module(path)
        except ImportError:
            continue
        for name, fn in swaps:
            if hasattr(mod, name) and getattr(mod, name) is not fn:
                _saved.setdefault((path, name), getattr(mod, name))
                setattr(mod, name, fn)
                done.append((path, name))
    return done


def uninstall() -> None:
    for (path, name), fn in list(_saved.items()):
        setattr(importlib.import_module(path), name, fn)
        del _saved[(path, name)]


@contextlib.contextmanager
def installed(decode: bool = False):
    install(decode=decode)
    try:
        yield
    finally:
        uninstall()

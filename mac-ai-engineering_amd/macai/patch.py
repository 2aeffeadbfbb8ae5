"""Put the MI355X gated delta rule into transformers' Qwen3.5-family models, so that existing training and inference
code runs the HIP kernels unchanged.

Those models reach the rule through the module-level name torch_chunk_gated_delta_rule, looked up at every call.
install() rebinds that name in the Qwen3.5, Qwen3.5-MoE and Qwen3-Next modeling modules and remembers the original,
uninstall() rebinds the originals, and installed() does both around a block (the reference's installer,
src/macai/patch.py:27-98, keeps the same three names and keywords).  decode=True also rebinds
torch_recurrent_gated_delta_rule, which the reference leaves to PyTorch.

The reference's installer can also replace methods of the rest of the layer, of the training path and of PEFT's LoRA
layer (its layer, training and lora keywords).  Those parts are not part of this build: the keywords are accepted,
asking for them (the default, as in the reference) installs the rule and warns once that they are absent, and
layer_patches(), training_patches() and lora_patches() report that nothing of theirs is installed.

Usage:

    from macai import patch
    patch.install()                # the models of every module above, loaded now or later
    with patch.installed():        # only for the duration of the block
        model(**batch)
"""
import contextlib
import importlib
import warnings

from .gated_delta import chunk_gated_delta_rule, recurrent_gated_delta_rule

MODULES = ("transformers.models.qwen3_5.modeling_qwen3_5", "transformers.models.qwen3_5_moe.modeling_qwen3_5_moe",
           "transformers.models.qwen3_next.modeling_qwen3_next")
NAME = "torch_chunk_gated_delta_rule"
DECODE_NAME = "torch_recurrent_gated_delta_rule"
# the reference installer's other parts, none of which this build provides
ABSENT_PARTS = ("layer", "training", "lora")
_saved = {}
_warned = set()


def _warn_absent(asked):
    missing = [p for p in asked if p not in _warned]
    if missing:
        _warned.update(missing)
        warnings.warn(f"macai.patch: this build installs the gated delta rule only; the {', '.join(missing)} part(s) "
                      "of the reference's installer are not provided (pass layer=False, training=False, lora=False to "
                      "silence this)", RuntimeWarning, stacklevel=3)


def install(layer: bool = True, training: bool = True, lora: bool = True, *, decode: bool = False) -> list:
    """Rebind the rule's name (and with decode the recurrent step's) in every module above that can be imported;
    returns the paths of the modules changed by this call, as the reference's install() does (patch.py:33-56).
    layer / training / lora keep the reference's positions and ask for parts this build does not have: nothing is
    installed for them and a RuntimeWarning says so once per part.  decode is keyword-only."""
    _warn_absent([p for p, on in zip(ABSENT_PARTS, (layer, training, lora)) if on])
    swaps = [(NAME, chunk_gated_delta_rule)] + ([(DECODE_NAME, recurrent_gated_delta_rule)] if decode else [])
    changed = []
    for path in MODULES:
        try:
            mod = importlib.import_module(path)
        except ImportError:
            continue
        for name, fn in swaps:
            if hasattr(mod, name) and getattr(mod, name) is not fn:
                _saved.setdefault((path, name), getattr(mod, name))
                setattr(mod, name, fn)
                if path not in changed:
                    changed.append(path)
    return changed


def swapped() -> list:
    """The (module path, name) pairs currently rebound by install()."""
    return list(_saved)


def layer_patches() -> list:
    """The layer parts' methods installed: none (this build replaces the rule only)."""
    return []


def training_patches() -> list:
    """The training path's methods installed: none (this build replaces the rule only)."""
    return []


def lora_patches() -> list:
    """The LoRA adapter path's methods installed: none (this build replaces the rule only)."""
    return []


def uninstall() -> None:
    """Rebind every name install() changed to what it was before."""
    for (path, name), fn in list(_saved.items()):
        setattr(importlib.import_module(path), name, fn)
        del _saved[(path, name)]


@contextlib.contextmanager
def installed(layer: bool = True, training: bool = True, lora: bool = True, *, decode: bool = False):
    """install() for the duration of a with-block, then uninstall()."""
    install(layer=layer, training=training, lora=lora, decode=decode)
    try:
        yield
    finally:
        uninstall()

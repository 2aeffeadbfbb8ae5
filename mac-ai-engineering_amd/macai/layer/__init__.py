"""The producers of the gated delta rule's inputs in the Qwen3.5 / Qwen3-Next linear-attention layer, on MI355X:
the convolution path (q, k, v from the input projection) and the gates (beta, g).  The reference's macai.layer holds
the whole decoder layer; only these two parts feed the rule (reference layer/_conv.py, layer/_gates.py)."""
from ._conv import ConvQKV, conv_qkv
from ._gates import Gates, gates

__all__ = ["ConvQKV", "conv_qkv", "Gates", "gates"]

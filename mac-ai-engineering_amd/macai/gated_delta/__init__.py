"""The gated delta rule (Qwen3.5 / Qwen3-Next linear attention) as HIP kernels for PyTorch-ROCm on MI355X."""
from .op import (GatedDeltaRule, chunk_gated_delta_rule, l2norm, recurrent_gated_delta_rule,
                 recurrent_reference)

__all__ = ["GatedDeltaRule", "chunk_gated_delta_rule", "l2norm", "recurrent_gated_delta_rule", "recurrent_reference"]

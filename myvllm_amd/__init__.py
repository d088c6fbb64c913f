"""MI355X (gfx950) kernels for the Gated DeltaNet linear-attention path.

Public ops keep the names and signatures of yuyifanbupt/myvllm's
``myvllm.ops.gated_delta_rule.gated_delta_rule`` and ``myvllm.ops.causal_conv1d``.
"""
from .causal_conv1d import causal_conv1d_fn, causal_conv1d_update
from .gated_delta_rule import (
    chunk_gated_delta_rule,
    chunk_gated_delta_rule_fwd,
    gated_delta_net_decode_step,
    recurrent_gated_delta_rule,
)

__all__ = [
    "causal_conv1d_fn",
    "causal_conv1d_update",
    "chunk_gated_delta_rule",
    "chunk_gated_delta_rule_fwd",
    "gated_delta_net_decode_step",
    "recurrent_gated_delta_rule",
]

"""MI355X (gfx950) kernels for the Gated DeltaNet linear-attention path and
the full-attention layers beside it.

Public ops keep the names and signatures of yuyifanbupt/myvllm's
``myvllm.ops.gated_delta_rule.gated_delta_rule``, ``myvllm.ops.causal_conv1d`` and
``myvllm.ops.full_attention``.
"""
from .causal_conv1d import causal_conv1d_fn, causal_conv1d_update
from .full_attention import (
    flash_attention_prefill,
    paged_flash_attention_decode,
    paged_flash_attention_prefill,
)
from .norm import RMSNormGated
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
    "flash_attention_prefill",
    "paged_flash_attention_decode",
    "paged_flash_attention_prefill",
    "chunk_gated_delta_rule_fwd",
    "gated_delta_net_decode_step",
    "recurrent_gated_delta_rule",
    "RMSNormGated",
]

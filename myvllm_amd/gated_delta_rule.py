"""Gated delta rule ops with the reference's signatures, on HIP kernels.

Drop-in for ``myvllm.ops.gated_delta_rule.gated_delta_rule`` (yuyifanbupt/myvllm,
``ops/gated_delta_rule/gated_delta_rule.py:31-92``): same function names,
argument order and meaning, output allocated by the op in v's dtype, state
cache updated in place at the indexed slots.  Differences (all deliberate):

* the prefill reads the initial state from ``recurrent_state[idx[n]]`` (the
  reference kernel starts from zero, ``ops/gated_delta_rule/h.py:61-67``);
* no host synchronisation (the reference calls ``.item()`` per sequence,
  ``gated_delta_rule.py:19``, ``:23``, ``:61``), so calls are stream-ordered;
* slot ids outside ``[0, num_slots)`` mark padding sequences (zero output,
  state untouched);
* bad arguments raise ``ValueError``/``GdnError`` instead of failing inside a
  kernel.
"""
from __future__ import annotations

import torch

from . import _lib

CHUNK_SIZE = 64


def _lastdim_contiguous(t: torch.Tensor) -> torch.Tensor:
    return t if t.stride(-1) == 1 else t.contiguous()


def chunk_gated_delta_rule(
    q: torch.Tensor,  # (total_tokens, num_k_heads, k_head_dim) bf16
    k: torch.Tensor,  # (total_tokens, num_k_heads, k_head_dim) bf16
    v: torch.Tensor,  # (total_tokens, num_v_heads, v_head_dim) bf16
    g: torch.Tensor,  # (total_tokens, num_v_heads) fp32 log-decay
    beta: torch.Tensor,  # (total_tokens, num_v_heads)
    recurrent_state: torch.Tensor,  # (max_seq_cnt, num_v_heads, k_head_dim, v_head_dim) fp32
    recurrent_state_indices: torch.Tensor,  # (seq_cnt,)
    cu_seqlens: torch.Tensor,  # (seq_cnt + 1,)
    scale: float | None = None,
) -> torch.Tensor:
    """Prefill over packed varlen sequences (reference ``gated_delta_rule.py:31-66``)."""
    dev = _lib.require_device(q, k, v, g, beta, recurrent_state, recurrent_state_indices, cu_seqlens)
    q, k, v = _lastdim_contiguous(q), _lastdim_contiguous(k), _lastdim_contiguous(v)
    if g.dtype != torch.float32:
        g = g.float()
    if scale is None:
        scale = k.shape[-1] ** -0.5
    o = torch.empty(v.shape, dtype=v.dtype, device=dev)
    lib = _lib.load()
    D = _lib.describe
    rc = lib.gdn_chunk_prefill(
        D(q), D(k), D(v), D(g), D(beta), D(recurrent_state), D(recurrent_state_indices), D(cu_seqlens), D(o),
        float(scale), CHUNK_SIZE, _lib.stream_handle(dev),
    )
    _lib.check("gdn_chunk_prefill", rc)
    return o


def recurrent_gated_delta_rule(
    q: torch.Tensor,  # (seq_cnt, num_k_heads, k_head_dim)
    k: torch.Tensor,  # (seq_cnt, num_k_heads, k_head_dim)
    v: torch.Tensor,  # (seq_cnt, num_v_heads, v_head_dim)
    g: torch.Tensor,  # (seq_cnt, num_v_heads)
    beta: torch.Tensor,  # (seq_cnt, num_v_heads)
    recurrent_state: torch.Tensor,  # (max_seq_cnt, num_v_heads, k_head_dim, v_head_dim) fp32
    recurrent_state_indices: torch.Tensor,  # (seq_cnt,)
    scale: float | None = None,
) -> torch.Tensor:
    """Decode step, one token per sequence (reference ``gated_delta_rule.py:69-92``)."""
    dev = _lib.require_device(q, k, v, g, beta, recurrent_state, recurrent_state_indices)
    q, k, v = _lastdim_contiguous(q), _lastdim_contiguous(k), _lastdim_contiguous(v)
    if scale is None:
        scale = k.shape[-1] ** -0.5
    o = torch.empty(v.shape, dtype=v.dtype, device=dev)
    lib = _lib.load()
    D = _lib.describe
    rc = lib.gdn_recurrent_step(
        D(q), D(k), D(v), D(g), D(beta), D(recurrent_state), D(recurrent_state_indices), D(o),
        float(scale), _lib.stream_handle(dev),
    )
    _lib.check("gdn_recurrent_step", rc)
    return o


def chunk_gated_delta_rule_fwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    cu_seqlens: torch.Tensor,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    scale: float | None = None,
):
    """Functional form: ``initial_state`` (N, Hv, K, V) fp32 in, ``(o, final_state)`` out.

    Implemented as :func:`chunk_gated_delta_rule` over a temporary cache whose
    slot n belongs to sequence n.
    """
    N = cu_seqlens.numel() - 1
    Hv, V = v.shape[1], v.shape[2]
    K = k.shape[2]
    if initial_state is None:
        cache = torch.zeros(N, Hv, K, V, dtype=torch.float32, device=v.device)
    else:
        cache = initial_state.to(torch.float32).clone()
    idx = torch.arange(N, dtype=torch.int32, device=v.device)
    o = chunk_gated_delta_rule(q, k, v, g, beta, cache, idx, cu_seqlens, scale=scale)
    return o, (cache if output_final_state else None)

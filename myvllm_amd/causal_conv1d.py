"""Causal conv1d ops with the reference's signatures, on HIP kernels.

Drop-in for ``myvllm.ops.causal_conv1d`` (yuyifanbupt/myvllm,
``ops/causal_conv1d.py:221-273`` and ``:434-470``): same names, argument order
and meaning (x (T, D), weight (D, W), conv_state (slots, W-1, D) oldest row
first, int32 indices and cu_seqlens), output allocated in x's dtype, conv
state updated in place.  The decode update shifts the new token into the
state (the reference kernel writes the old state back unchanged,
``ops/causal_conv1d.py:413-431``).  No host synchronisation (the reference
calls ``.tolist()`` on cu_seqlens, ``:230``).
"""
from __future__ import annotations

import torch

from . import _lib


def causal_conv1d_fn(
    x: torch.Tensor,  # (total_tokens, dim)
    weight: torch.Tensor,  # (dim, kernel_size)
    conv_state: torch.Tensor,  # (max_seq_cnt, kernel_size - 1, dim)
    conv_state_indices: torch.Tensor,  # (seq_cnt,)
    cu_seqlens: torch.Tensor,  # (seq_cnt + 1,)
) -> torch.Tensor:
    """Varlen prefill conv + SiLU with conv-state carry (reference ``causal_conv1d.py:221-273``)."""
    dev = _lib.require_device(x, weight, conv_state, conv_state_indices, cu_seqlens)
    if x.stride(-1) != 1:
        x = x.contiguous()
    o = torch.empty(x.shape, dtype=x.dtype, device=dev)
    D = _lib.describe
    rc = _lib.load().causal_conv1d_varlen(
        D(x), D(weight), D(conv_state), D(conv_state_indices), D(cu_seqlens), D(o), _lib.stream_handle(dev)
    )
    _lib.check("causal_conv1d_varlen", rc)
    return o


def causal_conv1d_update(
    x: torch.Tensor,  # (seq_cnt, dim)
    weight: torch.Tensor,  # (dim, kernel_size)
    conv_state: torch.Tensor,  # (max_seq_cnt, kernel_size - 1, dim)
    conv_state_indices: torch.Tensor,  # (seq_cnt,)
) -> torch.Tensor:
    """Single-token decode conv + SiLU (reference ``causal_conv1d.py:434-470``)."""
    dev = _lib.require_device(x, weight, conv_state, conv_state_indices)
    if x.stride(-1) != 1:
        x = x.contiguous()
    o = torch.empty(x.shape, dtype=x.dtype, device=dev)
    D = _lib.describe
    rc = _lib.load().causal_conv1d_step(
        D(x), D(weight), D(conv_state), D(conv_state_indices), D(o), _lib.stream_handle(dev)
    )
    _lib.check("causal_conv1d_step", rc)
    return o

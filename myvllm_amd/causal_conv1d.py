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
    l2norm_channels: int = 0,
) -> torch.Tensor:
    """Varlen prefill conv + SiLU with conv-state carry (reference ``causal_conv1d.py:221-273``).

    ``l2norm_channels > 0`` (a multiple of 128) also applies the layer's
    per-head L2 norm ``y * rsqrt(sum y^2 + 1e-6)`` over 128-channel heads to
    the first ``l2norm_channels`` output channels (the q and k of
    ``layers/linear_attention.py:113-114``), in fp32 before the one rounding
    to x's dtype.
    """
    dev = _lib.require_device(x, weight, conv_state, conv_state_indices, cu_seqlens)
    x = _lib.vec16(x)
    o = torch.empty(x.shape, dtype=x.dtype, device=dev)
    D = _lib.describe
    lib = _lib.load()
    if l2norm_channels:
        rc = lib.causal_conv1d_varlen_qknorm(
            D(x), D(weight), D(conv_state), D(conv_state_indices), D(cu_seqlens), D(o), int(l2norm_channels),
            _lib.stream_handle(dev),
        )
        _lib.check("causal_conv1d_varlen_qknorm", rc)
    else:
        rc = lib.causal_conv1d_varlen(
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

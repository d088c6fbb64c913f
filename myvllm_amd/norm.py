"""Gated RMSNorm of the GDN output on a HIP kernel.

Same math as ``RMSNormGated.forward`` (``layers/norm.py:50-58`` of
yuyifanbupt/myvllm): ``x * rsqrt(mean(x^2) + eps) * weight * silu(gate)`` over
the last dim in fp32, output in x's dtype.  The layer applies it per v-head
(``normalized_shape = (v_head_dim,)``, ``layers/linear_attention.py:59``, ``:121``).
"""
from __future__ import annotations

import torch

from . import _lib


def rms_norm_gated(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """x, gate: (T, H, 128) (or any (..., H, 128) view with unit inner stride); weight: (128,)."""
    dev = _lib.require_device(x, gate, weight)
    shape = x.shape
    x3 = x.reshape(-1, shape[-2], shape[-1]) if x.dim() != 3 else x
    g3 = gate.reshape(x3.shape) if gate.shape != x3.shape else gate
    out = torch.empty(x3.shape, dtype=x.dtype, device=dev)
    D = _lib.describe
    rc = _lib.load().gdn_rms_norm_gated(D(x3), D(g3), D(weight), D(out), float(eps), _lib.stream_handle(dev))
    _lib.check("gdn_rms_norm_gated", rc)
    return out.reshape(shape)


def gdn_gating(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    """The layer's gates (``layers/linear_attention.py:89-90``) in one launch:
    g = -exp(A_log) softplus(a + dt_bias), beta = sigmoid(b), both fp32 (T, H)."""
    dev = _lib.require_device(a, b, A_log, dt_bias)
    g = torch.empty(a.shape, dtype=torch.float32, device=dev)
    beta = torch.empty(a.shape, dtype=torch.float32, device=dev)
    D = _lib.describe
    rc = _lib.load().gdn_gating(D(a), D(b), D(A_log), D(dt_bias), D(g), D(beta), _lib.stream_handle(dev))
    _lib.check("gdn_gating", rc)
    return g, beta

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
    """Normalises over the last dim N of x (any shape (..., N)); gate has x's
    shape; weight is (N,), or (H, N) for x of shape (..., H, N) (the
    reference's weight of normalized_shape broadcast over the leading dims)."""
    dev = _lib.require_device(x, gate, weight)
    if gate.shape != x.shape:
        raise ValueError(f"gate shape {tuple(gate.shape)} != x shape {tuple(x.shape)}")
    shape = x.shape
    if weight.dim() == 2:
        x3 = x.reshape(-1, shape[-2], shape[-1])
    elif x.dim() >= 3:
        x3 = x.reshape(-1, shape[-2], shape[-1])
    else:
        x3 = x.reshape(-1, 1, shape[-1])
    g3 = gate.reshape(x3.shape)
    if x3.stride(-1) != 1:
        x3 = x3.contiguous()
    if g3.stride(-1) != 1:
        g3 = g3.contiguous()
    out = torch.empty(x3.shape, dtype=x.dtype, device=dev)
    D = _lib.describe
    rc = _lib.load().gdn_rms_norm_gated(D(x3), D(g3), D(weight), D(out), float(eps), _lib.stream_handle(dev))
    _lib.check("gdn_rms_norm_gated", rc)
    return out.reshape(shape)


class RMSNormGated(torch.nn.Module):
    """Drop-in for ``RMSNormGated`` (``layers/norm.py:44-58``): same
    constructor arguments, ``weight`` parameter and ``forward(x, gate)``, on
    the HIP kernel (no torch.compile)."""

    def __init__(self, normalized_shape, eps: float = 1e-6, device=None) -> None:
        super().__init__()
        self.weight = torch.nn.Parameter(torch.ones(normalized_shape, device=device))
        self.variance_epsilon = eps

    def forward(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        w = self.weight
        if w.dim() > 2:
            raise ValueError("normalized_shape of more than two dims is not supported")
        return rms_norm_gated(x, gate, w, self.variance_epsilon)


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

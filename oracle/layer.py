"""CPU restatement of the GDN layer glue around the hot path (test oracle only).

* gating: beta = sigmoid(b); g = -exp(A_log) * softplus(a + dt_bias) in fp32
  (``layers/linear_attention.py:89-90``);
* per-head L2 norm: x * rsqrt(sum x^2 + 1e-6) (``layers/linear_attention.py:113-114``);
* gated RMSNorm: x * rsqrt(mean x^2 + eps) * w * silu(gate), fp32 math, output in
  x's dtype (``layers/norm.py:50-58``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def gdn_gating_ref(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor):
    beta = b.sigmoid()
    g = -A_log.float().exp() * F.softplus(a.float() + dt_bias)
    return g, beta


def l2norm_ref(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).sum(dim=-1, keepdim=True) + eps)


def rms_norm_gated_ref(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    dt = x.dtype
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True) + eps
    y = xf * var.rsqrt() * weight.float() * F.silu(gate.float())
    return y.to(dt)

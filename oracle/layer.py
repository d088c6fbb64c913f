"""CPU restatement of the GDN layer glue around the hot path (test oracle only).

* gating: beta = sigmoid(b); g = -exp(A_log) * softplus(a + dt_bias) in fp32
  (``layers/linear_attention.py:89-90``);
* per-head L2 norm: x * rsqrt(sum x^2 + 1e-6) (``layers/linear_attention.py:113-114``);
* gated RMSNorm: x * rsqrt(mean x^2 + eps) * w * silu(gate), fp32 math, output in
  x's dtype (``layers/norm.py:50-58``);
* the decode branch of the layer as one step: conv update, split, L2 norm,
  gating, recurrent step (``layers/linear_attention.py:89-90``, ``:95``,
  ``:97-114``, ``:119``), composed from the restatements above and in
  ``oracle.conv`` / ``oracle.gdn``.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from .conv import causal_conv1d_fn_ref, causal_conv1d_update_ref
from .gdn import chunk_gated_delta_rule_ref, recurrent_gated_delta_rule_ref


def gdn_gating_ref(a: torch.Tensor, b: torch.Tensor, A_log: torch.Tensor, dt_bias: torch.Tensor,
                   dtype: torch.dtype | None = None):
    """g, beta as the layer forms them; ``dtype`` (e.g. fp64) evaluates the same
    formulas in that dtype instead of the layer's fp32 / b-dtype mix."""
    if dtype is not None:
        return -A_log.to(dtype).exp() * F.softplus(a.to(dtype) + dt_bias.to(dtype)), b.to(dtype).sigmoid()
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


def gdn_decode_step_ref(mixed_qkv, conv_weight, conv_state, conv_state_indices, a, b, A_log, dt_bias,
                        recurrent_state, recurrent_state_indices, num_k_heads, scale=None):
    """One decode token of the layer's recurrent part, in fp64 with no rounding
    between the pieces; mutates both caches, returns o (B, Hv, V) in
    ``mixed_qkv``'s dtype."""
    B = mixed_qkv.shape[0]
    Hv, K, V = recurrent_state.shape[1], recurrent_state.shape[2], recurrent_state.shape[3]
    Hk = num_k_heads
    y = causal_conv1d_update_ref(mixed_qkv.double(), conv_weight, conv_state, conv_state_indices)  # fp64
    q, k, v = torch.split(y, [Hk * K, Hk * K, Hv * V], dim=-1)
    q = l2norm_ref(q.reshape(B, Hk, K))
    k = l2norm_ref(k.reshape(B, Hk, K))
    v = v.reshape(B, Hv, V)
    g, beta = gdn_gating_ref(a, b, A_log, dt_bias, dtype=torch.float64)
    o = recurrent_gated_delta_rule_ref(q, k, v, g, beta, recurrent_state, recurrent_state_indices, scale=scale)
    return o.to(mixed_qkv.dtype)


def gdn_layer_ref(x, w_qkvz, w_ba, conv_weight, A_log, dt_bias, norm_weight, w_out, conv_state, conv_state_indices,
                  recurrent_state, recurrent_state_indices, cu_seqlens, num_k_heads, num_decode_tokens=0,
                  eps=1e-6):
    """The layer's intended forward (``layers/linear_attention.py:85-122`` with the
    conv on the qkv projection and the norm on o) over a mixed batch: prefill
    tokens first (``cu_seqlens``), then ``num_decode_tokens`` single-token
    sequences.  Values are rounded to x's dtype where the reference layer's
    ops return that dtype: the projections (``layers/linear.py:29-30``), the
    conv output (``ops/causal_conv1d.py:241``; here after the per-head L2
    norm, which the layer applies to it), the GDN output o (``v.dtype``,
    ``ops/gated_delta_rule/o.py:147``, ``fused_recurrent_gdn.py:116``) and
    the gated norm's output (``layers/norm.py:58``); everything between is
    fp64 (the gated norm fp32).  Mutates both caches; returns (T, hidden) in
    x's dtype."""
    T = x.shape[0]
    Hv, K, V = recurrent_state.shape[1], recurrent_state.shape[2], recurrent_state.shape[3]
    Hk = num_k_heads
    Dc = 2 * Hk * K + Hv * V
    Tp = T - num_decode_tokens
    Np = cu_seqlens.numel() - 1 if Tp > 0 else 0
    xd = x.double()
    qkvz = (xd @ w_qkvz.double().t()).to(x.dtype).double()
    ba = (xd @ w_ba.double().t()).to(x.dtype).double()
    qkv, z = qkvz[:, :Dc], qkvz[:, Dc:]
    b, a = ba[:, :Hv], ba[:, Hv:]
    o = torch.zeros(T, Hv, V, dtype=torch.float64)
    if Tp > 0:
        y = causal_conv1d_fn_ref(qkv[:Tp], conv_weight, conv_state, conv_state_indices[:Np], cu_seqlens)
        q = l2norm_ref(y[:, : Hk * K].reshape(Tp, Hk, K)).to(x.dtype).double()
        k = l2norm_ref(y[:, Hk * K: 2 * Hk * K].reshape(Tp, Hk, K)).to(x.dtype).double()
        v = y[:, 2 * Hk * K:].reshape(Tp, Hv, V).to(x.dtype).double()
        g, beta = gdn_gating_ref(a[:Tp], b[:Tp], A_log, dt_bias, dtype=torch.float64)
        o[:Tp] = chunk_gated_delta_rule_ref(q, k, v, g, beta, recurrent_state, recurrent_state_indices[:Np],
                                            cu_seqlens)
    if num_decode_tokens > 0:
        o[Tp:] = gdn_decode_step_ref(qkv[Tp:], conv_weight, conv_state, conv_state_indices[Np:], a[Tp:], b[Tp:],
                                     A_log, dt_bias, recurrent_state, recurrent_state_indices[Np:], Hk)
    o = o.to(x.dtype)
    on = rms_norm_gated_ref(o, z.reshape(T, Hv, V).to(x.dtype), norm_weight, eps=eps).double()
    return (on.reshape(T, Hv * V) @ w_out.double().t()).to(x.dtype)

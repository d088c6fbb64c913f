"""CPU restatement of the reference's depthwise causal conv1d + SiLU (test oracle only).

Conventions (``ops/causal_conv1d.py``, relative to the reference package):

* x: (T, D) packed tokens; weight: (D, W) (the ``conv1d`` weight of
  ``layers/linear_attention.py:48-56`` is an (out=D, in=W) linear weight);
* conv_state: (num_slots, W-1, D), token-major, oldest row first
  (``ops/causal_conv1d.py:16``, ``:41-63``);
* no bias; fp32 accumulation; SiLU; output in x's dtype (``:182``, ``:195``, ``:241``).

Math (intended; the reference kernel's pointer bugs are not reproduced):
  xt = [conv_state[slot] ; x_seq];  y_t = silu(sum_j w[:, j] * xt[t + j]);
  conv_state[slot] <- last W-1 rows of xt  (``:138-218``).
Decode update (``:276-431``): xt = [state ; x_b], y = silu(sum_j w[:, j] xt[j]),
state <- xt[1:] (the reference writes back the unshifted state, ``:413-431``;
the intended shift is restated here).  Slots outside ``[0, num_slots)`` mark a
padding sequence: zero output, state untouched.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def causal_conv1d_fn_ref(
    x: torch.Tensor,
    weight: torch.Tensor,
    conv_state: torch.Tensor,
    conv_state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    dtype: torch.dtype = torch.float64,
) -> torch.Tensor:
    """Varlen prefill via ``F.conv1d(groups=D)`` per sequence; mutates ``conv_state``."""
    T, D = x.shape
    W = weight.shape[1]
    cu = [int(c) for c in cu_seqlens.tolist()]
    idx = [int(c) for c in conv_state_indices.tolist()]
    num_slots = conv_state.shape[0]
    out = torch.zeros(T, D, dtype=dtype)
    wf = weight.to(dtype)[:, None, :]  # (D, 1, W)
    for n in range(len(cu) - 1):
        s, e = cu[n], cu[n + 1]
        slot = idx[n]
        if e <= s or slot < 0 or slot >= num_slots:
            continue
        xt = torch.cat([conv_state[slot].to(dtype), x[s:e].to(dtype)], 0)  # (W-1+L, D)
        y = F.conv1d(xt.t()[None], wf, groups=D)[0].t()  # (L, D)
        out[s:e] = F.silu(y)
        conv_state[slot] = xt[-(W - 1):].to(conv_state.dtype)
    return out.to(x.dtype)


def causal_conv1d_update_ref(
    x: torch.Tensor,
    weight: torch.Tensor,
    conv_state: torch.Tensor,
    conv_state_indices: torch.Tensor,
    dtype: torch.dtype = torch.float64,
) -> torch.Tensor:
    """Single-token decode update for a batch of B sequences; mutates ``conv_state``."""
    B, D = x.shape
    num_slots = conv_state.shape[0]
    out = torch.zeros(B, D, dtype=dtype)
    wf = weight.to(dtype)
    for b, slot in enumerate(int(c) for c in conv_state_indices.tolist()):
        if slot < 0 or slot >= num_slots:
            continue
        xt = torch.cat([conv_state[slot].to(dtype), x[b : b + 1].to(dtype)], 0)  # (W, D)
        out[b] = F.silu((xt.t() * wf).sum(-1))
        conv_state[slot] = xt[1:].to(conv_state.dtype)
    return out.to(x.dtype)


def causal_conv1d_loop_ref(x, weight, conv_state, conv_state_indices, cu_seqlens):
    """Brute-force scalar loop (fp64 Python floats) for tiny inputs; returns (out, new_state)."""
    T, D = x.shape
    W = weight.shape[1]
    cs = conv_state.clone()
    out = torch.zeros(T, D, dtype=torch.float64)
    cu = [int(c) for c in cu_seqlens.tolist()]
    for n in range(len(cu) - 1):
        slot = int(conv_state_indices[n])
        s, e = cu[n], cu[n + 1]
        if e <= s or slot < 0 or slot >= cs.shape[0]:
            continue
        for d in range(D):
            hist = [float(conv_state[slot, r, d]) for r in range(W - 1)]
            for t in range(s, e):
                hist.append(float(x[t, d]))
                acc = 0.0
                for j in range(W):
                    acc += float(weight[d, j]) * hist[len(hist) - W + j]
                out[t, d] = acc / (1.0 + math.exp(-acc))
            for r in range(W - 1):
                cs[slot, r, d] = hist[len(hist) - (W - 1) + r]
    return out, cs

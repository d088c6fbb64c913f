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
    q: torch.Tensor,  # (total_tokens, num_k_heads, k_head_dim) bf16, fp16 or fp32
    k: torch.Tensor,  # (total_tokens, num_k_heads, k_head_dim) q's dtype
    v: torch.Tensor,  # (total_tokens, num_v_heads, v_head_dim) q's dtype
    g: torch.Tensor,  # (total_tokens, num_v_heads) fp32 log-decay
    beta: torch.Tensor,  # (total_tokens, num_v_heads)
    recurrent_state: torch.Tensor,  # (max_seq_cnt, num_v_heads, k_head_dim, v_head_dim) fp32
    recurrent_state_indices: torch.Tensor,  # (seq_cnt,)
    cu_seqlens: torch.Tensor,  # (seq_cnt + 1,)
    scale: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Prefill over packed varlen sequences (reference ``gated_delta_rule.py:31-66``);
    ``out`` (optional) receives o in place of a new tensor."""
    dev = _lib.require_device(q, k, v, g, beta, recurrent_state, recurrent_state_indices, cu_seqlens)
    q, k, v = _lib.vec16(q), _lib.vec16(k), _lib.vec16(v)
    if g.dtype != torch.float32:
        g = g.float()
    if scale is None:
        scale = k.shape[-1] ** -0.5
    if torch.float32 in (q.dtype, k.dtype, v.dtype):
        if not q.dtype == k.dtype == v.dtype:
            raise ValueError(f"q, k and v must share one dtype (got {q.dtype}, {k.dtype}, {v.dtype})")
        return _chunk_gated_delta_rule_fp32(q, k, v, g, beta, recurrent_state, recurrent_state_indices, cu_seqlens,
                                            scale, out)
    # (an out the kernel cannot write with 16-byte stores is filled through a temporary)
    o = torch.empty(v.shape, dtype=v.dtype, device=dev) if out is None or not _lib.vec16_ok(out) else out
    lib = _lib.load()
    D = _lib.describe
    rc = lib.gdn_chunk_prefill(
        D(q), D(k), D(v), D(g), D(beta), D(recurrent_state), D(recurrent_state_indices), D(cu_seqlens), D(o),
        float(scale), CHUNK_SIZE, _lib.stream_handle(dev),
    )
    _lib.check("gdn_chunk_prefill", rc)
    if out is not None and o is not out:
        out.copy_(o)
        return out
    return o


def chunk_prefill_ex(q, k, v, g, beta, state, idx, cu_seqlens, out, scale, flags=0, items_per_wg=-1,
                     spin_limit=-1):
    """``gdn_chunk_prefill_ex``: the prefill with its options (flags
    ``_lib.PREFILL_*``, the schedule and the bound of the kernel's internal
    waits; include/gdn_hip.h).  q, k, v bf16 or fp16, last stride 1; out
    v's dtype, or fp32 for fp16 inputs; nothing is converted or allocated."""
    dev = _lib.require_device(q, k, v, g, beta, state, idx, cu_seqlens, out)
    D = _lib.describe
    rc = _lib.load().gdn_chunk_prefill_ex(
        D(q), D(k), D(v), D(g), D(beta), D(state), D(idx), D(cu_seqlens), D(out), float(scale), CHUNK_SIZE,
        int(flags), int(items_per_wg), int(spin_limit), _lib.stream_handle(dev),
    )
    _lib.check("gdn_chunk_prefill_ex", rc)
    return out


def _chunk_gated_delta_rule_fp32(q, k, v, g, beta, state, idx, cu_seqlens, scale, out):
    """fp32 q, k, v through the fp16 kernel with fp32 output.  q and k are
    rounded to fp16, the MFMA operand type (the reference's kernels run their
    fp32 dots in tf32, whose 10-bit mantissa fp16 matches); v is split into
    v_hi = fp16(v) and v_lo = fp16(v - v_hi) (22 significant bits), and since
    the recurrence is linear in (state, v) jointly the kernel runs twice: from
    the slot's state with v_hi, writing o and the final state, then from a
    zero state with v_lo, adding its o and final state to them
    (GDN_PREFILL_ZERO_INIT | ACCUM_STATE | ACCUM_OUT).  Two launches, no
    temporary state, no host synchronisation; padding sequences' slots are
    not touched.  o keeps the fp32 range; v itself must stay below fp16's
    65504 in magnitude (v_hi would overflow), as for the 16-bit inputs."""
    dev = v.device
    qh, kh = q.to(torch.float16), k.to(torch.float16)
    v_hi = v.to(torch.float16)
    v_lo = (v - v_hi.float()).to(torch.float16)
    o = torch.empty(v.shape, dtype=torch.float32, device=dev) if out is None or not _lib.vec16_ok(out) else out
    chunk_prefill_ex(qh, kh, v_hi, g, beta, state, idx, cu_seqlens, o, scale)
    chunk_prefill_ex(qh, kh, v_lo, g, beta, state, idx, cu_seqlens, o, scale,
                     flags=_lib.PREFILL_ZERO_INIT | _lib.PREFILL_ACCUM_STATE | _lib.PREFILL_ACCUM_OUT)
    if out is not None and o is not out:
        out.copy_(o)
        return out
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


def gated_delta_net_decode_step(
    mixed_qkv: torch.Tensor,  # (B, 2 Hk K + Hv V): the qkv projection before the conv
    conv_weight: torch.Tensor,  # (D, 4)
    conv_state: torch.Tensor,  # (conv_slots, 3, D)
    conv_state_indices: torch.Tensor,  # (B,)
    a: torch.Tensor,  # (B, Hv) gate input
    b: torch.Tensor,  # (B, Hv) beta input
    A_log: torch.Tensor,  # (Hv,)
    dt_bias: torch.Tensor,  # (Hv,)
    recurrent_state: torch.Tensor,  # (slots, Hv, K, V) fp32
    recurrent_state_indices: torch.Tensor,  # (B,)
    num_k_heads: int,
    scale: float | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """The decode branch of ``GatedDeltaNet.forward`` in one launch (reference
    ``layers/linear_attention.py:89-90`` gating, ``:95`` ``causal_conv1d_update``,
    ``:113-114`` per-head L2 norm of q and k, ``:119`` ``recurrent_gated_delta_rule``).

    Returns o (B, Hv, V) in ``mixed_qkv``'s dtype and updates both caches in
    place.  The conv output, the normalised q and k and the gates stay in fp32
    between the steps (the separate ops round them to the input dtype).
    """
    dev = _lib.require_device(mixed_qkv, conv_weight, conv_state, conv_state_indices, a, b, A_log, dt_bias,
                              recurrent_state, recurrent_state_indices)
    mixed_qkv = _lastdim_contiguous(mixed_qkv)
    Hv, K, V = recurrent_state.shape[1], recurrent_state.shape[2], recurrent_state.shape[3]
    if scale is None:
        scale = K ** -0.5
    o = torch.empty((mixed_qkv.shape[0], Hv, V), dtype=mixed_qkv.dtype, device=dev) if out is None else out
    lib = _lib.load()
    D = _lib.describe
    rc = lib.gdn_decode_step_fused(
        D(mixed_qkv), D(conv_weight), D(conv_state), D(conv_state_indices), D(a), D(b), D(A_log), D(dt_bias),
        D(recurrent_state), D(recurrent_state_indices), D(o), int(num_k_heads), float(scale),
        _lib.stream_handle(dev),
    )
    _lib.check("gdn_decode_step_fused", rc)
    return o

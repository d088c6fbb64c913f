"""Full attention of the hybrid stack's attention layers, on HIP kernels.

Same names, arguments and results as ``ops/full_attention.py`` of
yuyifanbupt/myvllm (``flash_attention_prefill`` ``:114-173``,
``paged_flash_attention_decode`` ``:282-335``, ``paged_flash_attention_prefill``
``:454-512``), with the output on q's device in q's dtype.  GQA: query head h
reads kv head ``h // (Hq // Hkv)``.  Supported: bf16 / fp16, head dim 64, 128
or 256 for q, k and v alike.

Differences from the reference kernels, all in the reference's disfavour
(each is a defect of its Triton code, not an intended behaviour): K and V of
sequence n are read from that sequence's rows (``:57-72`` read from token 0),
the output's dim stride is the dim stride (``:76``), the non-causal path masks
keys past the sequence end, and the paged prefill reads its work list and
``cu_seqlens`` correctly (``:378-380``); a query with no visible key gives a
zero row instead of 0/0.
"""
from __future__ import annotations

import torch

from . import _lib


def _out_for(out, shape, dtype, dev):
    """The tensor the kernel writes: `out` itself when it has 16-byte aligned
    rows, else a temporary copied into `out` afterwards (_finish)."""
    if out is not None and _lib.vec16_ok(out):
        return out
    return torch.empty(shape, dtype=dtype, device=dev)


def _finish(out, o):
    if out is not None and o is not out:
        out.copy_(o)
        return out
    return o


_DECODE_MIN_SPLIT_KEYS = 256
_DECODE_TARGET_WAVES = 512   # unit x kv-head waves aimed at with splits
_DECODE_SPLIT_ROWS = 2048    # (sequence, kv head) rows from which one split is enough
_DECODE_MAX_SPLITS = 256


def _max_seqlen(cu_seqlens: torch.Tensor) -> int:
    if cu_seqlens.numel() < 2:
        return 0
    return int((cu_seqlens[1:] - cu_seqlens[:-1]).max().item())


def flash_attention_prefill(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens: torch.Tensor,
    scale: float,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    head_v_dim: int,
    is_causal: bool,
    max_seqlen: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Varlen attention over packed sequences: q (T, Hq, D), k, v (T, Hkv, D) ->
    (T, Hq, D).  ``max_seqlen`` (the longest sequence) is read from
    ``cu_seqlens`` when not given, one host sync as in the reference (``:139``)."""
    if q.shape[1] != num_heads or k.shape[1] != num_kv_heads or q.shape[2] != head_dim or v.shape[2] != head_v_dim:
        raise ValueError("q/k/v shapes disagree with num_heads/num_kv_heads/head_dim/head_v_dim")
    dev = _lib.require_device(q, k, v, cu_seqlens)
    if max_seqlen is None:
        max_seqlen = _max_seqlen(cu_seqlens)
    if head_dim not in _KERNEL_HEAD_DIMS or head_v_dim != head_dim:
        return _padded_prefill(q, k, v, cu_seqlens, scale, head_dim, head_v_dim, is_causal, max_seqlen, out)
    q, k, v = _lib.vec16(q), _lib.vec16(k), _lib.vec16(v)
    o = _out_for(out, (q.shape[0], q.shape[1], head_v_dim), q.dtype, dev)
    D = _lib.describe
    rc = _lib.load().flash_attention_varlen(
        D(q), D(k), D(v), D(cu_seqlens), D(o), int(max_seqlen), float(scale), int(bool(is_causal)),
        _lib.stream_handle(dev),
    )
    _lib.check("flash_attention_varlen", rc)
    return _finish(out, o)


_KERNEL_HEAD_DIMS = (64, 128, 256)


def _padded_prefill(q, k, v, cu_seqlens, scale, head_dim, head_v_dim, is_causal, max_seqlen, out):
    """Head dims the kernel has no instantiation for (the vision tower's
    1152 / 16 = 72, ``models/qwen/vision.py:18``, ``configs/qwen3_5.py:11``,
    ``:16``) run zero-padded to the next of 64, 128 and 256: zero dims add
    nothing to q.k and give zero output columns, which are dropped.  The
    padded copies cost one pass over q, k and v."""
    Dp = next((d for d in _KERNEL_HEAD_DIMS if d >= max(head_dim, head_v_dim)), None)
    if Dp is None:
        raise ValueError(f"head dims {head_dim}/{head_v_dim} above {_KERNEL_HEAD_DIMS[-1]} are not supported")
    pad = lambda t: torch.nn.functional.pad(t, (0, Dp - t.shape[-1]))
    o = flash_attention_prefill(pad(q), pad(k), pad(v), cu_seqlens, scale, q.shape[1], k.shape[1], Dp, Dp, is_causal,
                                max_seqlen=max_seqlen)
    return _finish(out, o[..., :head_v_dim]) if out is not None else o[..., :head_v_dim]


def decode_num_splits(num_seqs: int, num_q_heads: int, num_kv_heads: int, capacity: int) -> int:
    """Splits of the decode launch.  With num_splits > 1 the kernel deals the
    batch's 16-key tiles evenly over num_seqs x (num_splits - 1) units
    (whatever the context lengths), and each unit's waves write partials that
    a second launch merges; with one split a wave streams a whole sequence.
    Balanced units saturate HBM from about 512 waves (unit x kv head x
    query-head group) on; more waves only add partials and concurrent page
    streams (256 sequences of U[512, 4096] keys, 2 kv heads: 256 units 232
    us, 512 units 245, 1,024 units 245; 64 of U[2k, 32k]: 192 units 397 us,
    1,024 units 429).  So: about 512 waves, at least one unit per sequence
    (one split leaves ragged batches unbalanced), one split once the batch
    alone has 2048 rows, and at least 256 keys of the table's capacity per
    unit."""
    rows = max(1, num_seqs * num_kv_heads * ((num_q_heads // max(num_kv_heads, 1) + 15) // 16))
    if rows >= _DECODE_SPLIT_ROWS:
        return 1
    units = max(1, round(_DECODE_TARGET_WAVES / rows))
    by_keys = -(-max(capacity, 1) // _DECODE_MIN_SPLIT_KEYS)
    return max(1, min(_DECODE_MAX_SPLITS, 1 + min(units, by_keys)))


def paged_flash_attention_decode(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    num_splits: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """One query per sequence over its paged cache: q (B, Hq, D), caches
    (num_blocks, block_size, Hkv, D), block_tables (B, max_blocks),
    context_lens (B,) -> (B, Hq, D).  No host sync."""
    if k_cache.shape[1] != block_size:
        raise ValueError(f"block_size {block_size} != k_cache.shape[1] {k_cache.shape[1]}")
    dev = _lib.require_device(q, k_cache, v_cache, block_tables, context_lens)
    B, Hq, Dh = q.shape
    if num_splits is None:
        num_splits = decode_num_splits(B, Hq, k_cache.shape[2], block_tables.shape[1] * block_size)
    lib = _lib.load()
    ws = None
    n_ws = lib.paged_attention_decode_workspace_size(B, Hq, Dh, int(num_splits))
    if n_ws > 0:
        ws = torch.empty(n_ws, dtype=torch.float32, device=dev)
    q, k_cache, v_cache = _lib.vec16(q), _lib.vec16(k_cache), _lib.vec16(v_cache)
    o = _out_for(out, (B, Hq, v_cache.shape[-1]), q.dtype, dev)
    D = _lib.describe
    rc = lib.paged_attention_decode(
        D(q), D(k_cache), D(v_cache), D(block_tables), D(context_lens), D(o),
        D(ws) if ws is not None else None, int(num_splits), float(scale), _lib.stream_handle(dev),
    )
    _lib.check("paged_attention_decode", rc)
    return _finish(out, o)


def paged_flash_attention_decode_noalloc(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    block_size: int,
    num_splits: int,
    out: torch.Tensor,
) -> torch.Tensor:
    """:func:`paged_flash_attention_decode` for callers that cannot allocate
    device memory: ``out`` is required, ``num_splits`` is explicit, and the
    split partials live in the library's static device array (C entry
    ``paged_attention_decode_noalloc``; at most ``GDN_DECODE_SCRATCH_FLOATS``
    fp32 values, else ``GdnError``).  Calls that overlap in time on one GPU
    share that array and race; order them on one stream."""
    if k_cache.shape[1] != block_size:
        raise ValueError(f"block_size {block_size} != k_cache.shape[1] {k_cache.shape[1]}")
    dev = _lib.require_device(q, k_cache, v_cache, block_tables, context_lens, out)
    D = _lib.describe
    rc = _lib.load().paged_attention_decode_noalloc(
        D(q), D(k_cache), D(v_cache), D(block_tables), D(context_lens), D(out), int(num_splits), float(scale),
        _lib.stream_handle(dev),
    )
    _lib.check("paged_attention_decode_noalloc", rc)
    return out


def paged_flash_attention_prefill(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    page_block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    cu_seqlens: torch.Tensor,
    block_m_indices: torch.Tensor | None,
    scale: float,
    page_block_size: int,
    max_seqlen: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Prefill over a paged cache that already holds the new keys: query i of
    sequence n sits at position ``context_lens[n] - len_n + i`` and attends
    causally to the cached keys.  ``block_m_indices`` (the reference's
    per-16-row work list) is accepted for interface parity and not needed:
    the kernel tiles the queries itself from ``cu_seqlens``."""
    if k_cache.shape[1] != page_block_size:
        raise ValueError(f"page_block_size {page_block_size} != k_cache.shape[1] {k_cache.shape[1]}")
    dev = _lib.require_device(q, k_cache, v_cache, page_block_tables, context_lens, cu_seqlens)
    if max_seqlen is None:
        max_seqlen = _max_seqlen(cu_seqlens)
    q, k_cache, v_cache = _lib.vec16(q), _lib.vec16(k_cache), _lib.vec16(v_cache)
    o = _out_for(out, (q.shape[0], q.shape[1], v_cache.shape[-1]), q.dtype, dev)
    D = _lib.describe
    rc = _lib.load().paged_attention_prefill(
        D(q), D(k_cache), D(v_cache), D(page_block_tables), D(context_lens), D(cu_seqlens), D(o),
        int(max_seqlen), float(scale), _lib.stream_handle(dev),
    )
    _lib.check("paged_attention_prefill", rc)
    return _finish(out, o)

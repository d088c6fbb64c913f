"""CPU restatement of the reference's full-attention ops (test oracle only).

``ops/full_attention.py`` of yuyifanbupt/myvllm (paths relative to
``src/myvllm``), the intended math of its three ops (its kernels' pointer
defects -- K/V read from token 0 of the batch instead of the sequence start
(``:57-72``), the output's dim stride taken from the head stride (``:76``),
``tl.maxmum`` (``:100``), ``tl.load(block_m_indices_ptr * ...)`` and
``tl.load(cu_seqlens_ptr, seq_idx)`` (``:378-380``) -- are not reproduced):

* GQA: query head h reads kv head h // (Hq // Hkv) (``:37``, ``:212``, ``:374``);
* varlen prefill (``:114-173``): per sequence of ``cu_seqlens``,
  o_i = softmax_j(scale q_i . k_j) v_j over the sequence's keys j (j <= i if causal);
* paged decode (``:282-335``): one query per sequence over its first
  ``context_lens[n]`` cached keys, key j at block ``block_tables[n, j // bs]``,
  row ``j % bs`` of the (blocks, bs, Hkv, D) caches;
* paged prefill (``:454-512``): query i of sequence n sits at position
  ``context_lens[n] - seqlen_n + i``, causal over the paged keys (``:393``, ``:401``);
* P is rounded to V's dtype before P V (``:105``, ``:438``); the reference's
  masked score -1e10 and running max start -1e10 (``:93``, ``:97``) give the
  softmax of the unmasked keys.

Computed here in fp64 without the rounding of P; results are returned in fp64.

Test infrastructure only (imported by ``tests/`` and the CPU baseline of
``bench.py``).  Pinning, in ``tests/test_oracle.py``: ``flash_attention_prefill_ref``
equals ``attention_loop_ref`` (scalar loops over heads, queries and keys) for
GQA, causal and not; closed forms (all-equal scores give the running mean of
v, the first token returns its own value); ``paged_attention_ref`` over pages
in permuted order equals the contiguous loop at the positions
``context_len - len + i``; the committed fixtures ``tests/golden/attn_*``
reproduce.  ``attention_loop_ref`` itself is the textbook definition written
as loops.
"""
from __future__ import annotations

import math

import torch


def _attend(q, k, v, scale, pos, causal):
    """q (n, Hq, D); k, v (m, Hkv, D); pos (n,) query positions; keys at 0..m-1."""
    Hq, Hkv = q.shape[1], k.shape[1]
    r = Hq // Hkv
    kq = k.repeat_interleave(r, dim=1)
    vq = v.repeat_interleave(r, dim=1)
    s = torch.einsum("nhd,mhd->hnm", q, kq) * scale
    if causal:
        keep = torch.arange(k.shape[0])[None, :] <= pos[:, None]
        s = s.masked_fill(~keep[None], float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.einsum("hnm,mhd->nhd", p, vq)


def flash_attention_prefill_ref(q, k, v, cu_seqlens, scale, is_causal=True):
    T, Hq, _ = q.shape
    o = torch.zeros(T, Hq, v.shape[2], dtype=torch.float64)
    cu = [int(c) for c in cu_seqlens.tolist()]
    for n in range(len(cu) - 1):
        s, e = cu[n], cu[n + 1]
        if e > s:
            o[s:e] = _attend(q[s:e].double(), k[s:e].double(), v[s:e].double(), scale, torch.arange(e - s), is_causal)
    return o


def attention_rows_ref(q_rows, k_seq, v_seq, pos, scale, causal=True):
    """Selected queries of one sequence: q_rows (n, Hq, D) at positions
    ``pos`` over the sequence's keys k_seq, v_seq (m, Hkv, D), fp64."""
    return _attend(q_rows.double(), k_seq.double(), v_seq.double(), scale, torch.as_tensor(pos), causal)


def gather_paged(cache, table_row, L):
    """Keys 0..L-1 of one sequence from a (blocks, page, Hkv, D) cache."""
    return _gather(cache, table_row, L, cache.shape[1])


def _gather(cache, table_row, L, bs):
    j = torch.arange(L)
    return cache[table_row[j // bs].long(), j % bs]  # (L, Hkv, D)


def paged_attention_ref(q, k_cache, v_cache, block_tables, context_lens, cu_seqlens, scale):
    """Paged prefill (queries of sequence n at positions ctx_n - len_n + i, causal);
    the decode step is the case of one query per sequence."""
    T, Hq, _ = q.shape
    bs = k_cache.shape[1]
    o = torch.zeros(T, Hq, v_cache.shape[3], dtype=torch.float64)
    cu = [int(c) for c in cu_seqlens.tolist()]
    for n in range(len(cu) - 1):
        s, e = cu[n], cu[n + 1]
        L = int(context_lens[n])
        if e <= s or L <= 0:
            continue
        k = _gather(k_cache, block_tables[n], L, bs).double()
        v = _gather(v_cache, block_tables[n], L, bs).double()
        pos = L - (e - s) + torch.arange(e - s)
        o[s:e] = _attend(q[s:e].double(), k, v, scale, pos, True)
    return o


def attention_loop_ref(q, k, v, scale, pos, causal):
    """Brute-force scalar loops (Python floats) for tiny inputs: one sequence,
    q (n, Hq, D), k, v (m, Hkv, D), pos (n,) query positions."""
    n, Hq, D = q.shape
    m, Hkv, Dv = v.shape
    r = Hq // Hkv
    out = torch.zeros(n, Hq, Dv, dtype=torch.float64)
    for i in range(n):
        for h in range(Hq):
            kh = h // r
            keys = [j for j in range(m) if not causal or j <= int(pos[i])]
            sc = [scale * sum(float(q[i, h, d]) * float(k[j, kh, d]) for d in range(D)) for j in keys]
            mx = max(sc)
            w = [math.exp(x - mx) for x in sc]
            z = sum(w)
            for dv in range(Dv):
                out[i, h, dv] = sum(w[t] * float(v[keys[t], kh, dv]) for t in range(len(keys))) / z
    return out

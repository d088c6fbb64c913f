"""CPU restatement of the reference's gated-delta-rule math (test oracle only).

Tensor conventions follow the reference ops (file:line are relative to the
reference package ``src/myvllm``):

* q, k: (T, Hk, K); v: (T, Hv, V); g, beta: (T, Hv)
  (``ops/gated_delta_rule/gated_delta_rule.py:31-40``, ``:69-77``).
* GVA: v-head ``h`` reads k-head ``h // (Hv // Hk)``
  (``ops/gated_delta_rule/fused_recurrent_gdn.py:47``,
  ``ops/gated_delta_rule/chunk_scaled_dot_kkt.py:35``).
* recurrent state cache: (num_slots, Hv, K, V), row-major [k][v] per head,
  indexed by int32 slot ids (``ops/gated_delta_rule/fused_recurrent_gdn.py:46``, ``:51-58``).
* scale = K ** -0.5 (``ops/gated_delta_rule/gated_delta_rule.py:46``,
  ``ops/gated_delta_rule/fused_recurrent_gdn.py:117``).
* g is a per-token natural-log decay; the reference rescales its cumsum by
  1/ln 2 and uses exp2 (``ops/gated_delta_rule/gated_delta_rule.py:12``, ``:48``,
  ``ops/gated_delta_rule/cumsum.py:39``) -- identical math, natural log here.

Semantics that deliberately differ from the reference's (defective) kernels:
the prefill reads the initial state from ``state[slot]`` (the reference starts
from zero, ``ops/gated_delta_rule/h.py:61-67``), the chunk is 64 (reference 32,
``ops/gated_delta_rule/gated_delta_rule.py:44``), and all intermediates are kept
at the compute dtype instead of bf16 (``ops/gated_delta_rule/wu.py:150``,
``ops/gated_delta_rule/h.py:162``, ``:213``).  Slots outside ``[0, num_slots)`` mark a
sequence as padding: its output is zero and no state is touched.
"""
from __future__ import annotations

import torch


def _heads_expand(x: torch.Tensor, r: int) -> torch.Tensor:
    """k-head tensor (T, Hk, K) -> per-v-head view (T, Hv, K) with v-head h -> k-head h // r."""
    return x.repeat_interleave(r, dim=1)


def recurrent_gated_delta_rule_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    recurrent_state: torch.Tensor,
    recurrent_state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor | None = None,
    scale: float | None = None,
    dtype: torch.dtype = torch.float64,
) -> torch.Tensor:
    """Token-by-token gated delta rule over packed sequences.

    Follows ``ops/gated_delta_rule/fused_recurrent_gdn.py:49`` (decay e^g),
    ``:96`` (S <- e^g S), ``:97`` (delta = beta (v - S^T k)), ``:98`` (S += k delta^T),
    ``:68``/``:99`` (o = S^T (scale q), after the update) and ``:101`` (state stored
    back in place).  With ``cu_seqlens=None`` every row is its own sequence
    (the decode step: one token per sequence, ``gated_delta_rule.py:69-92``).

    Mutates ``recurrent_state`` at the indexed slots (in its own dtype) and
    returns o (T, Hv, V) in v's dtype.
    """
    T, Hk, K = q.shape
    Hv, V = v.shape[1], v.shape[2]
    r = Hv // Hk
    if scale is None:
        scale = K ** -0.5
    if cu_seqlens is None:
        cu = list(range(T + 1))
    else:
        cu = [int(x) for x in cu_seqlens.tolist()]
    num_slots = recurrent_state.shape[0]
    qf = _heads_expand(q.to(dtype), r) * scale
    kf = _heads_expand(k.to(dtype), r)
    vf = v.to(dtype)
    gf = g.to(dtype)
    bf = beta.to(dtype)
    o = torch.zeros(T, Hv, V, dtype=dtype)
    idx = [int(x) for x in recurrent_state_indices.tolist()]
    for n in range(len(cu) - 1):
        slot = idx[n]
        if slot < 0 or slot >= num_slots:
            continue
        S = recurrent_state[slot].to(dtype).clone()  # (Hv, K, V)
        for t in range(cu[n], cu[n + 1]):
            S = S * torch.exp(gf[t])[:, None, None]
            kS = torch.einsum("hk,hkv->hv", kf[t], S)
            delta = bf[t][:, None] * (vf[t] - kS)
            S = S + kf[t][:, :, None] * delta[:, None, :]
            o[t] = torch.einsum("hk,hkv->hv", qf[t], S)
        if cu[n + 1] > cu[n]:
            recurrent_state[slot] = S.to(recurrent_state.dtype)
    return o.to(v.dtype)


def tril_inverse_ref(A: torch.Tensor) -> torch.Tensor:
    """(I + A)^-1 for strictly-lower A (..., C, C).

    Follows the contract of ``ops/gated_delta_rule/solve_tril.py:81-96``
    (docstring) -- computed here by forward substitution row by row, so that
    tests can pin it against ``torch.linalg.solve_triangular``.
    """
    C = A.shape[-1]
    Tm = torch.zeros_like(A)
    eye = torch.eye(C, dtype=A.dtype)
    for i in range(C):
        # row i of T: e_i - sum_{j<i} A[i, j] T[j, :]
        Tm[..., i, :] = eye[i] - torch.einsum("...j,...jc->...c", A[..., i, :i], Tm[..., :i, :])
    return Tm


def chunk_gated_delta_rule_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    recurrent_state: torch.Tensor,
    recurrent_state_indices: torch.Tensor,
    cu_seqlens: torch.Tensor,
    chunk_size: int = 64,
    scale: float | None = None,
    dtype: torch.dtype = torch.float64,
    use_library_solve: bool = True,
) -> torch.Tensor:
    """Chunked (UT/WY) gated delta rule prefill over packed varlen sequences.

    Per sequence (``cu_seqlens``) and chunk of L <= C tokens, per v-head:

    * gamma = in-chunk inclusive cumsum of g (``ops/gated_delta_rule/cumsum.py:37-39``);
    * A = strict-lower[beta_i k_i.k_j exp(gamma_i - gamma_j)]
      (``ops/gated_delta_rule/chunk_scaled_dot_kkt.py:50-84``);
    * Tm = (I + A)^-1 (``ops/gated_delta_rule/solve_tril.py:6-73``);
    * W = Tm diag(beta e^gamma) K, U = Tm diag(beta) V (``ops/gated_delta_rule/wu.py:90-133``);
    * V' = U - W S (``ops/gated_delta_rule/h.py:129-145``);
    * O = scale [diag(e^gamma) Q S + (tril0(Q K^T) * e^(gamma_i - gamma_j)) V']
      (``ops/gated_delta_rule/o.py:81-121``);
    * S <- e^gamma_last S + K^T diag(e^(gamma_last - gamma)) V' (``ops/gated_delta_rule/h.py:147-175``);
    * final S written to ``recurrent_state[slot]`` (``ops/gated_delta_rule/h.py:177-192``).

    The initial S is read from ``recurrent_state[slot]``.  All chunks of a
    sequence are formed at once (batched intra-chunk math); only the state
    propagation walks the chunks in order.  Mutates the indexed slots of
    ``recurrent_state`` and returns o (T, Hv, V) in v's dtype.
    """
    T, Hk, K = q.shape
    Hv, V = v.shape[1], v.shape[2]
    r = Hv // Hk
    C = chunk_size
    if scale is None:
        scale = K ** -0.5
    cu = [int(x) for x in cu_seqlens.tolist()]
    idx = [int(x) for x in recurrent_state_indices.tolist()]
    num_slots = recurrent_state.shape[0]
    o = torch.zeros(T, Hv, V, dtype=dtype)
    strict = torch.tril(torch.ones(C, C, dtype=torch.bool), diagonal=-1)
    causal = torch.tril(torch.ones(C, C, dtype=torch.bool), diagonal=0)
    for n in range(len(cu) - 1):
        s, e = cu[n], cu[n + 1]
        slot = idx[n]
        if e <= s or slot < 0 or slot >= num_slots:
            continue
        L = e - s
        nc = (L + C - 1) // C
        pad = nc * C - L

        def blocks(x: torch.Tensor) -> torch.Tensor:
            # (L, H, D) -> (H, nc, C, D) zero-padded
            x = x.to(dtype)
            if pad:
                x = torch.cat([x, x.new_zeros((pad,) + tuple(x.shape[1:]))], 0)
            return x.reshape((nc, C) + tuple(x.shape[1:])).movedim(2, 0)

        Qb = blocks(_heads_expand(q[s:e], r))  # (Hv, nc, C, K)
        Kb = blocks(_heads_expand(k[s:e], r))
        Vb = blocks(v[s:e])  # (Hv, nc, C, V)
        gb = g[s:e].to(dtype)
        bb = beta[s:e].to(dtype)
        if pad:
            gb = torch.cat([gb, gb.new_zeros(pad, Hv)], 0)
            bb = torch.cat([bb, bb.new_zeros(pad, Hv)], 0)
        gam = gb.reshape(nc, C, Hv).permute(2, 0, 1).cumsum(-1)  # (Hv, nc, C)
        bet = bb.reshape(nc, C, Hv).permute(2, 0, 1)

        diff = gam[..., :, None] - gam[..., None, :]
        dec_strict = torch.exp(torch.where(strict, diff, torch.full_like(diff, float("-inf"))))
        dec_causal = torch.exp(torch.where(causal, diff, torch.full_like(diff, float("-inf"))))
        A = bet[..., :, None] * (Kb @ Kb.transpose(-1, -2)) * dec_strict
        if use_library_solve:
            eye = torch.eye(C, dtype=dtype).expand_as(A)
            Tm = torch.linalg.solve_triangular(eye + A, eye, upper=False, unitriangular=True)
        else:
            Tm = tril_inverse_ref(A)
        eg = torch.exp(gam)
        Wm = Tm @ ((bet * eg)[..., None] * Kb)  # (Hv, nc, C, K)
        Um = Tm @ (bet[..., None] * Vb)  # (Hv, nc, C, V)
        P = (Qb @ Kb.transpose(-1, -2)) * dec_causal  # (Hv, nc, C, C)
        last = gam[..., -1]  # (Hv, nc): padded g is 0 so this is gamma at the last real token
        dlast = torch.exp(last[..., None] - gam)  # (Hv, nc, C)

        S = recurrent_state[slot].to(dtype).clone()  # (Hv, K, V)
        Ob = torch.empty(Hv, nc, C, V, dtype=dtype)
        for c in range(nc):
            Vn = Um[:, c] - Wm[:, c] @ S
            Ob[:, c] = scale * (eg[:, c, :, None] * (Qb[:, c] @ S) + P[:, c] @ Vn)
            S = torch.exp(last[:, c])[:, None, None] * S + Kb[:, c].transpose(-1, -2) @ (dlast[:, c, :, None] * Vn)
        o[s:e] = Ob.reshape(Hv, nc * C, V)[:, :L].transpose(0, 1)
        recurrent_state[slot] = S.to(recurrent_state.dtype)
    return o.to(v.dtype)


def chunk_gated_delta_rule_fla_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    g: torch.Tensor,
    beta: torch.Tensor,
    cu_seqlens: torch.Tensor,
    initial_state: torch.Tensor | None = None,
    output_final_state: bool = False,
    chunk_size: int = 64,
    scale: float | None = None,
    dtype: torch.dtype = torch.float64,
):
    """Functional form: initial_state (N, Hv, K, V) in, (o, final_state) out.

    Runs :func:`chunk_gated_delta_rule_ref` over a temporary cache with slot n
    for sequence n (the same state-in/state-out contract).
    """
    N = cu_seqlens.numel() - 1
    Hv, V = v.shape[1], v.shape[2]
    K = k.shape[2]
    if initial_state is None:
        cache = torch.zeros(N, Hv, K, V, dtype=torch.float32)
    else:
        cache = initial_state.clone()
    o = chunk_gated_delta_rule_ref(
        q, k, v, g, beta, cache, torch.arange(N, dtype=torch.int32), cu_seqlens, chunk_size, scale, dtype
    )
    return o, (cache if output_final_state else None)

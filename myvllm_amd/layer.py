"""The Gated DeltaNet layer around the hot path, on one MI355X.

Replaces ``GatedDeltaNet`` (``layers/linear_attention.py:15-124`` of
yuyifanbupt/myvllm) with the intended dataflow of its ``forward`` (the
reference convolves ``x`` instead of the qkv projection, norms with the
wrong shapes and projects ``z``, ``:93``, ``:95``, ``:121-122``):

  qkv | z = x W_qkvz^T ;  b | a = x W_ba^T                      (:85-88)
  g = -exp(A_log) softplus(a + dt_bias),  beta = sigmoid(b)     (:89-90)
  prefill tokens: y = causal_conv1d(qkv) with the per-head L2 norm of q, k
                  fused into its epilogue (:93, :97-114), then
                  o = chunk_gated_delta_rule(q, k, v, g, beta)   (:117)
  decode tokens:  o = gated_delta_net_decode_step(qkv, a, b)     (:95-119 in one launch)
  o = RMSNormGated(o, z) per v-head                              (:121)
  out = o W_out^T                                                (:122)

The four input projections are one GEMM (rows q|k|v|z|b|a; measured faster
than separate q|k|v|z and b|a GEMMs on this device) and every GEMM is
torch's (hipBLASLt); the gates are one small kernel.  One call takes a mixed batch: the prefill
sequences' tokens first (``cu_seqlens`` covers them), then
``num_decode_tokens`` decode tokens, one per sequence, whose slot ids follow
the prefill ones in the index tensors (the reference takes one
``is_prefill`` flag per call, ``:83``, ``:92``, ``:116``).  In a mixed batch
the decode step runs on a second stream (default priority) beside the chunked
prefill: the two touch disjoint cache slots, and the prefill, one workgroup
per (sequence, v-head) bound by its per-chunk chain, leaves CUs idle when a
batch has fewer such items than the GPU has CUs (128 on 4 x 2048 tokens,
Hv 32), which the HBM-bound decode step fills (886 -> 780 us per layer step
on that batch with 128 decode tokens; results bit-identical to the serial
order).  Single GPU: the tensor-parallel head split (``:28-38``) is one GPU's
share.
"""
from __future__ import annotations

import math

import torch
from torch import nn

from .causal_conv1d import causal_conv1d_fn
from .gated_delta_rule import chunk_gated_delta_rule, gated_delta_net_decode_step
from .norm import gdn_gating, rms_norm_gated

_side_streams: dict[int, torch.cuda.Stream] = {}


def _side_stream(dev: torch.device) -> torch.cuda.Stream:
    """A second stream per device, at the default priority, for the decode step."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    st = _side_streams.get(idx)
    if st is None:
        st = _side_streams[idx] = torch.cuda.Stream(device=idx)
    return st


class GatedDeltaNet(nn.Module):
    def __init__(
        self,
        hidden_size: int,
        num_k_heads: int,
        num_v_heads: int,
        k_head_dim: int,
        v_head_dim: int,
        conv_kernel_size: int = 4,
        rms_norm_eps: float = 1e-6,
        dtype: torch.dtype = torch.bfloat16,
        device: torch.device | str | None = None,
    ) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.num_k_heads = num_k_heads
        self.num_v_heads = num_v_heads
        self.k_head_dim = k_head_dim
        self.v_head_dim = v_head_dim
        self.conv_kernel_size = conv_kernel_size
        self.rms_norm_eps = rms_norm_eps
        self.k_size = num_k_heads * k_head_dim
        self.v_size = num_v_heads * v_head_dim
        self.conv_dim = 2 * self.k_size + self.v_size
        kw = dict(dtype=dtype, device=device)
        # rows: q | k | v | z | b | a
        self.in_proj = nn.Parameter(torch.empty(self.conv_dim + self.v_size + 2 * num_v_heads, hidden_size, **kw))
        self.conv1d_weight = nn.Parameter(torch.empty(self.conv_dim, conv_kernel_size, **kw))
        self.dt_bias = nn.Parameter(torch.ones(num_v_heads, device=device))
        self.A_log = nn.Parameter(torch.log(torch.empty(num_v_heads, device=device).uniform_(1, 16)))
        self.norm_weight = nn.Parameter(torch.ones(v_head_dim, device=device))
        self.out_proj = nn.Parameter(torch.empty(hidden_size, self.v_size, **kw))
        # caches of this layer (views of a LinearAttentionCache), set by the caller as in the reference (:74-75)
        self.conv_state: torch.Tensor = torch.empty(0)
        self.recurrent_state: torch.Tensor = torch.empty(0)

    @torch.no_grad()
    def init_random(self, std: float = 0.02, seed: int = 0) -> None:
        """Random-init weights ~N(0, std) (conv taps ~N(0, 1/W)), seeded on the CPU."""
        gen = torch.Generator().manual_seed(seed)
        for p, s in ((self.in_proj, std), (self.out_proj, std),
                     (self.conv1d_weight, 1.0 / math.sqrt(self.conv_kernel_size))):
            p.copy_((torch.randn(p.shape, generator=gen) * s).to(p.dtype))

    @staticmethod
    def _decode_count(T: int, is_prefill, num_decode_tokens) -> int:
        """Decode tokens of the call from the reference's ``is_prefill`` flag or
        the mixed-batch ``num_decode_tokens`` (not both, unless they agree)."""
        if is_prefill is not None and not isinstance(is_prefill, bool):
            raise TypeError(f"is_prefill must be a bool (got {type(is_prefill).__name__}); "
                            "pass num_decode_tokens= for a mixed batch")
        if num_decode_tokens is not None and (isinstance(num_decode_tokens, bool) or
                                              not isinstance(num_decode_tokens, int)):
            raise TypeError(f"num_decode_tokens must be an int (got {type(num_decode_tokens).__name__})")
        if is_prefill is None:
            n = 0 if num_decode_tokens is None else num_decode_tokens
        else:
            n = 0 if is_prefill else T
            if num_decode_tokens is not None and num_decode_tokens != n:
                raise ValueError(f"is_prefill={is_prefill} disagrees with num_decode_tokens={num_decode_tokens}")
        if T >= 0 and not 0 <= n <= T:
            raise ValueError(f"num_decode_tokens={n} outside [0, {T}]")
        return n

    def _check_inputs(self, x, cu_seqlens, conv_state_indices, recurrent_state_indices, Tp: int, Td: int) -> int:
        """Shapes, dtypes and devices of one call; returns the number of prefill sequences."""
        if x.dim() != 2 or x.shape[1] != self.hidden_size:
            raise ValueError(f"x must be (T, {self.hidden_size}), got {tuple(x.shape)}")
        dev = x.device
        idx_types = (torch.int32, torch.int64)
        Np = 0
        if Tp > 0:
            if not isinstance(cu_seqlens, torch.Tensor) or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
                raise ValueError("cu_seqlens must be a 1-D tensor of N_prefill + 1 >= 2 offsets")
            if cu_seqlens.dtype not in idx_types or cu_seqlens.device != dev:
                raise ValueError(f"cu_seqlens must be int32/int64 on {dev} (got {cu_seqlens.dtype} on "
                                 f"{cu_seqlens.device})")
            Np = cu_seqlens.numel() - 1
        for name, t in (("conv_state_indices", conv_state_indices), ("recurrent_state_indices", recurrent_state_indices)):
            if not isinstance(t, torch.Tensor) or t.dim() != 1 or t.dtype not in idx_types or t.device != dev:
                raise ValueError(f"{name} must be a 1-D int32/int64 tensor on {dev}")
            if t.numel() != Np + Td:
                raise ValueError(f"{name} has {t.numel()} entries; the call has {Np} prefill sequences and "
                                 f"{Td} decode tokens")
        cs, rs = self.conv_state, self.recurrent_state
        if rs.dim() != 4 or tuple(rs.shape[1:]) != (self.num_v_heads, self.k_head_dim, self.v_head_dim) or \
                rs.dtype != torch.float32 or rs.device != dev:
            raise ValueError(f"recurrent_state must be (slots, {self.num_v_heads}, {self.k_head_dim}, "
                             f"{self.v_head_dim}) fp32 on {dev}; got {tuple(rs.shape)} {rs.dtype}")
        if cs.dim() != 3 or tuple(cs.shape[1:]) != (self.conv_kernel_size - 1, self.conv_dim) or cs.device != dev:
            raise ValueError(f"conv_state must be (slots, {self.conv_kernel_size - 1}, {self.conv_dim}) on {dev}; "
                             f"got {tuple(cs.shape)}")
        if Td > 0 and (self.conv_kernel_size != 4 or self.k_head_dim != 128 or self.v_head_dim != 128 or
                       self.num_v_heads // self.num_k_heads not in (1, 2, 4)):
            raise ValueError("decode tokens need conv width 4, K = V = 128 and Hv / Hk in {1, 2, 4} "
                             "(the fused decode step)")
        return Np

    def forward(
        self,
        x: torch.Tensor,  # (T, hidden)
        cu_seqlens: torch.Tensor,  # (N_prefill + 1,) over the first T - num_decode_tokens tokens
        conv_state_indices: torch.Tensor,  # (N_prefill + num_decode_tokens,)
        recurrent_state_indices: torch.Tensor,  # (N_prefill + num_decode_tokens,)
        is_prefill: bool | None = None,
        *,
        num_decode_tokens: int | None = None,
    ) -> torch.Tensor:
        """One layer step.  The reference's call form ``forward(x, cu_seqlens,
        conv_state_indices, recurrent_state_indices, is_prefill)``
        (``layers/linear_attention.py:77-84``) is accepted as is: ``is_prefill``
        True makes every token a prefill token, False makes every token one
        decode step of its own sequence (``cu_seqlens`` is then not read).  A
        mixed batch passes ``num_decode_tokens`` instead: the prefill tokens
        first, then that many decode tokens.  Every argument is checked before
        anything is launched, so a malformed call raises with both caches
        untouched.  (``cu_seqlens[-1]`` is a device value and is not compared
        with the prefill token count, which would synchronise the host; the
        kernels clamp sequences to it and zero the rows no sequence covers.)"""
        T = x.shape[0] if x.dim() == 2 else -1
        num_decode_tokens = self._decode_count(T, is_prefill, num_decode_tokens)
        Tp = T - num_decode_tokens
        Np = self._check_inputs(x, cu_seqlens, conv_state_indices, recurrent_state_indices, Tp, num_decode_tokens)
        Hk, Hv, K, V = self.num_k_heads, self.num_v_heads, self.k_head_dim, self.v_head_dim
        proj = x @ self.in_proj.t()
        cz = self.conv_dim + self.v_size
        qkv, z = proj[:, : self.conv_dim], proj[:, self.conv_dim: cz]
        b, a = proj[:, cz: cz + Hv], proj[:, cz + Hv:]
        o = torch.empty(T, Hv, V, dtype=x.dtype, device=x.device)

        def decode_step() -> None:
            gated_delta_net_decode_step(
                qkv[Tp:], self.conv1d_weight, self.conv_state, conv_state_indices[Np:], a[Tp:], b[Tp:], self.A_log,
                self.dt_bias, self.recurrent_state, recurrent_state_indices[Np:], Hk, out=o[Tp:])

        side = None
        if Tp > 0:
            y = causal_conv1d_fn(qkv[:Tp], self.conv1d_weight, self.conv_state, conv_state_indices[:Np], cu_seqlens,
                                 l2norm_channels=2 * self.k_size)
            q = y[:, : self.k_size].view(Tp, Hk, K)
            k = y[:, self.k_size: 2 * self.k_size].view(Tp, Hk, K)
            v = y[:, 2 * self.k_size:].view(Tp, Hv, V)
            g, beta = gdn_gating(a[:Tp], b[:Tp], self.A_log, self.dt_bias)
            if num_decode_tokens > 0 and x.is_cuda:
                # the decode step starts with the prefill launch and overlaps it;
                # every tensor it touches stays referenced until the join below,
                # and the caching allocator only reuses their memory for work
                # ordered after the join on this stream
                main = torch.cuda.current_stream(x.device)
                side = _side_stream(x.device)
                side.wait_stream(main)
            chunk_gated_delta_rule(q, k, v, g, beta, self.recurrent_state, recurrent_state_indices[:Np], cu_seqlens,
                                   out=o[:Tp])
        if num_decode_tokens > 0:
            if side is not None:
                with torch.cuda.stream(side):
                    decode_step()
                main.wait_stream(side)
            else:
                decode_step()
        on = rms_norm_gated(o, z.view(T, Hv, V), self.norm_weight, self.rms_norm_eps)
        return on.view(T, self.v_size) @ self.out_proj.t()

"""State caches of the GDN layers, in the layout the kernels read.

Replaces ``LinearAttentionCache`` (``cache/linear_attention_cache.py:7-88`` of
yuyifanbupt/myvllm) with the same constructor arguments, slot allocator and
zero-on-free semantics, and these corrections:

* the recurrent (SSM) cache holds ``num_v_heads`` heads, the heads the
  kernels index (the reference sizes it with ``num_k_heads``, ``:37-45``);
* the recurrent state is fp32 (``state_dtype``), whatever the activations'
  dtype (the reference uses the model dtype for both caches, ``:27``);
* the conv cache has its own dtype (``conv_dtype``, default the model dtype);
* freeing a slot zeroes it in every layer with one device fill per cache
  (the reference issues two fills per layer, ``:83-85``).

Layouts: conv cache ``(layers, slots, W-1, D)`` with ``D = 2 K Hk + V Hv``
channels q | k | v, token-major, oldest row first; recurrent cache
``(layers, slots, Hv, K, V)`` with ``[K][V]`` contiguous per head.  A layer's
views (``layer(l)``) are what ``causal_conv1d_fn`` / ``causal_conv1d_update`` /
``chunk_gated_delta_rule`` / ``recurrent_gated_delta_rule`` /
``gated_delta_net_decode_step`` take, indexed by the allocated slot ids.
"""
from __future__ import annotations

from collections import deque

import torch


class LinearAttentionCache:
    def __init__(
        self,
        layer_cnt: int,
        max_seq_cnt: int,
        conv_kernel_size: int,
        k_head_dim: int,
        v_head_dim: int,
        num_k_heads: int,
        num_v_heads: int,
        dtype: torch.dtype,
        device: torch.device,
        state_dtype: torch.dtype = torch.float32,
        conv_dtype: torch.dtype | None = None,
    ) -> None:
        if num_k_heads <= 0 or num_v_heads % num_k_heads != 0:
            raise ValueError("num_v_heads must be a positive multiple of num_k_heads")
        self.layer_cnt = layer_cnt
        self.max_seq_cnt = max_seq_cnt
        self.conv_kernel_size = conv_kernel_size
        self.k_head_dim = k_head_dim
        self.v_head_dim = v_head_dim
        self.num_k_heads = num_k_heads
        self.num_v_heads = num_v_heads
        self.dtype = dtype
        self.state_dtype = state_dtype
        self.conv_dtype = conv_dtype or dtype
        self.device = device
        self.conv_dim = 2 * k_head_dim * num_k_heads + v_head_dim * num_v_heads
        self.conv_cache = torch.zeros(
            layer_cnt, max_seq_cnt, conv_kernel_size - 1, self.conv_dim, dtype=self.conv_dtype, device=device
        )
        self.recurrent_cache = torch.zeros(
            layer_cnt, max_seq_cnt, num_v_heads, k_head_dim, v_head_dim, dtype=state_dtype, device=device
        )
        self.free_slot_ids: deque[int] = deque(range(max_seq_cnt))
        self.used_slot_ids: set[int] = set()

    @staticmethod
    def bytes_per_seq(
        layer_cnt: int,
        conv_kernel_size: int,
        k_head_dim: int,
        v_head_dim: int,
        num_k_heads: int,
        num_v_heads: int,
        dtype: torch.dtype,
        state_dtype: torch.dtype = torch.float32,
        conv_dtype: torch.dtype | None = None,
    ) -> int:
        """Cache bytes one sequence slot takes over all layers."""
        conv_dtype = conv_dtype or dtype
        conv = layer_cnt * (conv_kernel_size - 1) * (2 * k_head_dim * num_k_heads + v_head_dim * num_v_heads)
        recurrent = layer_cnt * num_v_heads * k_head_dim * v_head_dim
        return conv * conv_dtype.itemsize + recurrent * state_dtype.itemsize

    def layer(self, layer_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        """(conv_state (slots, W-1, D), recurrent_state (slots, Hv, K, V)) views of one layer."""
        return self.conv_cache[layer_idx], self.recurrent_cache[layer_idx]

    def can_allocate(self) -> bool:
        return len(self.free_slot_ids) > 0

    def allocate(self) -> int:
        if not self.free_slot_ids:
            raise RuntimeError("no free cache slot")
        slot_id = self.free_slot_ids.popleft()
        self.used_slot_ids.add(slot_id)
        return slot_id

    def deallocate(self, slot_id: int) -> None:
        self.deallocate_many([slot_id])

    def deallocate_many(self, slot_ids) -> None:
        """Free slots (zeroed in every layer; later frees are reused first, as
        one ``deallocate`` after another in the reference)."""
        slot_ids = [int(s) for s in slot_ids]
        for s in slot_ids:
            if s not in self.used_slot_ids:
                raise ValueError(f"slot {s} is not allocated")
        if len(set(slot_ids)) != len(slot_ids):
            raise ValueError("slot ids repeat")
        if slot_ids:
            idx = torch.tensor(slot_ids, dtype=torch.long, device=self.device)
            self.conv_cache.index_fill_(1, idx, 0)
            self.recurrent_cache.index_fill_(1, idx, 0)
        for s in slot_ids:
            self.used_slot_ids.remove(s)
            self.free_slot_ids.appendleft(s)

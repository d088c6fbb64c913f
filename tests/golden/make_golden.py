#!/usr/bin/env python3
"""Writes the golden fixtures of this directory from the CPU oracle (fp64).

The reference (yuyifanbupt/myvllm) ships no tests, fixtures or golden vectors
and cannot run its Triton kernels without a GPU, so these vectors come from
the oracle, which is itself pinned by closed forms and independent
algorithms in tests/test_oracle.py.  They freeze the oracle's answers so a
later change to it (or a GPU kernel) is checked against fixed data.

Fixtures (safetensors, all tensors stored as written below):
* gdn_recurrent_64tok.safetensors: one sequence of 64 tokens, Hk 16 / Hv 32,
  d 128, all fp32, zero initial state (the CPU reference-plumbing case);
  token recurrence.
* gdn_chunk_varlen_small.safetensors: lengths [0, 5, 64, 70, 1], Hk 1 / Hv 2,
  bf16 q/k/v, fp32 g/beta, fp32 initial state in 5 slots.
* gdn_decode_small.safetensors: batch 3 from a 4-slot cache, Hk 1 / Hv 2.
* conv_varlen_small.safetensors / conv_update_small.safetensors: 64 channels,
  width 4, lengths [3, 1, 10, 0, 7] / batch 5.
* attn_varlen_small.safetensors: causal varlen attention, lengths [1, 17, 40],
  Hq 4 / Hkv 2, d 64, bf16 inputs, fp32 output.
* attn_paged_small.safetensors: paged prefill (contexts [20, 7, 33], new
  [3, 7, 1], 8-token pages) and paged decode (contexts [20, 1, 40]) over one
  cache, Hq 4 / Hkv 2, d 64, bf16 inputs, fp32 outputs.

Run from the repository root: python tests/golden/make_golden.py [name ...]
"""
from __future__ import annotations

import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from myvllm_amd.workloads import (  # noqa: E402
    attn_varlen_case,
    conv_decode_case,
    conv_prefill_case,
    cu_from_lengths,
    decode_case,
    gdn_inputs,
    paged_case,
    prefill_case,
)
from oracle.attention import flash_attention_prefill_ref, paged_attention_ref  # noqa: E402
from oracle.conv import causal_conv1d_fn_ref, causal_conv1d_update_ref  # noqa: E402
from oracle.gdn import chunk_gated_delta_rule_ref, recurrent_gated_delta_rule_ref  # noqa: E402


def recurrent_64tok():
    gen = torch.Generator().manual_seed(0)
    q, k, v, g, beta = gdn_inputs(gen, 64, 16, 32, 128, 128, dtype=torch.float32)
    state = torch.zeros(1, 32, 128, 128)
    idx = torch.zeros(1, dtype=torch.int32)
    cu = torch.tensor([0, 64], dtype=torch.int32)
    o = recurrent_gated_delta_rule_ref(q, k, v, g, beta, state, idx, cu, dtype=torch.float64)
    return {"q": q, "k": k, "v": v, "g": g, "beta": beta, "cu_seqlens": cu, "state_indices": idx,
            "o": o.contiguous(), "final_state": state[0].contiguous()}


def chunk_varlen_small():
    c = prefill_case([0, 5, 64, 70, 1], seed=3, num_slots=5, Hk=1, Hv=2)
    st = c.state.clone()
    o = chunk_gated_delta_rule_ref(c.q, c.k, c.v, c.g, c.beta, st, c.idx, c.cu, dtype=torch.float64)
    return {"q": c.q, "k": c.k, "v": c.v, "g": c.g, "beta": c.beta, "initial_state": c.state,
            "state_indices": c.idx, "cu_seqlens": c.cu, "o": o.float().contiguous(), "final_state": st}


def decode_small():
    c = decode_case(B=3, num_slots=4, seed=5, Hk=1, Hv=2)
    st = c.state.clone()
    o = recurrent_gated_delta_rule_ref(c.q, c.k, c.v, c.g, c.beta, st, c.idx, dtype=torch.float64)
    return {"q": c.q, "k": c.k, "v": c.v, "g": c.g, "beta": c.beta, "initial_state": c.state,
            "state_indices": c.idx, "o": o.float().contiguous(), "final_state": st}


def conv_varlen_small():
    c = conv_prefill_case([3, 1, 10, 0, 7], seed=4, D=64, W=4, num_slots=8)
    st = c.state.clone()
    y = causal_conv1d_fn_ref(c.x, c.weight, st, c.idx, c.cu)
    return {"x": c.x, "weight": c.weight, "initial_state": c.state, "state_indices": c.idx, "cu_seqlens": c.cu,
            "y": y.float().contiguous(), "final_state": st}


def conv_update_small():
    c = conv_decode_case(B=5, seed=6, D=64, W=4, num_slots=8)
    st = c.state.clone()
    y = causal_conv1d_update_ref(c.x, c.weight, st, c.idx)
    return {"x": c.x, "weight": c.weight, "initial_state": c.state, "state_indices": c.idx,
            "y": y.float().contiguous(), "final_state": st}


def attn_varlen_small():
    c = attn_varlen_case([1, 17, 40], seed=8, Hq=4, Hkv=2, D=64)
    o = flash_attention_prefill_ref(c.q, c.k, c.v, c.cu, c.scale, is_causal=True)
    return {"q": c.q, "k": c.k, "v": c.v, "cu_seqlens": c.cu, "scale": torch.tensor([c.scale]),
            "o": o.float().contiguous()}


def attn_paged_small():
    c = paged_case([20, 7, 33], [3, 7, 1], page=8, seed=9, Hq=4, Hkv=2, D=64)
    o = paged_attention_ref(c.q, c.k_cache, c.v_cache, c.block_tables, c.context_lens, c.cu, c.scale)
    # decode over the same cache: one query per sequence at position ctx - 1
    dctx = torch.tensor([20, 1, 40], dtype=torch.int32)
    dq = torch.randn(3, 4, 64, generator=torch.Generator().manual_seed(10)).to(torch.bfloat16)
    # (sequence 2's five pages hold 40 keys: the 33 of the prefill and 7 more cache rows)
    od = paged_attention_ref(dq, c.k_cache, c.v_cache, c.block_tables, dctx, cu_from_lengths([1, 1, 1]), c.scale)
    return {"q": c.q, "k_cache": c.k_cache, "v_cache": c.v_cache, "block_tables": c.block_tables,
            "context_lens": c.context_lens, "cu_seqlens": c.cu, "scale": torch.tensor([c.scale]),
            "o": o.float().contiguous(), "decode_q": dq, "decode_context_lens": dctx,
            "decode_o": od.float().contiguous()}


FIXTURES = {
    "gdn_recurrent_64tok": recurrent_64tok,
    "gdn_chunk_varlen_small": chunk_varlen_small,
    "gdn_decode_small": decode_small,
    "conv_varlen_small": conv_varlen_small,
    "conv_update_small": conv_update_small,
    "attn_varlen_small": attn_varlen_small,
    "attn_paged_small": attn_paged_small,
}


def main():
    names = sys.argv[1:] or list(FIXTURES)
    for name in names:
        fn = FIXTURES[name]
        tensors = {k: v.contiguous() for k, v in fn().items()}
        path = os.path.join(HERE, name + ".safetensors")
        save_file(tensors, path)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()

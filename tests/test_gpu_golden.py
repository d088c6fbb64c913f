"""GPU parity against the committed golden fixtures (tests/golden)."""
import os

import pytest
import torch
from safetensors.torch import load_file

from conftest import assert_out_close, assert_state_close
from myvllm_amd import (causal_conv1d_fn, causal_conv1d_update, chunk_gated_delta_rule, flash_attention_prefill,
                        paged_flash_attention_decode, paged_flash_attention_prefill, recurrent_gated_delta_rule)

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name, dev):
    return {k: v.to(dev) for k, v in load_file(os.path.join(GOLDEN, name + ".safetensors")).items()}


def test_golden_recurrent_64tok_fp32_token_by_token(dev):
    """All-fp32 64-token sequence (Hk 16 / Hv 32) through the fp32 decode kernel, one token per call."""
    f = _load("gdn_recurrent_64tok", dev)
    st = torch.zeros(1, 32, 128, 128, device=dev)
    idx = f["state_indices"]
    outs = [recurrent_gated_delta_rule(f["q"][t:t + 1], f["k"][t:t + 1], f["v"][t:t + 1], f["g"][t:t + 1],
                                       f["beta"][t:t + 1], st, idx) for t in range(64)]
    o = torch.cat(outs)
    assert o.dtype == torch.float32
    assert_out_close(o, f["o"], rtol=1e-4, atol=1e-5)
    assert_state_close(st[0], f["final_state"])


def test_golden_chunk_varlen_small(dev):
    f = _load("gdn_chunk_varlen_small", dev)
    st = f["initial_state"].clone()
    o = chunk_gated_delta_rule(f["q"], f["k"], f["v"], f["g"], f["beta"], st, f["state_indices"], f["cu_seqlens"])
    assert_out_close(o, f["o"])
    assert_state_close(st, f["final_state"])


def test_golden_decode_small(dev):
    f = _load("gdn_decode_small", dev)
    st = f["initial_state"].clone()
    o = recurrent_gated_delta_rule(f["q"], f["k"], f["v"], f["g"], f["beta"], st, f["state_indices"])
    assert_out_close(o, f["o"])
    assert_state_close(st, f["final_state"])


def test_golden_conv(dev):
    f = _load("conv_varlen_small", dev)
    st = f["initial_state"].clone()
    y = causal_conv1d_fn(f["x"], f["weight"], st, f["state_indices"], f["cu_seqlens"])
    assert_out_close(y, f["y"])
    assert torch.equal(st, f["final_state"])
    f = _load("conv_update_small", dev)
    st = f["initial_state"].clone()
    y = causal_conv1d_update(f["x"], f["weight"], st, f["state_indices"])
    assert_out_close(y, f["y"])
    assert torch.equal(st, f["final_state"])


def test_golden_attention(dev):
    f = _load("attn_varlen_small", dev)
    o = flash_attention_prefill(f["q"], f["k"], f["v"], f["cu_seqlens"], float(f["scale"]), 4, 2, 64, 64, True)
    assert_out_close(o, f["o"])
    f = _load("attn_paged_small", dev)
    page = f["k_cache"].shape[1]
    o = paged_flash_attention_prefill(f["q"], f["k_cache"], f["v_cache"], f["block_tables"], f["context_lens"],
                                      f["cu_seqlens"], None, float(f["scale"]), page)
    assert_out_close(o, f["o"])
    for splits in (1, 3):
        od = paged_flash_attention_decode(f["decode_q"], f["k_cache"], f["v_cache"], f["block_tables"],
                                          f["decode_context_lens"], float(f["scale"]), page, num_splits=splits)
        assert_out_close(od, f["decode_o"])

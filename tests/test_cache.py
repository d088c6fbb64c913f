"""State-cache allocator: the reference's slot order and zero-on-free
(cache/linear_attention_cache.py:46-88), with Hv heads and fp32 state."""
import pytest
import torch

from myvllm_amd.cache import LinearAttentionCache


def _cache(**kw):
    args = dict(layer_cnt=3, max_seq_cnt=4, conv_kernel_size=4, k_head_dim=8, v_head_dim=16, num_k_heads=2,
                num_v_heads=4, dtype=torch.bfloat16, device=torch.device("cpu"))
    args.update(kw)
    return LinearAttentionCache(**args)


def test_layouts_follow_the_kernels():
    c = _cache()
    assert c.conv_cache.shape == (3, 4, 3, 2 * 8 * 2 + 16 * 4)
    assert c.conv_cache.dtype == torch.bfloat16
    assert c.recurrent_cache.shape == (3, 4, 4, 8, 16)  # Hv heads, not Hk
    assert c.recurrent_cache.dtype == torch.float32
    conv, rec = c.layer(1)
    assert conv.shape == (4, 3, 96) and rec.shape == (4, 4, 8, 16)
    assert rec.stride(3) == 1 and rec.stride(2) == 16  # [K][V] contiguous per head
    assert _cache(conv_dtype=torch.float32).conv_cache.dtype == torch.float32


def test_bytes_per_seq_matches_the_tensors():
    c = _cache(conv_dtype=torch.float32)
    per = LinearAttentionCache.bytes_per_seq(3, 4, 8, 16, 2, 4, torch.bfloat16, conv_dtype=torch.float32)
    total = c.conv_cache.numel() * c.conv_cache.element_size() + c.recurrent_cache.numel() * 4
    assert per * c.max_seq_cnt == total


def test_slot_order_is_the_references():
    # free ids start as deque(range(n)); allocate pops the left end, deallocate
    # pushes on the left, so the most recently freed slot is reused first
    c = _cache()
    assert [c.allocate() for _ in range(3)] == [0, 1, 2]
    c.deallocate(1)
    c.deallocate(0)
    assert c.allocate() == 0
    assert c.allocate() == 1
    assert c.allocate() == 3
    assert not c.can_allocate()
    with pytest.raises(RuntimeError):
        c.allocate()
    c.deallocate_many([2, 3])
    assert c.allocate() == 3 and c.allocate() == 2


def test_free_zeroes_the_slot_in_every_layer_and_nothing_else():
    c = _cache()
    a, b = c.allocate(), c.allocate()
    c.conv_cache.fill_(1.0)
    c.recurrent_cache.fill_(2.0)
    c.deallocate(a)
    assert torch.count_nonzero(c.conv_cache[:, a]) == 0 and torch.count_nonzero(c.recurrent_cache[:, a]) == 0
    assert bool((c.conv_cache[:, b] == 1.0).all()) and bool((c.recurrent_cache[:, b] == 2.0).all())


def test_bad_frees_raise():
    c = _cache()
    s = c.allocate()
    with pytest.raises(ValueError):
        c.deallocate(s + 1)
    with pytest.raises(ValueError):
        c.deallocate_many([s, s])
    with pytest.raises(ValueError):
        _cache(num_k_heads=3)

"""GPU: the state cache's layer views drive the ops, and a freed slot behaves
exactly like a fresh one (zero-on-free, cache/linear_attention_cache.py:80-88)."""
import pytest
import torch

from myvllm_amd import (causal_conv1d_fn, chunk_gated_delta_rule, gated_delta_net_decode_step)
from myvllm_amd.cache import LinearAttentionCache
from myvllm_amd.workloads import cu_from_lengths

pytestmark = pytest.mark.gpu

HK, HV, K, V = 2, 4, 128, 128
D = 2 * HK * K + HV * V


def _inputs(seed, T, dev):
    g = torch.Generator().manual_seed(seed)
    r = lambda *s: torch.randn(*s, generator=g)
    return dict(x=r(T, D).bfloat16().to(dev), a=r(T, HV).bfloat16().to(dev), b=r(T, HV).bfloat16().to(dev),
                xd=r(1, D).bfloat16().to(dev), ad=r(1, HV).bfloat16().to(dev), bd=r(1, HV).bfloat16().to(dev))


def _sequence(cache, layer, slot, inp, w, A_log, dt_bias, dev):
    """Prefill T tokens then decode one, on one slot; returns both outputs."""
    conv, rec = cache.layer(layer)
    T = inp["x"].shape[0]
    idx = torch.tensor([slot], dtype=torch.int32, device=dev)
    cu = cu_from_lengths([T]).to(dev)
    y = causal_conv1d_fn(inp["x"], w, conv, idx, cu)
    q, k, v = torch.split(y, [HK * K, HK * K, HV * V], dim=-1)
    q = torch.nn.functional.normalize(q.float().reshape(T, HK, K), dim=-1, eps=1e-6).bfloat16()
    k = torch.nn.functional.normalize(k.float().reshape(T, HK, K), dim=-1, eps=1e-6).bfloat16()
    gate = -A_log.exp() * torch.nn.functional.softplus(inp["a"].float() + dt_bias)
    beta = inp["b"].float().sigmoid()
    o = chunk_gated_delta_rule(q, k, v.reshape(T, HV, V), gate, beta, rec, idx, cu)
    od = gated_delta_net_decode_step(inp["xd"], w, conv, idx, inp["ad"], inp["bd"], A_log, dt_bias, rec, idx, HK)
    return o, od


def test_freed_slot_behaves_like_a_fresh_one(dev):
    g = torch.Generator().manual_seed(0)
    w = (torch.randn(D, 4, generator=g) * 0.3).bfloat16().to(dev)
    A_log = torch.log(torch.rand(HV, generator=g) * 15 + 1).to(dev)
    dt_bias = torch.ones(HV, device=dev)
    first, other = _inputs(1, 100, dev), _inputs(2, 70, dev)

    fresh = LinearAttentionCache(2, 3, 4, K, V, HK, HV, torch.bfloat16, dev)
    s = fresh.allocate()
    ref = _sequence(fresh, 1, s, first, w, A_log, dt_bias, dev)
    assert torch.count_nonzero(fresh.recurrent_cache[1, s]) > 0
    assert torch.count_nonzero(fresh.recurrent_cache[0]) == 0  # other layer untouched

    used = LinearAttentionCache(2, 3, 4, K, V, HK, HV, torch.bfloat16, dev)
    s2 = used.allocate()
    assert s2 == s
    _sequence(used, 1, s2, other, w, A_log, dt_bias, dev)
    used.deallocate(s2)
    assert torch.count_nonzero(used.conv_cache[:, s2]) == 0 and torch.count_nonzero(used.recurrent_cache[:, s2]) == 0
    s3 = used.allocate()
    assert s3 == s2
    got = _sequence(used, 1, s3, first, w, A_log, dt_bias, dev)
    torch.cuda.synchronize()
    for a, b in zip(got, ref):
        assert torch.equal(a, b)
    assert torch.equal(used.recurrent_cache[1, s3], fresh.recurrent_cache[1, s])
    assert torch.equal(used.conv_cache[1, s3], fresh.conv_cache[1, s])

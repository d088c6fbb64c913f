"""GPU: the GDN layer (projections, conv with fused q/k L2 norm, chunked
prefill, fused decode step, gated RMSNorm, out_proj) on mixed prefill+decode
batches vs the fp64 layer oracle (oracle.layer.gdn_layer_ref).

Tolerances: outputs as for every bf16 output (rtol 2e-2, atol 1e-2).  The
layer rounds its activations to bf16 between ops (the projections, the conv
output, o before the norm), as the reference layer does, while the oracle
keeps fp64 after the projections; the carried states therefore differ by
about bf16 precision and are checked at rtol 3e-2, atol 1e-3 here (the ops'
own tests hold them to 1e-3 with exact inputs).
"""
import pytest
import torch

from conftest import assert_out_close, assert_state_close
from myvllm_amd.cache import LinearAttentionCache
from myvllm_amd.layer import GatedDeltaNet
from myvllm_amd.workloads import cu_from_lengths
from oracle.layer import gdn_layer_ref

pytestmark = pytest.mark.gpu

HID, HK, HV, K, V = 256, 2, 4, 128, 128


def _params(layer):
    cz = layer.conv_dim + layer.v_size  # in_proj rows: q | k | v | z, then b | a
    w = layer.in_proj.detach().cpu()
    return [w[:cz], w[cz:]] + [p.detach().cpu() for p in (layer.conv1d_weight, layer.A_log, layer.dt_bias,
                                                            layer.norm_weight, layer.out_proj)]


def _step(layer, cache, x, lengths, slots, n_dec, ref_conv, ref_rec, dev):
    cu = cu_from_lengths(lengths)
    idx = torch.tensor(slots, dtype=torch.int32)
    out = layer(x.to(dev), cu.to(dev), idx.to(dev), idx.to(dev), num_decode_tokens=n_dec)
    ref = gdn_layer_ref(x, *_params(layer), ref_conv, idx, ref_rec, idx, cu, HK, num_decode_tokens=n_dec)
    torch.cuda.synchronize()
    return out.cpu(), ref


def test_layer_mixed_batches_carry_state(dev):
    torch.manual_seed(0)
    layer = GatedDeltaNet(HID, HK, HV, K, V, device=dev)
    layer.init_random(seed=1)
    cache = LinearAttentionCache(1, 6, 4, K, V, HK, HV, torch.bfloat16, dev, conv_dtype=torch.float32)
    layer.conv_state, layer.recurrent_state = cache.layer(0)
    ref_conv, ref_rec = cache.conv_cache[0].cpu().clone(), cache.recurrent_cache[0].cpu().clone()
    slots = [cache.allocate() for _ in range(5)]
    g = torch.Generator().manual_seed(2)
    # call 1: prefill sequences of 100 and 37 tokens, plus 2 decode tokens (fresh slots)
    x1 = torch.randn(139, HID, generator=g).bfloat16()
    out, ref = _step(layer, cache, x1, [100, 37], slots[:4], 2, ref_conv, ref_rec, dev)
    assert_out_close(out, ref)
    # call 2: the two prefilled sequences and one earlier decode sequence decode one token each,
    # a new 70-token sequence prefills in the same batch
    x2 = torch.randn(73, HID, generator=g).bfloat16()
    out, ref = _step(layer, cache, x2, [70], [slots[4], slots[0], slots[1], slots[2]], 3, ref_conv, ref_rec, dev)
    assert_out_close(out, ref)
    assert_state_close(cache.recurrent_cache[0].cpu(), ref_rec, rtol=3e-2, atol=1e-3)
    assert torch.allclose(cache.conv_cache[0].cpu(), ref_conv, rtol=1e-2, atol=1e-2)


def test_layer_decode_only_and_prefill_only_calls(dev):
    layer = GatedDeltaNet(HID, HK, HV, K, V, device=dev)
    layer.init_random(seed=3)
    cache = LinearAttentionCache(1, 3, 4, K, V, HK, HV, torch.bfloat16, dev)
    layer.conv_state, layer.recurrent_state = cache.layer(0)
    ref_conv, ref_rec = cache.conv_cache[0].cpu().clone(), cache.recurrent_cache[0].cpu().clone()
    s = [cache.allocate() for _ in range(2)]
    g = torch.Generator().manual_seed(4)
    out, ref = _step(layer, cache, torch.randn(64, HID, generator=g).bfloat16(), [64], s[:1], 0, ref_conv, ref_rec,
                     dev)
    assert_out_close(out, ref)
    out, ref = _step(layer, cache, torch.randn(2, HID, generator=g).bfloat16(), [], s, 2, ref_conv, ref_rec, dev)
    assert_out_close(out, ref)

"""GPU: the GDN layer (projections, conv with fused q/k L2 norm, chunked
prefill, fused decode step, gated RMSNorm, out_proj) on mixed prefill+decode
batches vs the fp64 layer oracle (oracle.layer.gdn_layer_ref).

Tolerances: outputs as for every bf16 output (rtol 2e-2, atol 1e-2).  The
layer rounds its activations to bf16 between ops (the projections, the conv
output, o before the norm), as the reference layer does, while the
end-to-end oracle keeps fp64 after the projections; the carried states of
that comparison therefore differ by about bf16 precision and are checked at
rtol 3e-2, atol 1e-3.  The full-shape test also holds the layer's states to
the 1e-3 bar against the oracle fed with the very activations the layer
handed to its GDN ops (its own projection, conv and gates, recomputed on the
GPU), which removes the rounding difference.
"""
import pytest
import torch

from conftest import S_ATOL, S_RTOL, assert_out_close, assert_state_close
from myvllm_amd import causal_conv1d_fn
from myvllm_amd.cache import LinearAttentionCache
from myvllm_amd.layer import GatedDeltaNet
from myvllm_amd.norm import gdn_gating
from myvllm_amd.workloads import cu_from_lengths
from oracle.gdn import chunk_gated_delta_rule_ref
from oracle.layer import gdn_decode_step_ref, gdn_layer_ref

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


def test_layer_full_shape_4x2048_prefill_128_decode(dev):
    """The layer workload at its full shape: hidden 2048, Hk 16 / Hv 32,
    d 128, 4 x 2048 prefill tokens (fresh sequences) and 128 decode tokens
    (continuing sequences with random conv and SSM states) in one call,
    weights ~N(0, 0.02)."""
    hidden, Hk, Hv, n_pre, len_pre, n_dec = 2048, 16, 32, 4, 2048, 128
    Tp, T = n_pre * len_pre, n_pre * len_pre + n_dec
    print(f"layer full shape: hidden {hidden}, Hk {Hk} / Hv {Hv}, {n_pre} x {len_pre} prefill + {n_dec} decode",
          flush=True)
    layer = GatedDeltaNet(hidden, Hk, Hv, K, V, device=dev)
    layer.init_random(std=0.02, seed=5)
    nslots = n_pre + n_dec + 8
    cache = LinearAttentionCache(1, nslots, 4, K, V, Hk, Hv, torch.bfloat16, dev, conv_dtype=torch.float32)
    layer.conv_state, layer.recurrent_state = cache.layer(0)
    gen = torch.Generator().manual_seed(6)
    idx = torch.randperm(nslots, generator=gen)[: n_pre + n_dec].to(torch.int32)
    dec = idx[n_pre:].long()
    conv0 = torch.zeros(cache.conv_cache[0].shape)
    rec0 = torch.zeros(cache.recurrent_cache[0].shape)
    conv0[dec] = torch.randn((n_dec,) + tuple(conv0.shape[1:]), generator=gen)
    rec0[dec] = torch.randn((n_dec,) + tuple(rec0.shape[1:]), generator=gen) * 0.1
    cache.conv_cache[0].copy_(conv0)
    cache.recurrent_cache[0].copy_(rec0)
    x = torch.randn(T, hidden, generator=gen).bfloat16()
    cu = cu_from_lengths([len_pre] * n_pre)
    xd, cud, idxd = x.to(dev), cu.to(dev), idx.to(dev)

    out = layer(xd, cud, idxd, idxd, num_decode_tokens=n_dec)
    torch.cuda.synchronize()
    out, conv_gpu, rec_gpu = out.cpu(), cache.conv_cache[0].cpu(), cache.recurrent_cache[0].cpu()

    # 1) the GDN ops at the 1e-3 state bar, on the activations the layer formed
    L = layer
    cz = L.conv_dim + L.v_size
    with torch.no_grad():
        proj = xd @ L.in_proj.t()
        y = causal_conv1d_fn(proj[:Tp, :L.conv_dim], L.conv1d_weight, conv0.to(dev), idxd[:n_pre], cud,
                             l2norm_channels=2 * L.k_size)
        g, beta = gdn_gating(proj[:Tp, cz + Hv:], proj[:Tp, cz:cz + Hv], L.A_log, L.dt_bias)
    y, g, beta, proj = y.cpu(), g.cpu(), beta.cpu(), proj.cpu()
    rec_ops = rec0.clone()
    print("layer full shape: op-level oracle", flush=True)
    chunk_gated_delta_rule_ref(y[:, :L.k_size].view(Tp, Hk, K), y[:, L.k_size:2 * L.k_size].view(Tp, Hk, K),
                               y[:, 2 * L.k_size:].view(Tp, Hv, V), g, beta, rec_ops, idx[:n_pre], cu)
    gdn_decode_step_ref(proj[Tp:, :L.conv_dim], L.conv1d_weight.detach().cpu(), conv0.clone(), idx[n_pre:],
                        proj[Tp:, cz + Hv:], proj[Tp:, cz:cz + Hv], L.A_log.detach().cpu(), L.dt_bias.detach().cpu(),
                        rec_ops, idx[n_pre:], Hk)
    used = idx.long()
    assert_state_close(rec_gpu[used], rec_ops[used])
    untouched = torch.ones(nslots, dtype=torch.bool)
    untouched[used] = False
    assert torch.equal(rec_gpu[untouched], rec0[untouched])
    assert torch.equal(conv_gpu[untouched], conv0[untouched])

    # 2) end to end against the fp64 layer oracle
    print("layer full shape: end-to-end oracle", flush=True)
    conv_ref, rec_ref = conv0.clone(), rec0.clone()
    ref = gdn_layer_ref(x, *_params(layer), conv_ref, idx, rec_ref, idx, cu, Hk, num_decode_tokens=n_dec)
    assert_out_close(out, ref)
    err = (rec_gpu[used].double() - rec_ref[used].double()).abs()
    worst = (err / (S_ATOL + S_RTOL * rec_ref[used].double().abs())).max().item()
    print(f"layer full shape: worst state error vs the end-to-end oracle = {worst:.3f} x the 1e-3 bar", flush=True)
    assert_state_close(rec_gpu[used], rec_ref[used], rtol=3e-2, atol=1e-3)
    assert torch.allclose(conv_gpu, conv_ref.float(), rtol=1e-2, atol=1e-2)



def test_layer_overlapped_decode_matches_serial_order(dev):
    """In a mixed batch the layer runs its decode step on a second stream,
    beside the chunked prefill.  The two touch disjoint cache slots, so the
    output and both caches must equal, bit for bit, the same ops issued in
    order on one stream (three calls in a row, caches carried)."""
    from myvllm_amd import chunk_gated_delta_rule, gated_delta_net_decode_step
    from myvllm_amd.norm import rms_norm_gated

    hidden, Hk, Hv, n_pre, len_pre, n_dec = 512, 4, 8, 4, 600, 64
    Tp, T = n_pre * len_pre, n_pre * len_pre + n_dec
    layer = GatedDeltaNet(hidden, Hk, Hv, K, V, device=dev)
    layer.init_random(std=0.02, seed=7)
    nslots = n_pre + n_dec
    cache = LinearAttentionCache(1, nslots, 4, K, V, Hk, Hv, torch.bfloat16, dev, conv_dtype=torch.float32)
    gen = torch.Generator().manual_seed(8)
    cache.conv_cache[0].copy_(torch.randn(cache.conv_cache[0].shape, generator=gen))
    cache.recurrent_cache[0].copy_(torch.randn(cache.recurrent_cache[0].shape, generator=gen) * 0.1)
    conv_s, rec_s = cache.conv_cache[0].clone(), cache.recurrent_cache[0].clone()
    idx = torch.randperm(nslots, generator=gen).to(torch.int32).to(dev)
    cu = cu_from_lengths([len_pre] * n_pre).to(dev)
    L = layer
    cz = L.conv_dim + L.v_size

    def serial(x):
        proj = x @ L.in_proj.t()
        qkv, z = proj[:, :L.conv_dim], proj[:, L.conv_dim:cz]
        b, a = proj[:, cz:cz + Hv], proj[:, cz + Hv:]
        o = torch.empty(T, Hv, V, dtype=x.dtype, device=dev)
        y = causal_conv1d_fn(qkv[:Tp], L.conv1d_weight, conv_s, idx[:n_pre], cu, l2norm_channels=2 * L.k_size)
        g, beta = gdn_gating(a[:Tp], b[:Tp], L.A_log, L.dt_bias)
        chunk_gated_delta_rule(y[:, :L.k_size].view(Tp, Hk, K), y[:, L.k_size:2 * L.k_size].view(Tp, Hk, K),
                               y[:, 2 * L.k_size:].view(Tp, Hv, V), g, beta, rec_s, idx[:n_pre], cu, out=o[:Tp])
        gated_delta_net_decode_step(qkv[Tp:], L.conv1d_weight, conv_s, idx[n_pre:], a[Tp:], b[Tp:], L.A_log,
                                    L.dt_bias, rec_s, idx[n_pre:], Hk, out=o[Tp:])
        on = rms_norm_gated(o, z.view(T, Hv, V), L.norm_weight, L.rms_norm_eps)
        return on.view(T, L.v_size) @ L.out_proj.t()

    layer.conv_state, layer.recurrent_state = cache.layer(0)
    with torch.no_grad():
        for call in range(3):
            x = torch.randn(T, hidden, generator=gen).bfloat16().to(dev)
            out = layer(x, cu, idx, idx, num_decode_tokens=n_dec)
            ref = serial(x)
            torch.cuda.synchronize()
            print(f"overlapped layer call {call}", flush=True)
            assert torch.equal(out, ref)
            assert torch.equal(cache.recurrent_cache[0], rec_s)
            assert torch.equal(cache.conv_cache[0], conv_s)


def test_layer_fp32_mixed_batch(dev):
    """The layer in float32 (weights, activations and caches): every op takes
    fp32, the chunked prefill through its fp32 route (q and k rounded to fp16,
    v as fp16 hi + lo).  Against the fp64 layer oracle: the output within
    rtol 1e-2 / atol 1e-3 and the SSM states within 1e-3 relative in norm."""
    torch.manual_seed(0)
    layer = GatedDeltaNet(HID, HK, HV, K, V, dtype=torch.float32, device=dev)
    layer.init_random(seed=11)
    cache = LinearAttentionCache(1, 6, 4, K, V, HK, HV, torch.float32, dev, conv_dtype=torch.float32)
    layer.conv_state, layer.recurrent_state = cache.layer(0)
    ref_conv, ref_rec = cache.conv_cache[0].cpu().clone(), cache.recurrent_cache[0].cpu().clone()
    slots = [cache.allocate() for _ in range(5)]
    g = torch.Generator().manual_seed(12)
    print("layer fp32 mixed batch", flush=True)
    for lengths, sl, n_dec, T in (([100, 37], slots[:4], 2, 139), ([70], [slots[4], slots[0], slots[1], slots[2]], 3, 73)):
        x = torch.randn(T, HID, generator=g)
        out, ref = _step(layer, cache, x, lengths, sl, n_dec, ref_conv, ref_rec, dev)
        assert out.dtype == torch.float32
        assert_out_close(out, ref, rtol=1e-2, atol=1e-3)
    rec = cache.recurrent_cache[0].cpu().double()
    used = torch.tensor(slots, dtype=torch.long)
    rel = ((rec[used] - ref_rec[used].double()).norm() / ref_rec[used].double().norm()).item()
    assert rel < 1e-3, rel
    assert torch.allclose(cache.conv_cache[0].cpu().double(), ref_conv.double(), rtol=1e-4, atol=1e-5)


def test_layer_reference_call_form(dev):
    """The reference's positional call ``layer(x, cu_seqlens,
    conv_state_indices, recurrent_state_indices, is_prefill)``
    (layers/linear_attention.py:77-84): True is an all-prefill call, False an
    all-decode call; each equals, bit for bit, the same batch given by
    ``num_decode_tokens``, from the same caches."""
    layer = GatedDeltaNet(HID, HK, HV, K, V, device=dev)
    layer.init_random(seed=11)
    g = torch.Generator().manual_seed(12)
    cache = LinearAttentionCache(1, 8, 4, K, V, HK, HV, torch.bfloat16, dev, conv_dtype=torch.float32)
    cache.conv_cache[0].copy_(torch.randn(cache.conv_cache[0].shape, generator=g))
    cache.recurrent_cache[0].copy_(torch.randn(cache.recurrent_cache[0].shape, generator=g) * 0.1)
    conv0, rec0 = cache.conv_cache[0].clone(), cache.recurrent_cache[0].clone()
    layer.conv_state, layer.recurrent_state = cache.layer(0)
    cu = cu_from_lengths([90, 38]).to(dev)
    idx = torch.tensor([5, 2], dtype=torch.int32, device=dev)
    x = torch.randn(128, HID, generator=g).bfloat16().to(dev)
    results = []
    for kw in (dict(), dict(num_decode_tokens=0)):
        cache.conv_cache[0].copy_(conv0)
        cache.recurrent_cache[0].copy_(rec0)
        out = layer(x, cu, idx, idx, True, **kw) if not kw else layer(x, cu, idx, idx, **kw)
        torch.cuda.synchronize()
        results.append((out.cpu(), cache.conv_cache[0].cpu(), cache.recurrent_cache[0].cpu()))
    for a, b in zip(*results):
        assert torch.equal(a, b)
    xd = torch.randn(3, HID, generator=g).bfloat16().to(dev)
    idx3 = torch.tensor([1, 6, 3], dtype=torch.int32, device=dev)
    results = []
    for form in ("flag", "count"):
        cache.conv_cache[0].copy_(conv0)
        cache.recurrent_cache[0].copy_(rec0)
        if form == "flag":
            out = layer(xd, cu, idx3, idx3, False)
        else:
            out = layer(xd, cu[:1], idx3, idx3, num_decode_tokens=3)
        torch.cuda.synchronize()
        results.append((out.cpu(), cache.conv_cache[0].cpu(), cache.recurrent_cache[0].cpu()))
    for a, b in zip(*results):
        assert torch.equal(a, b)


@pytest.mark.parametrize("bad", ["idx_len", "bool_count", "count_range", "cu_dtype", "flag_mismatch", "rec_dtype"])
def test_layer_rejects_bad_calls_before_launching(dev, bad):
    """A malformed call raises before any kernel runs: both caches stay bit
    for bit what they were (the last check used to come from the decode
    step's own validation, after the prefill had written the cache)."""
    layer = GatedDeltaNet(HID, HK, HV, K, V, device=dev)
    layer.init_random(seed=13)
    g = torch.Generator().manual_seed(14)
    cache = LinearAttentionCache(1, 6, 4, K, V, HK, HV, torch.bfloat16, dev, conv_dtype=torch.float32)
    cache.conv_cache[0].copy_(torch.randn(cache.conv_cache[0].shape, generator=g))
    cache.recurrent_cache[0].copy_(torch.randn(cache.recurrent_cache[0].shape, generator=g) * 0.1)
    conv0, rec0 = cache.conv_cache[0].clone(), cache.recurrent_cache[0].clone()
    layer.conv_state, layer.recurrent_state = cache.layer(0)
    x = torch.randn(70, HID, generator=g).bfloat16().to(dev)
    cu = cu_from_lengths([40, 28]).to(dev)
    idx = torch.tensor([0, 4, 2, 5], dtype=torch.int32, device=dev)
    kw = dict(num_decode_tokens=2)
    if bad == "idx_len":
        idx = idx[:3]
    elif bad == "bool_count":
        kw = dict(num_decode_tokens=True)
    elif bad == "count_range":
        kw = dict(num_decode_tokens=71)
    elif bad == "cu_dtype":
        cu = cu.float()
    elif bad == "flag_mismatch":
        args = (x, cu, idx, idx, True)
        kw = dict(num_decode_tokens=2)
    elif bad == "rec_dtype":
        layer.recurrent_state = cache.recurrent_cache[0].double()
    with pytest.raises((ValueError, TypeError)):
        if bad == "flag_mismatch":
            layer(*args, **kw)
        else:
            layer(x, cu, idx, idx, **kw)
    torch.cuda.synchronize()
    assert torch.equal(cache.conv_cache[0], conv0)
    assert torch.equal(cache.recurrent_cache[0], rec0)

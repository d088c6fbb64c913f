"""GPU: the ops replayed from a captured HIP graph.

The ops launch on torch's current stream, never synchronise the host and
issue no memset, so a caller can capture them.  Each test captures a step,
replays it three times with eager work and synchronisations between the
replays, resets the caches before each replay, and checks every replay
against the same step run eagerly from the same caches: bit for bit.
"""
import pytest
import torch

from myvllm_amd.cache import LinearAttentionCache
from myvllm_amd.layer import GatedDeltaNet
from myvllm_amd.workloads import cu_from_lengths, paged_case
from myvllm_amd import paged_flash_attention_decode

pytestmark = pytest.mark.gpu


def _eager_work(dev):
    a = torch.randn(256, 256, device=dev)
    (a @ a).sum().item()


def test_layer_step_replays_from_a_graph(dev):
    """A mixed batch through GatedDeltaNet (input GEMM, conv + q/k norm,
    gating, chunked prefill, the decode step on its second stream, gated
    RMSNorm, output GEMM): the fork to the second stream and the join are
    captured with the rest."""
    hidden, Hk, Hv, K, V = 512, 4, 8, 128, 128
    lengths, n_dec = [300, 64, 1, 129], 16
    Np = len(lengths)
    layer = GatedDeltaNet(hidden, Hk, Hv, K, V, device=dev)
    layer.init_random(std=0.02, seed=9)
    cache = LinearAttentionCache(1, Np + n_dec, 4, K, V, Hk, Hv, torch.bfloat16, dev, conv_dtype=torch.float32)
    layer.conv_state, layer.recurrent_state = cache.layer(0)
    gen = torch.Generator().manual_seed(10)
    cs0 = torch.randn(cache.conv_cache[0].shape, generator=gen).to(dev)
    rs0 = (torch.randn(cache.recurrent_cache[0].shape, generator=gen) * 0.1).to(dev)
    T = sum(lengths) + n_dec
    x = torch.randn(T, hidden, generator=gen).bfloat16().to(dev)
    cu = cu_from_lengths(lengths).to(dev)
    idx = torch.randperm(Np + n_dec, generator=gen).to(torch.int32).to(dev)

    def reset():
        cache.conv_cache[0].copy_(cs0)
        cache.recurrent_cache[0].copy_(rs0)

    def step():
        return layer(x, cu, idx, idx, num_decode_tokens=n_dec)

    with torch.no_grad():
        reset()
        ref = step()
        torch.cuda.synchronize()
        ref_cs, ref_rs = cache.conv_cache[0].clone(), cache.recurrent_cache[0].clone()

        side = torch.cuda.Stream(device=dev)  # warm-up off the capture stream, as torch asks
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                reset()
                step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()

        graph = torch.cuda.CUDAGraph()
        reset()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph):
            out = step()
        for rep in range(3):
            reset()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            print(f"layer graph replay {rep}", flush=True)
            assert torch.equal(out, ref)
            assert torch.equal(cache.conv_cache[0], ref_cs)
            assert torch.equal(cache.recurrent_cache[0], ref_rs)
            _eager_work(dev)


def test_paged_decode_with_splits_replays_from_a_graph(dev):
    """The split-KV paged decode (partials in a workspace the op allocates,
    then the combine kernel) captured and replayed."""
    case = paged_case([700, 33, 0, 256], [1, 1, 1, 1], page=16, seed=12, Hq=16, Hkv=2, D=256)
    args = [t.to(dev) for t in (case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens)]

    def step():
        return paged_flash_attention_decode(*args, case.scale, case.page, num_splits=4)

    ref = step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=dev)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        print(f"paged decode graph replay {rep}", flush=True)
        assert torch.equal(out, ref)
        _eager_work(dev)

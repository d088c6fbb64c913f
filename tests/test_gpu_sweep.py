"""GPU: a seeded random sweep of shapes through the ops vs the oracles.

The other GPU tests pin chosen cases.  This one draws configurations from a
fixed seed (sequence counts and ragged lengths including empty and one-token
sequences, head counts and GQA ratios, head dims, input dtypes, decay
strength, padding slots, int32/int64 index tensors, the prefill's item
stream, the fused decode step's two caches, the paged decode's key splits)
so that combinations no hand-written case names meet the same bars:
bf16/fp16 outputs within rtol 2e-2 / atol 1e-2 (fp32 decode outputs within
1e-4 / 1e-5), fp32 states within 1e-3 |ref| + 1e-6, conv states bit-exact,
and every slot outside the batch unchanged bit for bit.
"""
import random

import pytest
import torch

from conftest import assert_out_close, assert_state_close
from test_gpu_attention import _varlen, assert_attn_close
from test_gpu_conv import _prefill as conv_prefill
from test_gpu_decode import _run as decode_run
from test_gpu_prefill import _check as prefill_check
from test_gpu_prefill import _run as prefill_run
from myvllm_amd import causal_conv1d_update, paged_flash_attention_prefill
from myvllm_amd.workloads import (attn_varlen_case, conv_decode_case, conv_prefill_case, decode_case, paged_case,
                                   prefill_case)
from oracle.attention import flash_attention_prefill_ref, paged_attention_ref
from oracle.conv import causal_conv1d_update_ref

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16]


def _length(r: random.Random, hi: int) -> int:
    return r.choice([0, 1, r.randint(2, 63), 64, r.randint(65, hi)])


def _prefill_cfg(i: int) -> dict:
    r = random.Random(1000 + i)
    Hk = r.choice([1, 2, 4])
    return dict(lengths=[_length(r, 300) for _ in range(r.randint(1, 6))], Hk=Hk, Hv=Hk * r.choice([1, 2, 4]),
                K=r.choice([128, 64, 8 * r.randint(1, 16)]), V=r.choice([128, 64, 8 * r.randint(1, 16)]),
                dtype=r.choice(DTYPES), g_scale=r.choice([0.05, 1.0, 3.0]), pad=r.random() < 0.3,
                i64=r.random() < 0.3, per_wg=r.choice([None, None, 1, 3, 64]))


@pytest.mark.parametrize("i", range(40))
def test_sweep_prefill(dev, i):
    c = _prefill_cfg(i)
    print(f"sweep prefill {i}: {c}", flush=True)
    N = len(c["lengths"])
    case = prefill_case(c["lengths"], seed=i, num_slots=N + 2, Hk=c["Hk"], Hv=c["Hv"], K=c["K"], V=c["V"],
                        dtype=c["dtype"], g_scale=c["g_scale"])
    idx, cu = case.idx.clone(), case.cu.clone()
    if c["pad"]:
        idx[N // 2] = -1
    if c["i64"]:
        idx, cu = idx.long(), cu.long()
    o, st, o_ref, st_ref = prefill_run(case, dev, idx=idx, cu=cu, items_per_wg=c["per_wg"])
    prefill_check(case, o, st, o_ref, st_ref, idx=idx)
    if c["pad"]:
        s, e = int(cu[N // 2]), int(cu[N // 2 + 1])
        assert torch.count_nonzero(o[s:e]) == 0


@pytest.mark.parametrize("i", range(24))
def test_sweep_decode(dev, i):
    r = random.Random(2000 + i)
    Hk = r.choice([1, 2, 4])
    c = dict(B=r.randint(1, 40), Hk=Hk, Hv=Hk * r.choice([1, 2, 4]), K=r.choice([128, 64, 8 * r.randint(1, 16)]),
             V=r.choice([128, 64, 8 * r.randint(1, 16)]), dtype=r.choice(DTYPES + [torch.float32]),
             pad=r.random() < 0.3, i64=r.random() < 0.3)
    print(f"sweep decode {i}: {c}", flush=True)
    slots = c["B"] + 3
    case = decode_case(B=c["B"], num_slots=slots, seed=i, Hk=c["Hk"], Hv=c["Hv"], K=c["K"], V=c["V"],
                       dtype=c["dtype"])
    idx = case.idx.clone()
    if c["pad"]:
        idx[c["B"] // 2] = -1
    if c["i64"]:
        idx = idx.long()
    o, st, o_ref, st_ref = decode_run(case, dev, idx=idx)
    o = o.cpu()
    if c["dtype"] == torch.float32:
        assert_out_close(o, o_ref, rtol=1e-4, atol=1e-5)
    else:
        assert_out_close(o, o_ref)
    used = torch.tensor([int(s) for s in idx.tolist() if s >= 0], dtype=torch.long)
    assert_state_close(st[used], st_ref[used])
    untouched = torch.ones(slots, dtype=torch.bool)
    untouched[used] = False
    assert torch.equal(st[untouched], case.state[untouched])
    if c["pad"]:
        assert torch.count_nonzero(o[c["B"] // 2]) == 0


@pytest.mark.parametrize("i", range(16))
def test_sweep_conv(dev, i):
    r = random.Random(3000 + i)
    c = dict(lengths=[_length(r, 400) for _ in range(r.randint(1, 6))], D=8 * r.randint(1, 96), W=r.randint(2, 6),
             dtype=r.choice(DTYPES), state_dtype=r.choice([torch.float32, None]), i64=r.random() < 0.3)
    print(f"sweep conv {i}: {c}", flush=True)
    sd = c["state_dtype"] or c["dtype"]
    case = conv_prefill_case(c["lengths"], seed=i, D=c["D"], W=c["W"], num_slots=len(c["lengths"]) + 2,
                             dtype=c["dtype"], state_dtype=sd)
    if c["i64"]:
        case.idx, case.cu = case.idx.long(), case.cu.long()
    y, st, y_ref, st_ref = conv_prefill(case, dev)
    assert_out_close(y, y_ref)
    assert torch.equal(st, st_ref)


@pytest.mark.parametrize("i", range(10))
def test_sweep_conv_update(dev, i):
    r = random.Random(4000 + i)
    c = dict(B=r.randint(1, 64), D=8 * r.randint(1, 96), W=r.randint(2, 6), dtype=r.choice(DTYPES))
    print(f"sweep conv update {i}: {c}", flush=True)
    case = conv_decode_case(B=c["B"], seed=i, D=c["D"], W=c["W"], num_slots=c["B"] + 4, dtype=c["dtype"])
    st_ref = case.state.clone()
    y_ref = causal_conv1d_update_ref(case.x, case.weight, st_ref, case.idx)
    st = case.state.to(dev)
    y = causal_conv1d_update(case.x.to(dev), case.weight.to(dev), st, case.idx.to(dev))
    torch.cuda.synchronize()
    assert_out_close(y.cpu(), y_ref)
    assert torch.equal(st.cpu(), st_ref)


@pytest.mark.parametrize("i", range(20))
def test_sweep_attention_varlen(dev, i):
    r = random.Random(5000 + i)
    Hkv = r.choice([1, 2, 4])
    c = dict(lengths=[_length(r, 300) for _ in range(r.randint(1, 5))], Hkv=Hkv, Hq=Hkv * r.choice([1, 2, 3, 8]),
             D=r.choice([64, 128, 256]), causal=r.random() < 0.7, dtype=r.choice(DTYPES))
    print(f"sweep attention varlen {i}: {c}", flush=True)
    case = attn_varlen_case(c["lengths"], seed=i, Hq=c["Hq"], Hkv=c["Hkv"], D=c["D"], dtype=c["dtype"])
    out = _varlen(case, dev, c["causal"])
    ref = flash_attention_prefill_ref(case.q, case.k, case.v, case.cu, case.scale, is_causal=c["causal"])
    assert_attn_close(out, ref)


@pytest.mark.parametrize("i", range(16))
def test_sweep_paged_prefill(dev, i):
    r = random.Random(6000 + i)
    Hkv = r.choice([1, 2])
    n = r.randint(1, 4)
    new = [r.randint(1, 200) for _ in range(n)]
    ctx = [m + r.choice([0, r.randint(1, 300)]) for m in new]
    c = dict(ctx=ctx, new=new, page=r.choice([16, 32, 7, 48]), Hkv=Hkv, Hq=Hkv * r.choice([1, 4, 8]),
             D=r.choice([64, 128, 256]), dtype=r.choice(DTYPES))
    print(f"sweep paged prefill {i}: {c}", flush=True)
    case = paged_case(c["ctx"], c["new"], page=c["page"], seed=i, Hq=c["Hq"], Hkv=c["Hkv"], D=c["D"],
                      dtype=c["dtype"])
    out = paged_flash_attention_prefill(case.q.to(dev), case.k_cache.to(dev), case.v_cache.to(dev),
                                        case.block_tables.to(dev), case.context_lens.to(dev), case.cu.to(dev),
                                        None, case.scale, case.page).cpu()
    ref = paged_attention_ref(case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens, case.cu,
                              case.scale)
    assert_attn_close(out, ref)


@pytest.mark.parametrize("i", range(12))
def test_sweep_fused_decode(dev, i):
    from test_gpu_decode_fused import _check as fused_check
    from test_gpu_decode_fused import _run as fused_run
    from myvllm_amd.workloads import decode_fused_case

    r = random.Random(7000 + i)
    Hk = r.choice([1, 2, 4])
    dt = r.choice(DTYPES + [torch.float32])
    c = dict(B=r.randint(1, 24), Hk=Hk, Hv=Hk * r.choice([1, 2, 4]), dtype=dt,
             cs_dtype=r.choice([torch.float32, dt]), w_dtype=r.choice([torch.float32, dt]),
             conv_pad=r.random() < 0.3, state_pad=r.random() < 0.3, i64=r.random() < 0.3, steps=r.choice([1, 2]))
    print(f"sweep fused decode {i}: {c}", flush=True)
    slots = c["B"] + 3
    case = decode_fused_case(B=c["B"], num_slots=slots, seed=i, Hk=c["Hk"], Hv=c["Hv"], dtype=c["dtype"],
                             conv_state_dtype=c["cs_dtype"], weight_dtype=c["w_dtype"])
    cidx, idx = case.conv_idx.clone(), case.idx.clone()
    if c["conv_pad"]:
        cidx[0] = -1
    if c["state_pad"]:
        idx[c["B"] - 1] = slots + 5
    if c["i64"]:
        cidx, idx = cidx.long(), idx.long()
    outs, refs, cs, cs_ref, st, st_ref = fused_run(case, dev, cidx=cidx, idx=idx, steps=c["steps"])
    fused_check(outs, refs, cs, cs_ref, st, st_ref)
    if c["state_pad"]:
        assert all(torch.count_nonzero(o[c["B"] - 1]) == 0 for o in outs)
    used = {int(s) for s in idx.tolist() if 0 <= s < slots}
    untouched = [s for s in range(slots) if s not in used]
    assert torch.equal(st[untouched], case.state[untouched])


@pytest.mark.parametrize("i", range(12))
def test_sweep_paged_decode(dev, i):
    from test_gpu_attention import _decode, _decode_ref
    from myvllm_amd.workloads import paged_case

    r = random.Random(8000 + i)
    Hkv = r.choice([1, 2])
    B = r.randint(1, 12)
    c = dict(ctx=[r.choice([0, 1, r.randint(2, 600)]) for _ in range(B)], page=r.choice([16, 32, 7]), Hkv=Hkv,
             Hq=Hkv * r.choice([1, 4, 8, 16]), D=r.choice([64, 128, 256]), dtype=r.choice(DTYPES),
             splits=r.choice([1, 2, 4, 7]))
    print(f"sweep paged decode {i}: {c}", flush=True)
    # one query row per sequence, also for an empty context (its output must be zero)
    case = paged_case(c["ctx"], [1] * B, page=c["page"], seed=i, Hq=c["Hq"], Hkv=c["Hkv"], D=c["D"],
                      dtype=c["dtype"])
    out = _decode(case, dev, c["splits"])
    ref = _decode_ref(case)
    assert_attn_close(out, ref)
    for b, L in enumerate(c["ctx"]):
        if L == 0:
            assert torch.count_nonzero(out[b]) == 0


@pytest.mark.parametrize("i", range(10))
def test_sweep_prefill_fp32(dev, i):
    """fp32 q/k/v through the prefill's fp32 route: outputs within
    1e-3 + 2e-3 |ref| of the oracle on the raw inputs, states within the
    1e-3 |ref| + 1e-6 bar of the oracle fed the same fp16-rounded q and k."""
    from oracle.gdn import chunk_gated_delta_rule_ref

    c = _prefill_cfg(500 + i)
    print(f"sweep prefill fp32 {i}: {c}", flush=True)
    N = len(c["lengths"])
    case = prefill_case(c["lengths"], seed=500 + i, num_slots=N + 2, Hk=c["Hk"], Hv=c["Hv"], K=c["K"], V=c["V"],
                        dtype=torch.float32, g_scale=c["g_scale"])
    idx, cu = case.idx.clone(), case.cu.clone()
    if c["pad"]:
        idx[N // 2] = -1
    if c["i64"]:
        idx, cu = idx.long(), cu.long()
    o, st, o_ref, _ = prefill_run(case, dev, idx=idx, cu=cu)
    assert_out_close(o, o_ref, rtol=2e-3, atol=1e-3)
    st_r = case.state.clone()
    chunk_gated_delta_rule_ref(case.q.half().float(), case.k.half().float(), case.v, case.g, case.beta, st_r, idx, cu)
    used = torch.tensor([int(s) for s in idx.tolist() if 0 <= int(s) < N + 2], dtype=torch.long)
    assert_state_close(st[used], st_r[used])
    untouched = torch.ones(N + 2, dtype=torch.bool)
    untouched[used] = False
    assert torch.equal(st[untouched], case.state[untouched])

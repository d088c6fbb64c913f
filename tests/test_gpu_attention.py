"""GPU: full attention (ops/full_attention.py of the reference) vs the fp64 oracle.

Varlen prefill (causal and not, GQA and MHA, ragged and empty sequences),
paged prefill over permuted pages with a cached prefix, and paged decode with
1..7 key splits, at small sizes in full and at the attention layer's workload
sizes on sampled rows (prefill) or in full (decode).  Tolerance: the bf16
bar |o - ref| <= 1e-2 + 2e-2 |ref| per element (P is rounded to bf16 before
P V, as in the reference, which alone moves a short row by up to
2^-9 max|v|); since outputs over thousands of keys are small (|o| ~ 0.05),
the relative error norm over the tensor must also stay below 5e-3.
"""
import pytest
import torch

from conftest import assert_out_close
from myvllm_amd import flash_attention_prefill, paged_flash_attention_decode, paged_flash_attention_prefill
from myvllm_amd.workloads import (attn_decode_case, attn_paged_prefill_case, attn_prefill_32k_case, attn_varlen_case,
                                   paged_case)
from oracle.attention import attention_rows_ref, flash_attention_prefill_ref, gather_paged, paged_attention_ref

pytestmark = pytest.mark.gpu


def assert_attn_close(out, ref):
    assert_out_close(out, ref)
    ref = ref.double()
    err = (out.double() - ref).norm() / ref.norm().clamp_min(1e-12)
    assert err < 5e-3, f"relative error norm {err:.3e}"


def _varlen(case, dev, causal, **kw):
    Hq, Hkv, Dh = case.q.shape[1], case.k.shape[1], case.q.shape[2]
    return flash_attention_prefill(case.q.to(dev), case.k.to(dev), case.v.to(dev), case.cu.to(dev), case.scale,
                                   Hq, Hkv, Dh, Dh, causal, **kw).cpu()


@pytest.mark.parametrize(
    "lengths, Hq, Hkv, Dh, causal, dtype",
    [
        ([1, 31, 33, 100, 257], 16, 2, 256, True, torch.bfloat16),
        ([70, 0, 129], 16, 2, 256, False, torch.bfloat16),
        ([5, 64, 200], 4, 4, 128, True, torch.bfloat16),  # MHA: four query blocks per workgroup
        ([300, 17], 4, 4, 128, False, torch.float16),
        ([96, 1, 45], 8, 4, 64, True, torch.bfloat16),  # two heads per kv head
        ([130], 6, 2, 128, True, torch.bfloat16),  # three heads per kv head
    ],
)
def test_varlen_prefill(dev, lengths, Hq, Hkv, Dh, causal, dtype):
    case = attn_varlen_case(lengths, seed=sum(lengths), Hq=Hq, Hkv=Hkv, D=Dh, dtype=dtype)
    print(f"varlen lengths={lengths} Hq={Hq} Hkv={Hkv} D={Dh} causal={causal} {dtype}", flush=True)
    out = _varlen(case, dev, causal)
    ref = flash_attention_prefill_ref(case.q, case.k, case.v, case.cu, case.scale, is_causal=causal)
    assert out.dtype == dtype
    assert_attn_close(out, ref)


def test_varlen_prefill_int64_cu_and_explicit_max(dev):
    case = attn_varlen_case([40, 90], seed=5, Hq=4, Hkv=2, D=128)
    case.cu = case.cu.to(torch.int64)
    out = _varlen(case, dev, True, max_seqlen=90)
    assert_attn_close(out, flash_attention_prefill_ref(case.q, case.k, case.v, case.cu, case.scale))


@pytest.mark.parametrize("Dh, causal", [(256, True), (256, False), (128, True), (64, True)])
def test_varlen_prefill_sharp_scores(dev, Dh, causal):
    """Scores spread over hundreds of exp2 units (scale 4 on unit-variance q, k):
    the running maximum must be the maximum over both lane halves of a query's
    keys, or the exponentials of the other half overflow to inf."""
    case = attn_varlen_case([1, 33, 130], seed=Dh + causal, Hq=4, Hkv=2, D=Dh)
    case.scale = 4.0
    print(f"varlen sharp scores D={Dh} causal={causal}", flush=True)
    out = _varlen(case, dev, causal)
    ref = flash_attention_prefill_ref(case.q, case.k, case.v, case.cu, case.scale, is_causal=causal)
    assert torch.isfinite(out).all()
    assert_attn_close(out, ref)


def test_varlen_prefill_negative_scale(dev):
    case = attn_varlen_case([50, 7], seed=6, Hq=4, Hkv=2, D=64)
    case.scale = -0.2
    out = _varlen(case, dev, True)
    assert_attn_close(out, flash_attention_prefill_ref(case.q, case.k, case.v, case.cu, case.scale))


def test_varlen_prefill_layer_workload_sampled_rows(dev):
    """The 16-sequence causal prefill of the attention layer (Hq 16, Hkv 2,
    D 256): every sequence's first, last and 14 random rows vs the oracle."""
    case = attn_prefill_32k_case()
    print(f"attn prefill workload T={case.q.shape[0]}", flush=True)
    out = _varlen(case, dev, True)
    g = torch.Generator().manual_seed(7)
    cu = case.cu.tolist()
    for n in range(len(cu) - 1):
        s, e = cu[n], cu[n + 1]
        pos = torch.cat([torch.tensor([0, e - s - 1]), torch.randint(0, e - s, (14,), generator=g)])
        ref = attention_rows_ref(case.q[s + pos], case.k[s:e], case.v[s:e], pos, case.scale, causal=True)
        assert_attn_close(out[s + pos], ref)


@pytest.mark.parametrize(
    "ctx, new, page, Hq, Hkv, Dh",
    [
        ([40, 300, 17], [40, 100, 1], 16, 16, 2, 256),  # no prefix / prefix / one new token
        ([77, 130], [33, 130], 7, 4, 4, 128),  # page size 7, MHA
        ([64, 0, 5], [10, 0, 5], 16, 8, 2, 64),  # an empty sequence
        ([200, 1000], [200, 300], 32, 16, 2, 256),  # a page holds a whole 32-key tile
        ([300, 513], [100, 513], 48, 8, 2, 128),  # page 48: tiles of 64 keys straddle pages
        ([129, 64], [65, 64], 16, 8, 8, 128),  # four 16-row groups per 64-key tile
    ],
)
def test_paged_prefill(dev, ctx, new, page, Hq, Hkv, Dh):
    case = paged_case(ctx, new, page=page, seed=len(ctx) + page, Hq=Hq, Hkv=Hkv, D=Dh)
    print(f"paged prefill ctx={ctx} new={new} page={page} Hq={Hq} Hkv={Hkv} D={Dh}", flush=True)
    out = paged_flash_attention_prefill(case.q.to(dev), case.k_cache.to(dev), case.v_cache.to(dev),
                                        case.block_tables.to(dev), case.context_lens.to(dev), case.cu.to(dev),
                                        None, case.scale, page).cpu()
    ref = paged_attention_ref(case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens, case.cu,
                              case.scale)
    assert_attn_close(out, ref)


def test_paged_prefill_int64_table(dev):
    case = paged_case([300, 77], [150, 77], page=16, seed=11, Hq=16, Hkv=2, D=256)
    tab = case.block_tables.to(torch.int64)
    print("paged prefill int64 block table", flush=True)
    out = paged_flash_attention_prefill(case.q.to(dev), case.k_cache.to(dev), case.v_cache.to(dev), tab.to(dev),
                                        case.context_lens.to(dev), case.cu.to(dev), None, case.scale, 16).cpu()
    ref = paged_attention_ref(case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens, case.cu,
                              case.scale)
    assert_attn_close(out, ref)


def test_paged_prefill_workload_sampled_rows(dev):
    """The chunked-prefill workload over the paged cache (16 sequences, cached
    prefixes U[0, 4096], new chunks U[256, 2048], 16-token pages, Hq 16, Hkv 2,
    D 256): every sequence's first, last and 14 random new rows vs the oracle."""
    case = attn_paged_prefill_case()
    print(f"paged prefill workload T={case.q.shape[0]}", flush=True)
    out = paged_flash_attention_prefill(case.q.to(dev), case.k_cache.to(dev), case.v_cache.to(dev),
                                        case.block_tables.to(dev), case.context_lens.to(dev), case.cu.to(dev),
                                        None, case.scale, case.page, max_seqlen=case.max_len).cpu()
    g = torch.Generator().manual_seed(8)
    cu = case.cu.tolist()
    for n in range(len(cu) - 1):
        s, e = cu[n], cu[n + 1]
        L = int(case.context_lens[n])
        k = gather_paged(case.k_cache, case.block_tables[n], L)
        v = gather_paged(case.v_cache, case.block_tables[n], L)
        rows = torch.cat([torch.tensor([0, e - s - 1]), torch.randint(0, e - s, (14,), generator=g)])
        ref = attention_rows_ref(case.q[s + rows], k, v, rows + (L - (e - s)), case.scale, causal=True)
        assert_attn_close(out[s + rows], ref)


def _decode(case, dev, splits):
    return paged_flash_attention_decode(case.q.to(dev), case.k_cache.to(dev), case.v_cache.to(dev),
                                        case.block_tables.to(dev), case.context_lens.to(dev), case.scale, case.page,
                                        num_splits=splits).cpu()


def _decode_ref(case):
    ref = torch.zeros(case.q.shape, dtype=torch.float64)
    for b in range(case.q.shape[0]):
        L = int(case.context_lens[b])
        if L == 0:
            continue
        k = gather_paged(case.k_cache, case.block_tables[b], L)
        v = gather_paged(case.v_cache, case.block_tables[b], L)
        ref[b:b + 1] = attention_rows_ref(case.q[b:b + 1], k, v, [L - 1], case.scale, causal=True)
    return ref


@pytest.mark.parametrize("splits", [1, 4, 7])
@pytest.mark.parametrize(
    "ctx, Hq, Hkv, Dh, page",
    [
        ([1, 17, 300, 0, 64], 16, 2, 256, 16),
        ([33, 500], 4, 4, 128, 16),
        ([129, 16, 3], 64, 2, 64, 32),  # 32 query heads per kv head: two head groups
    ],
)
def test_paged_decode(dev, ctx, Hq, Hkv, Dh, page, splits):
    case = paged_case(ctx, [1] * len(ctx), page=page, seed=Dh + len(ctx), Hq=Hq, Hkv=Hkv, D=Dh)
    print(f"paged decode ctx={ctx} Hq={Hq} Hkv={Hkv} D={Dh} page={page} splits={splits}", flush=True)
    out = _decode(case, dev, splits)
    assert_attn_close(out, _decode_ref(case))
    assert (out[torch.tensor(ctx) == 0] == 0).all()


@pytest.mark.parametrize(
    "label, ctx, splits, page, D",
    [
        # one long sequence among many short ones: units cross many sequence
        # ends and the long one spans many units
        ("skewed", [5000] + [int(x) for x in torch.randint(1, 41, (300,), generator=torch.Generator().manual_seed(5))], 3,
         16, 64),
        # more than 1,024 sequences: the price prefix comes from its own launch
        ("b1100", [int(x) for x in torch.randint(0, 70, (1100,), generator=torch.Generator().manual_seed(6))], 2, 16, 64),
        # fewer priced tiles than units: empty units, sequences without keys
        ("sparse", [1, 0, 0, 2, 0, 33], 16, 16, 64),
        # pages that are not a multiple of 16 (rows looked up one by one) and
        # pages of 48 (three tiles per page), head dim 256
        ("page7", [700, 3, 0, 129, 1000, 31], 3, 7, 256),
        ("page48", [700, 3, 0, 129, 1000, 31], 3, 48, 256),
    ],
)
def test_paged_decode_balanced_units(dev, label, ctx, splits, page, D):
    """Split decode over units that each take an equal share of the batch's
    priced tiles, checked against the float64 reference on every row."""
    case = paged_case(ctx, [1] * len(ctx), page=page, seed=len(ctx), Hq=8, Hkv=2, D=D)
    print(f"paged decode balanced units {label}: B={len(ctx)} splits={splits} page={page} D={D}", flush=True)
    out = _decode(case, dev, splits)
    assert_attn_close(out, _decode_ref(case))
    assert (out[torch.tensor(ctx) == 0] == 0).all()


@pytest.mark.parametrize("B, splits", [(6, 1), (6, 3), (1100, 2)])
def test_paged_decode_int64_indices(dev, B, splits):
    """int64 block tables and context lengths: one split, units priced by the
    decode waves (6 sequences) and by the separate prefix launch (1,100)."""
    gen = torch.Generator().manual_seed(B + splits)
    ctx = torch.randint(0, 300, (B,), generator=gen).tolist()
    case = paged_case(ctx, [1] * B, page=16, seed=B, Hq=8, Hkv=2, D=128)
    case.block_tables = case.block_tables.to(torch.int64)
    case.context_lens = case.context_lens.to(torch.int64)
    print(f"paged decode int64 indices B={B} splits={splits}", flush=True)
    out = _decode(case, dev, splits)
    assert_attn_close(out, _decode_ref(case))


def test_paged_decode_equals_paged_prefill_of_one_token(dev):
    case = paged_case([90, 33], [1, 1], seed=3, Hq=8, Hkv=2, D=128)
    a = _decode(case, dev, 3)
    b = paged_flash_attention_prefill(case.q.to(dev), case.k_cache.to(dev), case.v_cache.to(dev),
                                      case.block_tables.to(dev), case.context_lens.to(dev), case.cu.to(dev), None,
                                      case.scale, case.page).cpu()
    assert_out_close(a, b.double(), rtol=1e-2, atol=4e-3)


def test_paged_decode_layer_workload(dev):
    """Batch 256, contexts uniform in [512, 4096], Hq 16, Hkv 2, D 256, in full."""
    case = attn_decode_case()
    print(f"attn decode workload B=256 keys={int(case.context_lens.sum())}", flush=True)
    out = _decode(case, dev, None)
    assert_attn_close(out, _decode_ref(case))


@pytest.mark.parametrize("Dh, causal", [(72, False), (72, True), (40, True), (200, False)])
def test_varlen_prefill_other_head_dims(dev, Dh, causal):
    """Head dims without a kernel instantiation, such as the vision tower's
    1152 / 16 = 72 (models/qwen/vision.py:18, non-causal), run zero-padded to
    the next of 64, 128 and 256; against the oracle at the unpadded dim."""
    case = attn_varlen_case([100, 37, 1], seed=Dh, Hq=16, Hkv=16, D=Dh)
    print(f"varlen head dim {Dh} causal={causal}", flush=True)
    out = _varlen(case, dev, causal)
    ref = flash_attention_prefill_ref(case.q, case.k, case.v, case.cu, case.scale, is_causal=causal)
    assert out.shape == case.q.shape
    assert_attn_close(out, ref)

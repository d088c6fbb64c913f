"""GPU test of paged_attention_decode_noalloc, the paged decode entry that
allocates nothing (its split partials live in the library's static device
array): through the C ABI it must give exactly what paged_attention_decode
gives with a caller workspace and the same split count, on two calls in a row
(the second on a smaller batch, so it runs over what the first left in the
array), and a call that needs more than the array holds must be refused.
"""
import pytest
import torch

from myvllm_amd import _lib
from myvllm_amd.full_attention import paged_flash_attention_decode, paged_flash_attention_decode_noalloc
from myvllm_amd.workloads import paged_case

pytestmark = pytest.mark.gpu


def _run_both(case, dev, splits):
    q, kc, vc = case.q.to(dev), case.k_cache.to(dev), case.v_cache.to(dev)
    tab, ctx = case.block_tables.to(dev), case.context_lens.to(dev)
    page = kc.shape[1]
    ref = paged_flash_attention_decode(q, kc, vc, tab, ctx, case.scale, page, num_splits=splits)
    out = torch.full_like(q, float("nan"))
    paged_flash_attention_decode_noalloc(q, kc, vc, tab, ctx, case.scale, page, splits, out)
    torch.cuda.synchronize()
    return out.cpu(), ref.cpu()


@pytest.mark.parametrize("splits", [1, 3, 8])
def test_noalloc_decode_equals_workspace_decode_twice(dev, splits):
    gen = torch.Generator().manual_seed(11)
    ctx_big = torch.randint(0, 901, (24,), generator=gen).tolist()
    ctx_small = torch.randint(1, 301, (5,), generator=gen).tolist()
    big = paged_case(ctx_big, [1] * 24, page=16, seed=11, Hq=16, Hkv=2, D=256)
    small = paged_case(ctx_small, [1] * 5, page=16, seed=12, Hq=8, Hkv=2, D=128)
    for name, case in (("first (B=24, D=256)", big), ("second (B=5, D=128)", small)):
        print(f"noalloc decode splits={splits} {name}", flush=True)
        out, ref = _run_both(case, dev, splits)
        assert torch.equal(out, ref), f"{name}: max |diff| {(out.float() - ref.float()).abs().max().item()}"


def test_noalloc_decode_refuses_more_than_the_static_scratch(dev):
    # 64 x 64 query heads x 256 splits x (256 + 4) fp32 partials > GDN_DECODE_SCRATCH_FLOATS
    B, Hq, Hkv, Dh = 64, 64, 8, 256
    q = torch.zeros(B, Hq, Dh, dtype=torch.bfloat16, device=dev)
    kc = torch.zeros(4, 16, Hkv, Dh, dtype=torch.bfloat16, device=dev)
    tab = torch.zeros(B, 4, dtype=torch.int32, device=dev)
    ctx = torch.ones(B, dtype=torch.int32, device=dev)
    out = torch.zeros_like(q)
    with pytest.raises(_lib.GdnError) as err:
        paged_flash_attention_decode_noalloc(q, kc, kc, tab, ctx, 1.0, 16, 256, out)
    assert err.value.code == -12

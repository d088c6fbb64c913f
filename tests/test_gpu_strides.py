"""GPU: the ops accept any strided input, as the reference passes every
stride to its kernels (ops/gated_delta_rule/fused_recurrent_gdn.py:120-126,
ops/causal_conv1d.py:242-245).  Views whose rows are not 16-byte aligned
(an element of offset, odd token strides) are copied to contiguous tensors
by the Python ops, and an `out` the kernel cannot write with 16-byte stores
is filled through a temporary; the results equal the contiguous runs bit for
bit."""
import pytest
import torch

from myvllm_amd import (causal_conv1d_fn, chunk_gated_delta_rule, flash_attention_prefill,
                        paged_flash_attention_decode)
from myvllm_amd.workloads import attn_varlen_case, conv_prefill_case, paged_case, prefill_case

pytestmark = pytest.mark.gpu


def _misaligned(t: torch.Tensor) -> torch.Tensor:
    """The same values in a view one element into a wider buffer (rows not 16-byte aligned)."""
    buf = torch.zeros(t.shape[:-1] + (t.shape[-1] + 3,), dtype=t.dtype, device=t.device)
    v = buf[..., 1:1 + t.shape[-1]]
    v.copy_(t)
    assert v.data_ptr() % 16 != 0
    return v


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prefill_misaligned_views(dev, dtype):
    case = prefill_case([90, 40], seed=71, num_slots=3, Hk=2, Hv=4, dtype=dtype)
    args = [t.to(dev) for t in (case.q, case.k, case.v, case.g, case.beta)]
    st_a, st_b = case.state.to(dev), case.state.to(dev)
    idx, cu = case.idx.to(dev), case.cu.to(dev)
    o_a = chunk_gated_delta_rule(*args, st_a, idx, cu)
    q, k, v = (_misaligned(t) for t in args[:3])
    out = _misaligned(torch.zeros(case.v.shape, dtype=dtype, device=dev))
    o_b = chunk_gated_delta_rule(q, k, v, args[3], args[4], st_b, idx, cu, out=out)
    torch.cuda.synchronize()
    assert o_b is out
    assert torch.equal(o_a.cpu(), out.cpu())
    assert torch.equal(st_a.cpu(), st_b.cpu())


def test_conv_misaligned_view(dev):
    case = conv_prefill_case([50, 31], seed=72, D=256, W=4, num_slots=3)
    w, idx, cu = case.weight.to(dev), case.idx.to(dev), case.cu.to(dev)
    st_a, st_b = case.state.to(dev), case.state.to(dev)
    y_a = causal_conv1d_fn(case.x.to(dev), w, st_a, idx, cu)
    y_b = causal_conv1d_fn(_misaligned(case.x.to(dev)), w, st_b, idx, cu)
    torch.cuda.synchronize()
    assert torch.equal(y_a.cpu(), y_b.cpu())
    assert torch.equal(st_a.cpu(), st_b.cpu())


def test_attention_misaligned_views(dev):
    c = attn_varlen_case([70, 33], seed=73, Hq=8, Hkv=2, D=128)
    q, k, v, cu = (t.to(dev) for t in (c.q, c.k, c.v, c.cu))
    o_a = flash_attention_prefill(q, k, v, cu, c.scale, 8, 2, 128, 128, True)
    out = _misaligned(torch.zeros(q.shape, dtype=q.dtype, device=dev))
    o_b = flash_attention_prefill(_misaligned(q), _misaligned(k), _misaligned(v), cu, c.scale, 8, 2, 128, 128, True,
                                  out=out)
    torch.cuda.synchronize()
    assert o_b is out
    assert torch.equal(o_a.cpu(), out.cpu())
    pc = paged_case([300, 77], [1, 1], page=16, seed=74, Hq=8, Hkv=2, D=128)
    args = [t.to(dev) for t in (pc.k_cache, pc.v_cache, pc.block_tables, pc.context_lens)]
    d_a = paged_flash_attention_decode(pc.q.to(dev), *args, pc.scale, pc.page, num_splits=2)
    d_b = paged_flash_attention_decode(_misaligned(pc.q.to(dev)), *args, pc.scale, pc.page, num_splits=2)
    torch.cuda.synchronize()
    assert torch.equal(d_a.cpu(), d_b.cpu())

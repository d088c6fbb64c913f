"""GPU: the chunked prefill's output contract and options.

* Rows of tokens no sequence covers (cu_seqlens[-1] < T) come back exactly
  zero, as the reference allocates its outputs zero-filled
  (ops/gated_delta_rule/o.py:147, ops/causal_conv1d.py:241,
  ops/full_attention.py:467); checked on outputs pre-filled with NaN.
* gdn_chunk_prefill_ex's flags (zero initial state, state added into the
  slot, o added into an fp32 out) against the oracle.
* A skewed batch (many one-chunk sequences and one long one) through the
  launcher's own schedule.
* fp32 q/k/v with large and mixed-magnitude states: o keeps the fp32 range.
"""
import pytest
import torch

from conftest import assert_out_close, assert_state_close
from myvllm_amd import _lib, causal_conv1d_fn, chunk_gated_delta_rule, paged_flash_attention_prefill
from myvllm_amd.gated_delta_rule import chunk_prefill_ex
from myvllm_amd.workloads import conv_prefill_case, cu_from_lengths, paged_case, prefill_case
from oracle.gdn import chunk_gated_delta_rule_ref

from test_gpu_prefill import _check, _run

pytestmark = pytest.mark.gpu


def _short_cu(cu: torch.Tensor, drop: int) -> torch.Tensor:
    """The same sequences with the last one `drop` tokens shorter: those tokens are covered by no sequence."""
    cu = cu.clone()
    cu[-1] -= drop
    return cu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("items_per_wg", [None, 0, 3])
def test_prefill_uncovered_rows_are_zero(dev, dtype, items_per_wg):
    """cu_seqlens[-1] < T: the tokens past it get o = 0 exactly, whether the
    op allocates o or writes into a given one (NaN-filled here), under both
    schedules; the covered tokens and the states meet the usual bars."""
    case = prefill_case([70, 130, 90], seed=51, num_slots=5, Hk=2, Hv=4, dtype=dtype)
    cu = _short_cu(case.cu, 50)
    end = int(cu[-1])
    print(f"prefill uncovered rows {dtype} schedule {items_per_wg}: tokens {end}..{case.tokens}", flush=True)
    o, st, o_ref, st_ref = _run(case, dev, cu=cu, items_per_wg=items_per_wg)
    assert torch.count_nonzero(o[end:].float()) == 0
    assert not torch.isnan(o[end:].float()).any()
    assert_out_close(o[:end], o_ref[:end])
    sel = case.idx.long()
    assert_state_close(st[sel], st_ref[sel])
    if items_per_wg is None:
        # and into a caller's NaN-filled out through the public op
        st2 = case.state.to(dev)
        out = torch.full(case.v.shape, float("nan"), dtype=dtype, device=dev)
        chunk_gated_delta_rule(case.q.to(dev), case.k.to(dev), case.v.to(dev), case.g.to(dev), case.beta.to(dev), st2,
                               case.idx.to(dev), cu.to(dev), out=out)
        torch.cuda.synchronize()
        assert torch.count_nonzero(out[end:].float().cpu()) == 0
        assert torch.equal(out.cpu(), o)


def test_prefill_no_sequences_zero_all_rows(dev):
    """No sequence at all (cu = [0]): every output row is zero, no slot touched."""
    case = prefill_case([40], seed=52, num_slots=2, Hk=2, Hv=4)
    st = case.state.to(dev)
    out = torch.full(case.v.shape, float("nan"), dtype=case.v.dtype, device=dev)
    chunk_gated_delta_rule(case.q.to(dev), case.k.to(dev), case.v.to(dev), case.g.to(dev), case.beta.to(dev), st,
                           case.idx[:0].to(dev), torch.zeros(1, dtype=torch.int32, device=dev), out=out)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out.float().cpu()) == 0
    assert torch.equal(st.cpu(), case.state)


def test_prefill_fp32_uncovered_rows_are_zero(dev):
    """The fp32 route (two launches, the second adding into o) leaves
    uncovered rows at zero as well."""
    case = prefill_case([60, 100], seed=53, num_slots=3, Hk=2, Hv=4, dtype=torch.float32)
    cu = _short_cu(case.cu, 30)
    end = int(cu[-1])
    st = case.state.to(dev)
    out = torch.full(case.v.shape, float("nan"), dtype=torch.float32, device=dev)
    chunk_gated_delta_rule(case.q.to(dev), case.k.to(dev), case.v.to(dev), case.g.to(dev), case.beta.to(dev), st,
                           case.idx.to(dev), cu.to(dev), out=out)
    torch.cuda.synchronize()
    o = out.cpu()
    assert torch.count_nonzero(o[end:]) == 0
    st_ref = case.state.clone()
    o_ref = chunk_gated_delta_rule_ref(case.q, case.k, case.v, case.g, case.beta, st_ref, case.idx, cu)
    assert_out_close(o[:end], o_ref[:end], rtol=2e-3, atol=1e-3)


def test_conv_uncovered_rows_are_zero(dev):
    """causal_conv1d_fn with cu_seqlens[-1] < T: y = 0 past it (the reference
    allocates y zero-filled, ops/causal_conv1d.py:241)."""
    case = conv_prefill_case([50, 90, 33], seed=54, D=256, W=4, num_slots=5)
    cu = _short_cu(case.cu, 20)
    end = int(cu[-1])
    x = case.x.to(dev)
    y = causal_conv1d_fn(x, case.weight.to(dev), case.state.to(dev), case.idx.to(dev), cu.to(dev))
    torch.cuda.synchronize()
    y = y.cpu()
    assert torch.count_nonzero(y[end:].float()) == 0
    y_full = causal_conv1d_fn(x, case.weight.to(dev), case.state.to(dev), case.idx.to(dev), case.cu.to(dev)).cpu()
    assert torch.equal(y[:end], y_full[:end])


def test_paged_attention_prefill_uncovered_rows_are_zero(dev):
    """paged_flash_attention_prefill with cu_seqlens[-1] < T: o = 0 past it
    (the reference allocates o zero-filled, ops/full_attention.py:467)."""
    pc = paged_case([120, 60, 90], [70, 60, 40], page=16, seed=55, Hq=8, Hkv=2, D=128)
    cu = _short_cu(pc.cu, 5)
    ctx = pc.context_lens.clone()
    ctx[-1] -= 5  # the shortened last sequence's queries still end at its last cached key
    end = int(cu[-1])
    o = paged_flash_attention_prefill(pc.q.to(dev), pc.k_cache.to(dev), pc.v_cache.to(dev), pc.block_tables.to(dev),
                                      ctx.to(dev), cu.to(dev), None, pc.scale, pc.page)
    torch.cuda.synchronize()
    assert torch.count_nonzero(o[end:].float().cpu()) == 0


def test_prefill_ex_flags(dev):
    """gdn_chunk_prefill_ex: ZERO_INIT runs from a zero state (the slot is
    not read), ACCUM_STATE adds the final state to the slot, ACCUM_OUT adds o
    to an fp32 out.  Reference: the oracle from a zero state; the slot must
    end as its old value plus that final state, out as its old value plus o."""
    case = prefill_case([100, 64, 1], seed=56, num_slots=5, Hk=2, Hv=4, dtype=torch.float16)
    scale = case.q.shape[-1] ** -0.5
    zero = torch.zeros_like(case.state)
    o_zero = chunk_gated_delta_rule_ref(case.q, case.k, case.v, case.g, case.beta, zero, case.idx, case.cu)
    st = case.state.to(dev)
    base = torch.randn(case.v.shape, generator=torch.Generator().manual_seed(57))
    out = base.to(dev)
    flags = _lib.PREFILL_ZERO_INIT | _lib.PREFILL_ACCUM_STATE | _lib.PREFILL_ACCUM_OUT
    chunk_prefill_ex(case.q.to(dev), case.k.to(dev), case.v.to(dev), case.g.to(dev), case.beta.to(dev), st,
                     case.idx.to(dev), case.cu.to(dev), out, scale, flags=flags)
    torch.cuda.synchronize()
    assert_out_close(out.cpu() - base, o_zero)
    sel = case.idx.long()
    assert_state_close(st.cpu()[sel] - case.state[sel], zero[sel])
    untouched = torch.ones(case.state.shape[0], dtype=torch.bool)
    untouched[sel] = False
    assert torch.equal(st.cpu()[untouched], case.state[untouched])
    # ZERO_INIT alone: the slot is replaced by the zero-start final state
    st = case.state.to(dev)
    o = torch.empty(case.v.shape, dtype=torch.float16, device=dev)
    chunk_prefill_ex(case.q.to(dev), case.k.to(dev), case.v.to(dev), case.g.to(dev), case.beta.to(dev), st,
                     case.idx.to(dev), case.cu.to(dev), o, scale, flags=_lib.PREFILL_ZERO_INIT)
    torch.cuda.synchronize()
    assert_out_close(o.cpu(), o_zero)
    assert_state_close(st.cpu()[sel], zero[sel])


def test_prefill_ex_rejects_bad_options(dev):
    """Unknown flags or out-of-range options return GDN_ERR_ARG; ACCUM_OUT on a
    16-bit out and an fp32 out for bf16 inputs return GDN_ERR_DTYPE; nothing
    is launched."""
    case = prefill_case([10], seed=58, num_slots=1, Hk=1, Hv=1)
    args = [t.to(dev) for t in (case.q, case.k, case.v, case.g, case.beta, case.state, case.idx, case.cu)]
    o16 = torch.empty(case.v.shape, dtype=torch.bfloat16, device=dev)
    o32 = torch.empty(case.v.shape, dtype=torch.float32, device=dev)
    for kw, out, code in ((dict(flags=8), o16, -13), (dict(items_per_wg=65), o16, -13), (dict(spin_limit=-2), o16, -13),
                          (dict(flags=_lib.PREFILL_ACCUM_OUT), o16, -4), (dict(), o32, -4)):
        with pytest.raises(_lib.GdnError) as e:
            chunk_prefill_ex(*args, out, 0.1, **kw)
        assert e.value.code == code, (kw, e.value.code)
    assert torch.equal(args[5].cpu(), case.state)


def test_prefill_skewed_batch_auto_schedule(dev):
    """384 one-chunk sequences and one 16,384-token sequence (a chunked-prefill
    scheduler's batch with one long prompt chunk): the launcher takes the
    many-items schedule, whose runs are priced by tokens, so the long
    sequence's items spread over workgroups.  Parity against the oracle."""
    lengths = [64] * 384 + [16384]
    case = prefill_case(lengths, seed=59, num_slots=400, Hk=1, Hv=2)
    print(f"prefill skewed batch: {case.tokens} tokens, {len(lengths)} sequences", flush=True)
    o, st, o_ref, st_ref = _run(case, dev)
    _check(case, o, st, o_ref, st_ref)


@pytest.mark.parametrize("state_scale", ["large", "mixed"])
def test_prefill_fp32_state_magnitudes(dev, state_scale):
    """fp32 q/k/v with a 1e7 state and with per-column states from 1e-15 to
    1e15: |o| reaches ~1e5 and beyond, past fp16's range, and must come back
    finite (the fp32 route writes o in fp32).  Compared in units of the
    column's scale where it exceeds 1, at the fp32 route's bars."""
    case = prefill_case([200, 70], seed=60, num_slots=3, Hk=2, Hv=4, g_scale=0.05, dtype=torch.float32)
    col = torch.ones(case.state.shape[-1], dtype=torch.float64)
    if state_scale == "large":
        case.state.mul_(1e7)
        col.fill_(1e7)
    else:
        col = torch.logspace(-15, 15, case.state.shape[-1], dtype=torch.float64)
        case.state.mul_(col.float())
    o, st, o_ref, st_ref = _run(case, dev)
    assert torch.isfinite(o).all()
    assert o.abs().max().item() > 65504.0
    unit = col.clamp_min(1.0)
    assert_out_close(o.double() / unit, o_ref.double() / unit, rtol=2e-3, atol=1e-3)
    sel = case.idx.long()
    rel = ((st[sel].double() - st_ref[sel]) / unit).norm() / (st_ref[sel] / unit).norm()
    assert rel.item() < 1e-3, rel.item()

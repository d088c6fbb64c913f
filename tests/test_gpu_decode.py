"""GPU parity: fused recurrent decode step vs the CPU oracle (token recurrence, fp64)."""
import pytest
import torch

from conftest import assert_out_close, assert_state_close
from myvllm_amd import recurrent_gated_delta_rule
from myvllm_amd.workloads import decode_case
from oracle.gdn import recurrent_gated_delta_rule_ref

pytestmark = pytest.mark.gpu


def _run(case, dev, idx=None, beta=None):
    idx = case.idx if idx is None else idx
    beta = case.beta if beta is None else beta
    st_ref = case.state.clone()
    o_ref = recurrent_gated_delta_rule_ref(case.q, case.k, case.v, case.g, beta, st_ref, idx)
    st = case.state.to(dev)
    o = recurrent_gated_delta_rule(
        case.q.to(dev), case.k.to(dev), case.v.to(dev), case.g.to(dev), beta.to(dev), st, idx.to(dev)
    )
    torch.cuda.synchronize()
    return o, st.cpu(), o_ref, st_ref


@pytest.mark.parametrize("K", [128, 64])
def test_decode_small(dev, K):
    case = decode_case(B=8, num_slots=16, seed=1, K=K, V=K)
    o, st, o_ref, st_ref = _run(case, dev)
    assert_out_close(o, o_ref)
    assert_state_close(st, st_ref)
    untouched = torch.ones(16, dtype=torch.bool)
    untouched[case.idx.long()] = False
    assert torch.equal(st[untouched], case.state[untouched])


@pytest.mark.parametrize("K, V", [(32, 32), (128, 64), (64, 128), (96, 40), (8, 8), (256, 256), (192, 256),
                                  (256, 136), (136, 72), (8, 256)])
def test_decode_other_head_dims(dev, K, V):
    """Head dims other than 64 x 64 and 128 x 128 (multiples of 8) run
    zero-padded in the 128 x 128 kernel, or in the 256 x 256 one when either
    exceeds 128 (the reference's decode kernel has no head-dim cap,
    ops/gated_delta_rule/fused_recurrent_gdn.py:51-58); a padding slot among them."""
    case = decode_case(B=7, num_slots=12, seed=K + V, Hk=2, Hv=4, K=K, V=V)
    idx = case.idx.clone()
    idx[3] = -1
    print(f"decode head dims K={K} V={V}", flush=True)
    o, st, o_ref, st_ref = _run(case, dev, idx=idx)
    assert torch.count_nonzero(o[3]) == 0
    assert_out_close(o, o_ref)
    assert_state_close(st, st_ref)
    untouched = torch.ones(12, dtype=torch.bool)
    untouched[[int(i) for i in idx.tolist() if i >= 0]] = False
    assert torch.equal(st[untouched], case.state[untouched])


def test_decode_fp32_inputs_bf16_beta(dev):
    case = decode_case(B=5, num_slots=9, seed=2, dtype=torch.float32, beta_dtype=torch.bfloat16)
    o, st, o_ref, st_ref = _run(case, dev)
    assert o.dtype == torch.float32
    assert_out_close(o, o_ref, rtol=1e-4, atol=1e-5)
    assert_state_close(st, st_ref)


def test_decode_padding_and_int64_slots(dev):
    case = decode_case(B=6, num_slots=8, seed=3)
    idx = case.idx.clone().long()
    idx[1] = -1
    idx[4] = 8  # == num_slots: out of range, also padding
    o, st, o_ref, st_ref = _run(case, dev, idx=idx)
    assert torch.count_nonzero(o[1]) == 0 and torch.count_nonzero(o[4]) == 0
    assert_out_close(o, o_ref)
    assert_state_close(st, st_ref)
    touched = torch.zeros(8, dtype=torch.bool)
    touched[[int(i) for i in idx.tolist() if 0 <= i < 8]] = True
    assert torch.equal(st[~touched], case.state[~touched])


def test_decode_strided_views(dev):
    """q/k/v as head-split views of one packed projection (layer layout)."""
    case = decode_case(B=7, num_slots=10, seed=4)
    B = 7
    packed = torch.cat([case.q.reshape(B, -1), case.k.reshape(B, -1), case.v.reshape(B, -1)], 1).to(dev)
    qd, kd, vd = torch.split(packed, [16 * 128, 16 * 128, 32 * 128], dim=1)
    qd, kd, vd = qd.view(B, 16, 128), kd.view(B, 16, 128), vd.view(B, 32, 128)
    assert not vd.is_contiguous()
    st_ref = case.state.clone()
    o_ref = recurrent_gated_delta_rule_ref(case.q, case.k, case.v, case.g, case.beta, st_ref, case.idx)
    st = case.state.to(dev)
    o = recurrent_gated_delta_rule(qd, kd, vd, case.g.to(dev), case.beta.to(dev), st, case.idx.to(dev))
    assert_out_close(o, o_ref)
    assert_state_close(st.cpu(), st_ref)


def test_decode_batch256_full(dev):
    """Benchmark shape: B=256 from a 1024-slot fp32 cache (2 GiB), untouched slots bit-identical."""
    case = decode_case(B=256, num_slots=1024, seed=0)
    o, st, o_ref, st_ref = _run(case, dev)
    assert_out_close(o, o_ref)
    sel = case.idx.long()
    assert_state_close(st[sel], st_ref[sel])
    untouched = torch.ones(1024, dtype=torch.bool)
    untouched[sel] = False
    assert torch.equal(st[untouched], case.state[untouched])


@pytest.mark.parametrize("Hk, Hv", [(1, 3), (2, 2), (3, 6)])
def test_decode_head_pairing(dev, Hk, Hv):
    """Odd Hv (one v-head per workgroup) and GVA ratios 1 and 2 with paired v-heads."""
    case = decode_case(B=5, num_slots=7, seed=11, Hk=Hk, Hv=Hv)
    o, st, o_ref, st_ref = _run(case, dev)
    assert_out_close(o, o_ref)
    assert_state_close(st, st_ref)

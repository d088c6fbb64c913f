"""GPU parity: fused decode step (conv update + L2 norm + gating + recurrent step)
vs the fp64 composition of the oracle pieces (oracle.layer.gdn_decode_step_ref)."""
import pytest
import torch

from conftest import assert_out_close, assert_state_close
from myvllm_amd import gated_delta_net_decode_step
from myvllm_amd.workloads import decode_fused_case
from oracle.layer import gdn_decode_step_ref

pytestmark = pytest.mark.gpu


def _run(case, dev, cidx=None, idx=None, steps=1):
    cidx = case.conv_idx if cidx is None else cidx
    idx = case.idx if idx is None else idx
    cs_ref, st_ref = case.conv_state.clone(), case.state.clone()
    cs, st = case.conv_state.to(dev), case.state.to(dev)
    outs, refs = [], []
    for s in range(steps):
        x = case.mixed_qkv if s == 0 else torch.roll(case.mixed_qkv, s, dims=1)
        refs.append(gdn_decode_step_ref(x, case.conv_weight, cs_ref, cidx, case.a, case.b, case.A_log,
                                        case.dt_bias, st_ref, idx, case.Hk))
        outs.append(gated_delta_net_decode_step(
            x.to(dev), case.conv_weight.to(dev), cs, cidx.to(dev), case.a.to(dev), case.b.to(dev),
            case.A_log.to(dev), case.dt_bias.to(dev), st, idx.to(dev), case.Hk).cpu())
    torch.cuda.synchronize()
    return outs, refs, cs.cpu(), cs_ref, st.cpu(), st_ref


def _check(outs, refs, cs, cs_ref, st, st_ref):
    for o, r in zip(outs, refs):
        assert_out_close(o, r)
    # the conv state is a shift of stored values: bit-exact
    assert torch.equal(cs, cs_ref)
    assert_state_close(st, st_ref)


@pytest.mark.parametrize("Hk,Hv", [(2, 4), (4, 4), (1, 4)])
def test_fused_decode_head_ratios(dev, Hk, Hv):
    case = decode_fused_case(B=6, num_slots=9, seed=Hv * 10 + Hk, Hk=Hk, Hv=Hv)
    _check(*_run(case, dev))


def test_fused_decode_three_steps_carry_both_states(dev):
    case = decode_fused_case(B=5, num_slots=7, seed=3, Hk=2, Hv=4)
    _check(*_run(case, dev, steps=3))


def test_fused_decode_padding_slots_and_int64(dev):
    case = decode_fused_case(B=6, num_slots=8, seed=4, Hk=2, Hv=4)
    cidx = case.conv_idx.clone().long()
    idx = case.idx.clone().long()
    cidx[1] = -1   # conv padding, state slot valid: zero conv output, the state still decays
    idx[2] = 99    # state padding, conv slot valid: zero output, the conv state still advances
    cidx[4] = -3
    idx[4] = -3    # both padding
    outs, refs, cs, cs_ref, st, st_ref = _run(case, dev, cidx=cidx, idx=idx)
    _check(outs, refs, cs, cs_ref, st, st_ref)
    assert torch.count_nonzero(outs[0][2]) == 0 and torch.count_nonzero(outs[0][4]) == 0
    untouched = [s for s in range(8) if s not in set(idx.tolist())]
    assert torch.equal(st[untouched], case.state[untouched])


@pytest.mark.parametrize("dtype,cs_dtype,w_dtype", [(torch.float16, torch.float16, torch.float32),
                                                     (torch.float32, torch.float32, torch.float32),
                                                     (torch.bfloat16, torch.bfloat16, torch.bfloat16)])
def test_fused_decode_dtypes(dev, dtype, cs_dtype, w_dtype):
    case = decode_fused_case(B=4, num_slots=6, seed=5, Hk=2, Hv=4, dtype=dtype, conv_state_dtype=cs_dtype,
                             weight_dtype=w_dtype)
    _check(*_run(case, dev))


def test_fused_decode_benchmark_shape_sample(dev):
    """Hk 16, Hv 32, D 8192 (the benchmark's layer shape) on 8 sequences."""
    case = decode_fused_case(B=8, num_slots=16, seed=6)
    _check(*_run(case, dev))

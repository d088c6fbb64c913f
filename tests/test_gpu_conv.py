"""GPU parity: causal conv1d prefill/update vs the CPU oracle (F.conv1d, fp64)."""
import pytest
import torch

from conftest import assert_out_close
from myvllm_amd import causal_conv1d_fn, causal_conv1d_update
from myvllm_amd.workloads import conv_decode_case, conv_prefill_case, cu_from_lengths
from oracle.conv import causal_conv1d_fn_ref, causal_conv1d_update_ref

pytestmark = pytest.mark.gpu


def _prefill(case, dev):
    st_ref = case.state.clone()
    y_ref = causal_conv1d_fn_ref(case.x, case.weight, st_ref, case.idx, case.cu)
    st = case.state.to(dev)
    y = causal_conv1d_fn(case.x.to(dev), case.weight.to(dev), st, case.idx.to(dev), case.cu.to(dev))
    torch.cuda.synchronize()
    return y.cpu(), st.cpu(), y_ref, st_ref


@pytest.mark.parametrize("W", [2, 3, 4, 5, 6])
def test_conv_varlen_edges(dev, W):
    lengths = [0, 1, 2, 3, 5, 64, 65, 130, 0, 7]
    case = conv_prefill_case(lengths, seed=W, D=64, W=W, num_slots=16)
    y, st, y_ref, st_ref = _prefill(case, dev)
    assert_out_close(y, y_ref)
    assert torch.equal(st, st_ref)  # states are copies of inputs: bit-exact


def test_conv_varlen_padding_slot_and_int64(dev):
    lengths = [4, 70, 2]
    case = conv_prefill_case(lengths, seed=11, D=128, W=4, num_slots=8)
    case.idx = case.idx.long()
    case.idx[1] = -1
    case.cu = case.cu.long()
    y, st, y_ref, st_ref = _prefill(case, dev)
    assert torch.count_nonzero(y[4:74]) == 0
    assert_out_close(y, y_ref)
    assert torch.equal(st, st_ref)


def test_conv_varlen_bf16_state(dev):
    case = conv_prefill_case([9, 100, 3], seed=12, D=256, W=4, num_slots=4, state_dtype=torch.bfloat16)
    y, st, y_ref, st_ref = _prefill(case, dev)
    assert_out_close(y, y_ref)
    assert torch.equal(st, st_ref)


def test_conv_varlen_full_config(dev):
    """Benchmark shape: 8 sequences (19,762 tokens), 8192 channels, width 4."""
    case = conv_prefill_case()
    assert int(case.cu[-1]) == 19762
    y, st, y_ref, st_ref = _prefill(case, dev)
    assert_out_close(y, y_ref)
    assert torch.equal(st, st_ref)


def test_conv_update_batch256(dev):
    case = conv_decode_case()
    st_ref = case.state.clone()
    y_ref = causal_conv1d_update_ref(case.x, case.weight, st_ref, case.idx)
    st = case.state.to(dev)
    y = causal_conv1d_update(case.x.to(dev), case.weight.to(dev), st, case.idx.to(dev))
    assert_out_close(y, y_ref)
    assert torch.equal(st.cpu(), st_ref)


def test_conv_update_equals_one_token_prefill(dev):
    case = conv_decode_case(B=16, D=512, num_slots=32, seed=5)
    st_a = case.state.to(dev)
    st_b = case.state.to(dev)
    x = case.x.to(dev)
    y_a = causal_conv1d_update(x, case.weight.to(dev), st_a, case.idx.to(dev))
    cu = cu_from_lengths([1] * 16).to(dev)
    y_b = causal_conv1d_fn(x, case.weight.to(dev), st_b, case.idx.to(dev), cu)
    assert torch.equal(y_a, y_b)
    assert torch.equal(st_a, st_b)


def test_conv_strided_weight(dev):
    """A (D, W) weight view of a (W, D) buffer takes the element-wise tap loads."""
    case = conv_prefill_case([40, 3], seed=13, D=128, W=4, num_slots=4)
    st_ref = case.state.clone()
    y_ref = causal_conv1d_fn_ref(case.x, case.weight, st_ref, case.idx, case.cu)
    w_t = case.weight.t().contiguous().to(dev).t()
    assert w_t.stride() == (1, 128)
    st = case.state.to(dev)
    y = causal_conv1d_fn(case.x.to(dev), w_t, st, case.idx.to(dev), case.cu.to(dev))
    assert_out_close(y.cpu(), y_ref)
    assert torch.equal(st.cpu(), st_ref)
    st2 = case.state.to(dev)
    x1 = case.x[:2].to(dev)
    idx2 = case.idx.to(dev)
    y2 = causal_conv1d_update(x1, w_t, st2, idx2)
    st2_ref = case.state.clone()
    y2_ref = causal_conv1d_update_ref(case.x[:2], case.weight, st2_ref, case.idx)
    assert_out_close(y2.cpu(), y2_ref)
    assert torch.equal(st2.cpu(), st2_ref)

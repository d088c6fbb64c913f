"""GPU: gated RMSNorm (layers/norm.py:44-58) and the conv with the layer's q/k
L2 norm fused into its epilogue (layers/linear_attention.py:113-114) vs the oracle."""
import pytest
import torch

from conftest import assert_out_close
from myvllm_amd import causal_conv1d_fn
from myvllm_amd.norm import gdn_gating, rms_norm_gated
from myvllm_amd.workloads import cu_from_lengths
from oracle.conv import causal_conv1d_fn_ref
from oracle.layer import gdn_gating_ref, l2norm_ref, rms_norm_gated_ref

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_rms_norm_gated(dev, dtype):
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(37, 6, 128, generator=g) * 3).to(dtype)
    z = torch.randn(37, 6 * 128 + 64, generator=g).to(dtype)[:, 64:].view(37, 6, 128)  # strided gate, as the layer's
    w = torch.rand(128, generator=g) + 0.5
    ref = rms_norm_gated_ref(x, z, w)
    out = rms_norm_gated(x.to(dev), z.to(dev), w.to(dev)).cpu()
    if dtype == torch.float32:
        assert torch.allclose(out, ref, rtol=1e-5, atol=1e-6)
    else:
        assert_out_close(out, ref)


@pytest.mark.parametrize("N,per_head,dtype", [(64, False, torch.bfloat16), (72, False, torch.float16),
                                               (1000, False, torch.float32), (3, True, torch.bfloat16),
                                               (128, True, torch.bfloat16), (256, False, torch.bfloat16)])
def test_rms_norm_gated_any_row_length(dev, N, per_head, dtype):
    """Any normalized_shape (the reference's RMSNormGated takes one and
    reduces over its last dim, layers/norm.py:44-58): row lengths other than
    128, odd ones included, with one shared weight row or one per head, through
    the nn.Module drop-in as well."""
    from myvllm_amd.norm import RMSNormGated

    g = torch.Generator().manual_seed(N)
    x = (torch.randn(29, 5, N, generator=g) * 3).to(dtype)
    z = torch.randn(29, 5, N, generator=g).to(dtype)
    w = torch.rand((5, N) if per_head else (N,), generator=g) + 0.5
    ref = rms_norm_gated_ref(x, z, w)
    out = rms_norm_gated(x.to(dev), z.to(dev), w.to(dev)).cpu()
    if dtype == torch.float32:
        assert torch.allclose(out, ref, rtol=1e-5, atol=1e-6)
    else:
        assert_out_close(out, ref)
    m = RMSNormGated((5, N) if per_head else (N,), eps=1e-6, device=dev)
    with torch.no_grad():
        m.weight.copy_(w)
    assert torch.equal(m(x.to(dev), z.to(dev)).cpu(), out)


def test_rms_norm_gated_empty(dev):
    x = torch.zeros(0, 4, 128, dtype=torch.bfloat16, device=dev)
    assert rms_norm_gated(x, x, torch.ones(128, device=dev)).shape == (0, 4, 128)


@pytest.mark.parametrize("lengths", [[100, 37, 1], [64, 0, 130]])
def test_conv_with_fused_qk_norm(dev, lengths):
    g = torch.Generator().manual_seed(len(lengths))
    Hk, Hv = 2, 4
    D = 2 * Hk * 128 + Hv * 128
    cu = cu_from_lengths(lengths)
    T = int(cu[-1])
    x = torch.randn(T, D, generator=g).bfloat16()
    w = (torch.randn(D, 4, generator=g) * 0.5).bfloat16()
    st = torch.randn(5, 3, D, generator=g)
    idx = torch.tensor([3, 0, 4][: len(lengths)], dtype=torch.int32)
    st_ref = st.clone()
    y = causal_conv1d_fn_ref(x.double(), w, st_ref, idx, cu)  # fp64
    nrm = 2 * Hk * 128
    y[:, :nrm] = l2norm_ref(y[:, :nrm].reshape(T, 2 * Hk, 128)).reshape(T, nrm)
    st_d = st.to(dev)
    out = causal_conv1d_fn(x.to(dev), w.to(dev), st_d, idx.to(dev), cu.to(dev), l2norm_channels=nrm).cpu()
    assert_out_close(out, y)
    assert torch.equal(st_d.cpu(), st_ref)
    # q and k rows have unit norm (to bf16 rounding); v rows are the plain conv
    qk = out[:, :nrm].float().reshape(T, 2 * Hk, 128)
    assert torch.allclose(qk.pow(2).sum(-1), torch.ones(T, 2 * Hk), atol=2e-2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gating(dev, dtype):
    g = torch.Generator().manual_seed(5)
    ab = (torch.randn(33, 2 * 6 + 3, generator=g) * 4).to(dtype)  # strided a, b as the layer's views
    b, a = ab[:, :6], ab[:, 6:12]
    a[0, 0] = 30.0  # softplus past its threshold
    A_log = torch.log(torch.rand(6, generator=g) * 15 + 1)
    dt_bias = torch.rand(6, generator=g).to(dtype)
    g_ref, beta_ref = gdn_gating_ref(a, b, A_log, dt_bias, dtype=torch.float64)
    gg, beta = gdn_gating(a.to(dev), b.to(dev), A_log.to(dev), dt_bias.to(dev))
    assert torch.allclose(gg.cpu().double(), g_ref, rtol=1e-5, atol=1e-6)
    assert torch.allclose(beta.cpu().double(), beta_ref, rtol=1e-5, atol=1e-6)

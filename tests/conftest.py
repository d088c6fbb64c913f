import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD Instinct GPU (HIP device)")


@pytest.fixture(scope="session")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    return torch.device("cuda:0")


# Tolerances of the parity bar: bf16 outputs, fp32 states.
O_RTOL, O_ATOL = 2e-2, 1e-2
S_RTOL, S_ATOL = 1e-3, 1e-6


def assert_out_close(got: torch.Tensor, ref: torch.Tensor, rtol=O_RTOL, atol=O_ATOL):
    got = got.detach().float().cpu()
    ref = ref.detach().float().cpu()
    assert got.shape == ref.shape
    bad = (got - ref).abs() > atol + rtol * ref.abs()
    assert not bad.any(), (
        f"{int(bad.sum())}/{bad.numel()} outputs outside rtol={rtol}, atol={atol}; "
        f"max |diff| {(got - ref).abs().max().item():.3e}"
    )


def assert_state_close(got: torch.Tensor, ref: torch.Tensor, rtol=S_RTOL, atol=S_ATOL):
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    assert got.shape == ref.shape
    err = (got - ref).abs()
    bad = err > atol + rtol * ref.abs()
    assert not bad.any(), (
        f"{int(bad.sum())}/{bad.numel()} state elements outside |d| <= {rtol}|ref| + {atol}; "
        f"max |diff| {err.max().item():.3e}"
    )

import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu on the GPU box")


@pytest.fixture(scope="session")
def device():
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but no HIP device is visible")
    return torch.device("cuda:0")


def assert_close(actual, expected, rtol, atol, what=""):
    """Elementwise |a - e| <= atol + rtol * |e| in float64, with a message
    naming the worst element."""
    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    assert a.shape == e.shape, f"{what}: shape {tuple(a.shape)} vs {tuple(e.shape)}"
    err = (a - e).abs()
    bound = atol + rtol * e.abs()
    bad = err > bound
    if bool(bad.any()):
        idx = int(torch.argmax((err - bound).flatten()))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{a.numel()} elements out of tolerance (rtol={rtol}, atol={atol}); "
            f"worst flat index {idx}: got {a.flatten()[idx].item():.9g}, want {e.flatten()[idx].item():.9g}; "
            f"max abs err {err.max().item():.3g}, max |ref| {e.abs().max().item():.3g}")


BF16_RTOL = 2.0 ** -8  # unit roundoff of bf16 (8 significant bits): one rounding to nearest


def assert_close_bf16(actual, expected, what="", floor=1e-3):
    """A bf16-stored result against a float64 reference: one rounding to
    nearest (relative 2^-8) plus an absolute floor of `floor` * max|ref| for
    the fp32 arithmetic before the rounding and for elements near zero."""
    assert actual.dtype == torch.bfloat16, f"{what}: expected bf16 storage, got {actual.dtype}"
    assert_close(actual, expected, BF16_RTOL, grad_atol(expected, floor), what)


def grad_atol(ref: torch.Tensor, frac: float = 1e-4) -> float:
    """Absolute floor for gradient comparisons: frac * max|ref| (gradients
    summed over many tokens can have entries near zero after cancellation)."""
    return frac * float(ref.detach().abs().max().clamp_min(1e-30))

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


def assert_close_bf16(actual, expected, what="", floor=1e-3, big=1e-2):
    """A bf16-stored result against a float64 reference, in two parts.

    Every element: relative 2^-8 (one rounding to nearest) plus an absolute
    floor of `floor` * max|ref| for the fp32 arithmetic before the rounding
    and for elements near zero.  The floor dominates below about 2^8 * floor
    * max|ref|, so on its own it cannot tell one rounding from several there.

    Elements with |ref| >= `big` * max|ref|: relative only, 2^-8 + 2^-11 (one
    bf16 rounding plus fp32 arithmetic of at most 2^-11 of the element, i.e.
    about 5e-6 of max|ref| at the threshold).  A second rounding to bf16 of
    such an element (up to 2 * 2^-8) fails this part.  The bf16 dx of the
    dynamic backward is checked element by element in
    test_gpu_dx_transport.py."""
    assert actual.dtype == torch.bfloat16, f"{what}: expected bf16 storage, got {actual.dtype}"
    assert_close(actual, expected, BF16_RTOL, grad_atol(expected, floor), what)
    a = actual.detach().to("cpu", torch.float64).flatten()
    e = expected.detach().to("cpu", torch.float64).flatten()
    if big is None:
        return
    sel = e.abs() >= big * float(e.abs().max().clamp_min(1e-30))
    if bool(sel.any()):
        assert_close(a[sel], e[sel], BF16_RTOL + 2.0 ** -11, 0.0, f"{what} (|ref| >= {big} max|ref|, relative only)")


def assert_close_dyn_dx_bf16(actual, expected, what=""):
    """The bf16 dx of the dynamic layer's backward.  Its stream part travels
    between two kernels as fp16 against a power-of-two scale (11 significant
    bits), so where it cancels against the projection term an element can
    sit a little more than one bf16 rounding away: the per-element bound
    2^-8 |ref| + 2^-11 |stream part| is checked in test_gpu_dx_transport.py,
    and here the first part of assert_close_bf16 only."""
    assert_close_bf16(actual, expected, what, big=None)


def grad_atol(ref: torch.Tensor, frac: float = 1e-4) -> float:
    """Absolute floor for gradient comparisons: frac * max|ref| (gradients
    summed over many tokens can have entries near zero after cancellation)."""
    return frac * float(ref.detach().abs().max().clamp_min(1e-30))

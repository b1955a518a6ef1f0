"""Test configuration: import paths, the `gpu` marker and shared helpers.

Tests marked `gpu` run the HIP kernels on a ROCm GPU (MI355X); everything else
runs on the CPU and never launches a kernel.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mamba-cpu_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (gfx950) and runs the HIP kernels")


def gpu_available():
    import torch

    return torch.cuda.is_available()


@pytest.fixture(autouse=True)
def _skip_gpu_without_device(request):
    if request.node.get_closest_marker("gpu") is not None and not gpu_available():
        pytest.skip("needs a ROCm GPU")


# Gradient tolerances of the float32 path against the float64 oracle (or the
# reference's float32 kernels), unscaled: |got - want| <= atol + rtol |want|
# elementwise. rtol 1e-3 on every gradient. atol 1e-4 for per-element
# gradients (du, ddelta, dz); 1e-3 for gradients that are sums over the batch,
# the sequence or the channels (dA, dB, dC, dD, ddelta_bias), whose float32
# rounding grows with the number of terms: the reference's own kernels differ
# from the float64 oracle by up to 1.4e-4 on dD at the training-step shape
# (batch 8, dim 1536, seqlen 1024).
GRAD_RTOL = 1e-3
GRAD_ATOL = {"u": 1e-4, "delta": 1e-4, "z": 1e-4,
             "A": 1e-3, "B": 1e-3, "C": 1e-3, "D": 1e-3, "delta_bias": 1e-3}


def assert_close_report(got, want, rtol, atol, name=""):
    """numpy.testing.assert_allclose(got, want, rtol, atol) on float64 copies,
    printing the largest error and the worst ratio err / (atol + rtol |want|)
    so a log shows how much margin each check has (1.0 = at the bound)."""
    import numpy as np

    if hasattr(got, "detach"):
        got = got.detach().float().cpu().numpy()
    if hasattr(want, "detach"):
        want = want.detach().float().cpu().numpy()
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{name}: shape {got.shape} != {want.shape}"
    if got.size:
        err = np.abs(got - want)
        bound = atol + rtol * np.abs(want)
        with np.errstate(invalid="ignore", divide="ignore"):
            ratio = np.where(bound > 0, err / np.where(bound > 0, bound, 1.0), np.where(err > 0, np.inf, 0.0))
            ratio = np.nanmax(ratio) if np.isfinite(err).any() else float("nan")
        print(f"  {name}: max|want| {np.abs(want).max():.3g}  max err {np.nanmax(err):.3g}  "
              f"worst err/bound {ratio:.3g}", flush=True)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol, err_msg=name)

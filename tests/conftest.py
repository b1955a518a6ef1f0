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

"""pytest setup: import paths for the package (``grouped-gemms_amd``) and the
oracle, the ``gpu`` marker, and shared fixtures."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "grouped-gemms_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libmxgg.so")


def _gpu_ready() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    """Skip unless a GPU is visible; fail loudly if the native library is missing."""
    if not _gpu_ready():
        pytest.skip("no GPU visible")
    import kernels
    from kernels import _lib
    if not kernels._rocm_mxfp8_available:
        raise RuntimeError("GPU present but libmxgg.so is not loadable: build it first")
    lib = _lib.load()
    assert lib.mxgg_device_supported() == 1, "current device is not gfx950"
    import torch
    return torch.device("cuda:0")

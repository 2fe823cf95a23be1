"""Shared test configuration: the `gpu` marker, repository imports, GPU helpers."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
TESTS = os.path.dirname(os.path.abspath(__file__))
if TESTS not in sys.path:
    sys.path.insert(0, TESTS)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def hip():
    """The built torch binding module; fails loudly when the GPU or the build is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a visible GPU")
    from barqtrain_amd import _ffi

    backend = _ffi.load_cuda_backend()
    assert backend is not None, "barqtrain_cuda (HIP backend) is not built"
    return backend


@pytest.fixture(scope="session")
def capi():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected without a visible GPU")
    from barqtrain_amd import _capi

    return _capi.load_library()

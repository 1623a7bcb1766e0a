import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu_lib():
    """The product library, loaded for GPU tests; fails loudly when it is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but no GPU is visible")
    from helios_amd import qmm

    qmm.load_library()
    return qmm


@pytest.fixture
def gemm_from_32(gpu_lib):
    """Pins the GEMM path from 32 rows on for tests aimed at the GEMM: the automatic
    choice runs small weights on the decode kernels up to hundreds of rows."""
    with gpu_lib.gemm_min_rows(32):
        yield

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs with -m gpu on the GPU box)")


def _gpu_requested(config) -> bool:
    expr = config.getoption("-m") or ""
    return "gpu" in expr and "not gpu" not in expr


@pytest.fixture(scope="session")
def gpu(request):
    """One context shared by every GPU test, like the reference's OnceLock<Mutex<Gpu>>
    (crates/staleynet-cuda/tests/kernels_match_reference.rs:14-23)."""
    from staleynet_amd import gemm

    try:
        g = gemm.Gpu(0)
    except gemm.GpuError as error:
        if error.status == gemm.SN_ERR_NO_DEVICE and not _gpu_requested(request.config):
            pytest.skip("no GPU in this container")
        raise
    yield g
    g.close()

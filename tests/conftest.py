import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) GPU and the built HIP library")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


def _ensure_built():
    lib = ROOT / "turbopress_amd" / "libturbopress_amd.so"
    if not lib.exists():
        from turbopress_amd.build import build
        build()


@pytest.fixture(scope="session")
def built_lib():
    _ensure_built()
    from turbopress_amd import _lib
    return _lib.lib()


@pytest.fixture(scope="session")
def cuda():
    import torch
    _ensure_built()
    if not torch.cuda.is_available():
        pytest.fail("this test is marked gpu and needs a ROCm GPU (run with -m 'not gpu' on CPU)")
    from turbopress_amd import hip_kernel
    if not hip_kernel.HAS_HIP:
        raise RuntimeError("GPU present but libturbopress_amd.so failed to load")
    return torch.device("cuda", 0)

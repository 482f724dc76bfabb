import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_ROOT = REPO / "gcc-hif8-quantized-from-qwen3.5-9b_amd"
for p in (str(REPO), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        return False


@pytest.fixture(scope="session")
def device():
    if not _gpu_available():
        pytest.skip("no HIP device")
    import torch

    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def native_ops(device):
    """The loaded extension; GPU tests fail (not skip) if it is missing."""
    from hif8_rocm import native

    native.reset_extension_cache()
    return native.load_extension()

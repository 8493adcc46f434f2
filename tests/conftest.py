"""Shared pytest setup.

* registers the ``gpu`` marker (tests that need an MI355X and the built HIP
  library ``libnsw.so``);
* puts the repository root (for ``oracle``) and the package directory
  ``neural-scaling-weather_amd`` (for ``nsw``) on ``sys.path``.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "neural-scaling-weather_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (gfx950) and the built libnsw.so")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected on a machine without a GPU; run with -m gpu on the GPU box")
    # references evaluated on the device (full-size checks) use full fp32 products
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    torch.set_float32_matmul_precision("highest")
    return torch.device("cuda:0")

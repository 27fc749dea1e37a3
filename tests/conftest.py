import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

PKG_NAME = "qwen3-naive-inference_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def load_pkg():
    return importlib.import_module(PKG_NAME)


def ensure_built():
    """Build libqwen3mi.so only when no built library exists."""
    lib = ROOT / PKG_NAME / "libqwen3mi.so"
    if not lib.exists():
        build = importlib.import_module(PKG_NAME + ".build")
        build.build()
    return lib


@pytest.fixture(scope="session")
def pkg():
    ensure_built()
    return load_pkg()


@pytest.fixture(scope="session")
def gpu(pkg):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    pkg._lib.lib()  # raises if the native library is missing
    return torch.device("cuda:0")

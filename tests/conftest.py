"""pytest setup: the `gpu` marker and access to the package's ctypes binding.

GPU tests run only where libdsd_hip.so reports a visible gfx950 device; on a
machine without one they are skipped (the reference's GPU tests likewise
print "skipped" and pass, tests/test_sparse_cuda.cpp:210-213).
"""
from __future__ import annotations

import importlib.util
import pathlib
import sys

import pytest

try:  # torch first, so libdsd_hip.so binds to the single HIP runtime torch loads
    import torch  # noqa: F401
except ImportError:  # pragma: no cover
    torch = None

ROOT = pathlib.Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "15-618_dynamic_sparse_decode_amd"
sys.path.insert(0, str(pathlib.Path(__file__).resolve().parent))


def load_package():
    """Import the package directory (its name is not a Python identifier)."""
    if "dsd_amd" in sys.modules:
        return sys.modules["dsd_amd"]
    spec = importlib.util.spec_from_file_location(
        "dsd_amd", PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    module = importlib.util.module_from_spec(spec)
    sys.modules["dsd_amd"] = module
    spec.loader.exec_module(module)
    return module


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a visible MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def dsd():
    return load_package()


@pytest.fixture(scope="session")
def gpu(dsd):
    """The loaded library on a machine with a gfx950 GPU, else skip."""
    if not dsd.gpu_available():
        pytest.skip("no visible gfx950 GPU")
    return dsd

"""Shared fixtures. GPU tests are marked `gpu`; everything else runs on CPU."""

from __future__ import annotations

import importlib.util
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_package():
    spec = importlib.util.spec_from_file_location("dav2_amd", ROOT / "depth-anything-v2_amd" / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules.setdefault("dav2_amd", mod)
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def pkg():
    return load_package()


@pytest.fixture(scope="session")
def lib(pkg):
    return pkg.load()


@pytest.fixture(scope="session")
def oracle():
    from oracle_py import Oracle
    o = Oracle()
    threads = int(os.environ.get("DAV2_ORACLE_THREADS", "0") or 0)
    if threads > 0:
        o.lib.orc_set_threads(threads)
    return o


@pytest.fixture(scope="session")
def gpu():
    """torch on the one visible GPU; the tests hand its tensors to the C ABI."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    torch.cuda.init()
    return torch

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
def ref_lib():
    """The reference's own src/model.cpp + src/image.cpp (oracle/_ref), built
    by `make -C oracle ref` where the reference tree exists."""
    import ctypes as C
    path = ROOT / "oracle" / "_ref" / "libdav2_ref.so"
    if not path.exists():
        pytest.skip("oracle/_ref not built (reference sources absent)")
    lib = C.CDLL(str(path))
    lib.ref_network_shape.argtypes = [C.c_int, C.c_int, C.c_int, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                      C.c_char_p, C.c_size_t]
    lib.ref_model_open.argtypes = [C.c_char_p, C.c_int, C.POINTER(C.c_uint), C.POINTER(C.c_int),
                                   C.POINTER(C.c_float), C.c_char_p, C.c_size_t]
    lib.ref_model_tensor.argtypes = [C.c_char_p, C.c_int, C.c_char_p, C.c_void_p, C.c_size_t]
    lib.ref_model_tensor.restype = C.c_longlong
    return lib


@pytest.fixture(scope="session")
def gpu():
    """torch on the one visible GPU; the tests hand its tensors to the C ABI."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    torch.cuda.init()
    return torch

"""C ABI checks that need no GPU: exports, status strings, network shape,
argument validation (tests/c_abi_smoke.c:6-51, src/dav2.cpp:126-213)."""

import ctypes as C
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = h.read_text()
        for m in re.finditer(r"DAV2_API\s+[^;{]*?\b(dav2_\w+)\s*\(", text, re.S):
            names.add(m.group(1))
    return sorted(names)


def test_every_declared_symbol_is_exported(lib):
    names = declared_symbols()
    assert len(names) > 60
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_c_abi_smoke(pkg, lib):
    # tests/c_abi_smoke.c:7-49
    assert lib.dav2_abi_version() == 1
    assert len(lib.dav2_version_string()) > 0
    assert lib.dav2_status_string(0) == b"ok"
    assert lib.dav2_status_string(11) == b"cancelled"
    assert lib.dav2_status_string(99) == b"unknown status"
    shape = pkg.ImageShape()
    assert lib.dav2_get_network_shape(640, 480, 518, C.byref(shape)) == 0
    assert (shape.width, shape.height) == (686, 518)
    assert lib.dav2_get_network_shape(480, 640, 518, C.byref(shape)) == 0
    assert (shape.width, shape.height) == (518, 686)
    assert lib.dav2_get_network_shape(0, 480, 518, C.byref(shape)) == 1
    assert len(lib.dav2_last_error()) > 0
    info = pkg.ModelInfo()
    info.struct_size = C.sizeof(info)
    assert lib.dav2_get_model_info(None, C.byref(info)) == 1
    caps = pkg.GpuCapabilities()
    caps.struct_size = C.sizeof(caps)
    assert lib.dav2_probe_gpu_capabilities(0, C.byref(caps)) == 0
    assert caps.abi_version == 1 and caps.flags == 0
    assert lib.dav2_get_gpu_capabilities(None, C.byref(caps)) == 1
    req = pkg.D3D12TextureSubmitRequest()
    req.struct_size = C.sizeof(req)
    req.abi_version = 1
    job = C.c_void_p()
    assert lib.dav2_submit_d3d12_texture(None, C.byref(req), C.byref(job)) == 1
    assert lib.dav2_get_network_shape(640, 480, 518, None) == 1


def test_inferbridge_shape_is_transposed(pkg, lib):
    s = pkg.ImageShape()
    assert lib.dav2_get_inferbridge_shape(640, 480, 518, C.byref(s)) == 0
    assert (s.width, s.height) == (518, 686)


def test_network_shape_matches_reference_image_cpp(pkg, lib, ref_lib):
    # The reference's own src/image.cpp network_shape, built into oracle/_ref.
    s = pkg.ImageShape()
    ow, oh = C.c_int(), C.c_int()
    err = C.create_string_buffer(128)
    for w, h, size in [(640, 480, 518), (1920, 1080, 518), (517, 519, 518), (14, 14, 14), (100, 3000, 140),
                       (1037, 1036, 1036), (33, 77, 70), (1, 1, 518)]:
        assert lib.dav2_get_network_shape(w, h, size, C.byref(s)) == 0
        assert ref_lib.ref_network_shape(w, h, size, C.byref(ow), C.byref(oh), err, 128) == 0
        assert (s.width, s.height) == (ow.value, oh.value), (w, h, size)


def _create(pkg, lib, path, **kw):
    opts = pkg.create_options(kw.pop("encoder", "vits"), kw.pop("flags", pkg.FORCE_INT8), kw.pop("device", 0))
    for k, v in kw.items():
        setattr(opts, k, v)
    ctx = C.c_void_p()
    st = lib.dav2_create(str(path).encode() if path is not None else None, C.byref(opts), C.byref(ctx))
    if st == 0:
        lib.dav2_destroy(ctx)
    return st, lib.dav2_last_error().decode()


def test_create_option_validation(pkg, lib, tmp_path):
    # src/dav2.cpp:158-199; all checked before any device work.
    p = tmp_path / "none.dav2"
    assert _create(pkg, lib, None)[0] == 1
    assert _create(pkg, lib, "")[0] == 1
    assert _create(pkg, lib, p, struct_size=8) == (1, "invalid create options")
    assert _create(pkg, lib, p, abi_version=2) == (1, "ABI version mismatch")
    opts = pkg.create_options("vits")
    opts.encoder = 7
    ctx = C.c_void_p()
    assert lib.dav2_create(str(p).encode(), C.byref(opts), C.byref(ctx)) == 1
    assert _create(pkg, lib, p, flags=1 << 9) == (1, "unsupported create flags")
    assert _create(pkg, lib, p, flags=pkg.FORCE_INT8 | pkg.FORCE_FP16)[0] == 1
    assert _create(pkg, lib, p, device=-1)[0] == 1
    # FORCE_FP32, FORCE_FP16 and FORCE_FP32_WEIGHTS pass validation: the missing file then fails in the loader
    assert _create(pkg, lib, p, flags=pkg.FORCE_FP16)[0] == 9
    assert _create(pkg, lib, p, flags=pkg.FORCE_FP16 | pkg.FORCE_FP32_ATTENTION)[0] == 9
    assert _create(pkg, lib, p, flags=pkg.FORCE_FP32)[0] == 9
    assert _create(pkg, lib, p, flags=pkg.FORCE_INT8 | 2)[0] == 9
    assert _create(pkg, lib, p, flags=pkg.FORCE_METAL)[0] == 8
    # the binary16 attention flags need the int8 or fp16 precision
    for att in (pkg.REFERENCE_FP16_ATTENTION, pkg.REFERENCE_FP16_COOP_ATTENTION):
        assert _create(pkg, lib, p, flags=att)[0] == 9
        assert _create(pkg, lib, p, flags=pkg.FORCE_FP16 | att)[0] == 9
        assert _create(pkg, lib, p, flags=pkg.FORCE_FP32 | att) == (
            1, "binary16 attention needs the int8 execution precision")
        assert _create(pkg, lib, p, flags=pkg.FORCE_FP32_ATTENTION | att)[0] == 1
    assert _create(pkg, lib, p, flags=1 << 18) == (1, "unsupported create flags")
    assert lib.dav2_create(str(p).encode(), C.byref(opts), None) == 1
    # a missing file fails in the loader (std::runtime_error -> INTERNAL_ERROR)
    st, msg = _create(pkg, lib, p)
    assert st == 9 and "failed to open model file" in msg


def test_null_context_entry_points(pkg, lib):
    x = (C.c_float * 4)()
    assert lib.dav2_infer_tensor_f32(None, x, 14, 14, x, 196) == 1
    assert lib.dav2_infer_tensor_f32_device(None, x, 1, 14, 14, x, 196, None) == 1
    assert lib.dav2_prepare(None, 1, 1, 1) == 1
    img = (C.c_uint8 * 48)()
    assert lib.dav2_infer_bgr8(None, img, 4, 4, 12, 518, x, 16) == 1
    assert lib.dav2_inferbridge_bgra8_f32(None, img, 4, 4, 16, 518, x, 16) == 1
    job = C.c_void_p()
    assert lib.dav2_submit_hip(None, None, C.byref(job)) == 1
    assert lib.dav2_gpu_job_cancel(None) == 1
    lib.dav2_gpu_job_release(None)  # safe
    assert lib.dav2_profile_enable(None, 1) == 1
    lib.dav2_destroy(None)  # safe (src/dav2.cpp:227-229)
    assert lib.dav2_gpu_job_cancel(None) == 1

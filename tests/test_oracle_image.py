"""The oracle's host-image restatements (src/image.cpp:138-339, src/dav2.cpp:787-800)
pinned against the reference's own src/image.cpp (compiled into oracle/_ref from
the reference tree) and against closed forms that hold without it."""

import ctypes as C

import numpy as np
import pytest

MEAN = np.array([0.485, 0.456, 0.406])
STD = np.array([0.229, 0.224, 0.225])


def _ref_setup(ref_lib):
    for name in ("ref_preprocess_bgr8", "ref_preprocess_inferbridge_bgra8"):
        f = getattr(ref_lib, name)
        f.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_longlong, C.c_int, C.c_int, C.c_void_p, C.c_char_p,
                      C.c_size_t]
        f.restype = C.c_int
    return ref_lib


def _image(rng, width, height, channels, stride):
    buf = rng.integers(0, 256, size=height * stride, dtype=np.uint8)
    view = buf.reshape(height, stride)[:, : width * channels]
    return buf, view


# (width, height, input_size, extra stride bytes): up- and down-scaling,
# odd sizes, identity (518x518 at 518), a one-pixel-wide image, padded rows
SHAPES = [(37, 23, 70, 0), (100, 61, 140, 5), (640, 480, 518, 0), (640, 480, 140, 3), (518, 518, 518, 0),
          (1, 9, 28, 1), (333, 17, 56, 0), (1920, 1080, 518, 64)]


@pytest.mark.parametrize("width,height,input_size,pad", SHAPES)
def test_preprocess_bgr8_matches_reference(oracle, ref_lib, width, height, input_size, pad):
    ref = _ref_setup(ref_lib)
    rng = np.random.default_rng(width * 31 + height)
    stride = width * 3 + pad
    buf, _ = _image(rng, width, height, 3, stride)
    dw, dh = oracle.network_shape(width, height, input_size)
    got = oracle.preprocess_bgr8(buf, width, height, stride, dw, dh)
    want = np.empty_like(got)
    err = C.create_string_buffer(256)
    assert ref.ref_preprocess_bgr8(buf.ctypes.data, width, height, stride, dw, dh, want.ctypes.data, err, 256) == 0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("width,height,input_size,pad", SHAPES)
def test_preprocess_bgra8_matches_reference(oracle, ref_lib, width, height, input_size, pad):
    ref = _ref_setup(ref_lib)
    rng = np.random.default_rng(width * 17 + height)
    stride = width * 4 + 4 * pad
    buf, _ = _image(rng, width, height, 4, stride)
    uw, uh = oracle.network_shape(width, height, input_size)
    dw, dh = uh, uw  # the InferBridge output shape is the transposed network shape (dav2.cpp:767-770)
    got = oracle.preprocess_bgra8_nearest(buf, width, height, stride, dw, dh)
    want = np.empty_like(got)
    err = C.create_string_buffer(256)
    assert ref.ref_preprocess_inferbridge_bgra8(buf.ctypes.data, width, height, stride, dw, dh, want.ctypes.data,
                                                err, 256) == 0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_reference_rejects_short_stride(ref_lib):
    ref = _ref_setup(ref_lib)
    buf = np.zeros(64, np.uint8)
    out = np.zeros(3 * 14 * 14, np.float32)
    err = C.create_string_buffer(256)
    assert ref.ref_preprocess_bgr8(buf.ctypes.data, 4, 4, 11, 14, 14, out.ctypes.data, err, 256) == 1
    assert err.value.decode() == "invalid source image"


def test_network_shape_matches_reference(oracle, ref_lib):
    for w in (1, 13, 14, 300, 518, 640, 1920, 4000):
        for h in (1, 14, 99, 480, 1080):
            for s in (14, 70, 518, 700):
                ow, oh = C.c_int(), C.c_int()
                err = C.create_string_buffer(256)
                assert ref_lib.ref_network_shape(w, h, s, C.byref(ow), C.byref(oh), err, 256) == 0
                assert oracle.network_shape(w, h, s) == (ow.value, oh.value)
    with pytest.raises(ValueError):
        oracle.network_shape(0, 10, 518)


def test_preprocess_bgr8_identity_is_normalisation(oracle):
    # At scale 1 every coordinate is an integer: the weights are exactly
    # (0, 1, 0, 0), so the resize returns the pixel and the output is
    # float((p / 255 - mean) / std) per channel, in RGB order.
    rng = np.random.default_rng(1)
    w, h = 28, 42
    img = rng.integers(0, 256, size=(h, w, 3), dtype=np.uint8)
    got = oracle.preprocess_bgr8(img, w, h, w * 3, w, h)
    rgb = img[:, :, ::-1].transpose(2, 0, 1).astype(np.float64)
    want = ((rgb / 255.0 - MEAN[:, None, None]) / STD[:, None, None]).astype(np.float32)
    assert np.array_equal(got, want)


def test_preprocess_bgr8_constant_image(oracle):
    # The four weights sum to 1 within float32 rounding: a constant image
    # resizes to (almost exactly) the same constant at any scale.
    w, h = 50, 31
    img = np.full((h, w, 3), (10, 128, 250), dtype=np.uint8)
    for dw, dh in ((140, 84), (28, 14), (50, 31)):
        got = oracle.preprocess_bgr8(img, w, h, w * 3, dw, dh)
        want = (np.array([250, 128, 10]) / 255.0 - MEAN) / STD
        assert np.abs(got - want[:, None, None]).max() < 1e-5


def test_preprocess_bgr8_linear_ramp(oracle):
    # Cubic convolution reproduces linear functions away from the clamped
    # border: a horizontal ramp p = 2x stays a ramp at the sampled positions.
    w, h = 120, 8
    ramp = (2 * np.arange(w)).astype(np.uint8)
    img = np.repeat(ramp[None, :, None], 3, axis=2).repeat(h, axis=0)
    dw, dh = 60, 8
    got = oracle.preprocess_bgr8(img, w, h, w * 3, dw, dh)
    x = (np.arange(dw) + 0.5) * (w / dw) - 0.5
    want = (2 * x / 255.0 - MEAN[0]) / STD[0]
    inner = slice(2, dw - 2)
    assert np.abs(got[0, 3, inner] - want[inner]).max() < 1e-4


def test_preprocess_bgra8_nearest_picks_floor_pixels(oracle):
    rng = np.random.default_rng(2)
    w, h = 40, 30
    img = rng.integers(0, 256, size=(h, w, 4), dtype=np.uint8)
    got = oracle.preprocess_bgra8_nearest(img, w, h, w * 4, 20, 15)  # exact 2x: pixel (2x, 2y)
    picked = img[::2, ::2, :3].transpose(2, 0, 1).astype(np.float32)  # byte order kept: B, G, R
    mean, std = MEAN.astype(np.float32), STD.astype(np.float32)
    want = (picked / np.float32(255.0) - mean[:, None, None]) / std[:, None, None]
    assert np.array_equal(got, want.astype(np.float32))


def test_normalize_span(oracle):
    rng = np.random.default_rng(3)
    d = (rng.standard_normal(1000) * 3 + 1).astype(np.float32)
    got = oracle.normalize_span(d)
    assert got[np.argmin(d)] == 0.0 and got[np.argmax(d)] == 1.0
    span = np.float32(d.max() - d.min())
    assert np.array_equal(got, (d - d.min()) / span)
    assert np.array_equal(oracle.normalize_span(np.full(10, 2.5, np.float32)), np.zeros(10, np.float32))


def _words(img):
    """uint8 [H][W][4] -> uint32 little-endian pixel words."""
    return np.ascontiguousarray(img).view(np.uint32).reshape(img.shape[0], img.shape[1])


def test_preprocess_rgba8_identity_is_normalisation(oracle):
    # preprocess_rgba.glsl at scale 1: every fraction is 0 and the weights are
    # exactly (0, 1, 0, 0); R is byte 0 of an RGBA word and byte 2 of BGRA.
    rng = np.random.default_rng(4)
    w, h = 30, 17
    img = rng.integers(0, 256, size=(h, w, 4), dtype=np.uint8)
    mean = np.array([0.485, 0.456, 0.406], np.float32)[:, None, None]
    std = np.array([0.229, 0.224, 0.225], np.float32)[:, None, None]
    for rgba, order in ((True, [0, 1, 2]), (False, [2, 1, 0])):
        got = oracle.preprocess_rgba8(_words(img), w, h, w, w, h, rgba)
        rgb = img[:, :, order].transpose(2, 0, 1).astype(np.float32)
        assert np.array_equal(got, (rgb / np.float32(255.0) - mean) / std)


def test_preprocess_rgba8_close_to_reference_cpu_resize(oracle, ref_lib):
    # The float32 GPU resize and the reference's float64 CPU resize
    # (image.cpp, built from its sources) are the same cubic filter up to
    # rounding; the GPU path rounds the sample coordinate to float32 first
    # (an ulp of 600 is 6e-5 of a pixel), so they agree to 1e-4.
    _ref_setup(ref_lib)
    rng = np.random.default_rng(5)
    for (w, h, s) in ((97, 61, 140), (640, 480, 518), (300, 17, 56)):
        img = rng.integers(0, 256, size=(h, w, 4), dtype=np.uint8)
        dw, dh = oracle.network_shape(w, h, s)
        got = oracle.preprocess_rgba8(_words(img), w, h, w, dw, dh, False)  # BGRA
        bgr = np.ascontiguousarray(img[:, :, :3])
        want = np.empty_like(got)
        err = C.create_string_buffer(256)
        assert ref_lib.ref_preprocess_bgr8(bgr.ctypes.data, w, h, 3 * w, dw, dh, want.ctypes.data, err, 256) == 0
        assert np.abs(got - want).max() < 1e-4

"""Host-image paths on the GPU (src/image.cpp:163-339, src/dav2.cpp:630-665,
:754-802): the preprocessing kernels bit for bit against the oracle (itself
pinned to the reference's image.cpp), then dav2_infer_bgr8 and
dav2_inferbridge_bgra8_f32 end to end against the oracle's pipeline on a
seeded synthetic model."""

import numpy as np
import pytest

from gpu_util import dev, empty, host, ok, ptr, stream

pytestmark = pytest.mark.gpu

SEED = 0xDA20000

# (width, height, input_size, extra stride bytes)
SHAPES = [(37, 23, 70, 0), (100, 61, 140, 5), (640, 480, 518, 0), (640, 480, 140, 3), (518, 518, 518, 0),
          (1, 9, 28, 1), (333, 17, 56, 0), (1920, 1080, 518, 64)]


def _announce(*args):
    print("case:", *args, flush=True)


def _image(seed, width, height, channels, stride):
    rng = np.random.default_rng(seed)
    return rng.integers(0, 256, size=height * stride, dtype=np.uint8)


@pytest.mark.parametrize("width,height,input_size,pad", SHAPES)
def test_preprocess_bgr8_bit_exact(gpu, lib, oracle, width, height, input_size, pad):
    torch = gpu
    stride = width * 3 + pad
    dw, dh = oracle.network_shape(width, height, input_size)
    _announce("preprocess_bgr8", width, height, stride, dw, dh)
    buf = _image(width * 7 + height, width, height, 3, stride)
    ref = oracle.preprocess_bgr8(buf, width, height, stride, dw, dh)
    bd = dev(torch, buf)
    out = empty(torch, (3, dh, dw), torch.float32)
    ok(lib, lib.dav2_hip_preprocess_bgr8(ptr(bd), width, height, stride, dw, dh, ptr(out), stream(torch)))
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("width,height,input_size,pad", SHAPES)
def test_preprocess_bgra8_nearest_bit_exact(gpu, lib, oracle, width, height, input_size, pad):
    torch = gpu
    stride = width * 4 + 4 * pad
    uw, uh = oracle.network_shape(width, height, input_size)
    dw, dh = uh, uw
    _announce("preprocess_bgra8_nearest", width, height, stride, dw, dh)
    buf = _image(width * 5 + height, width, height, 4, stride)
    ref = oracle.preprocess_bgra8_nearest(buf, width, height, stride, dw, dh)
    bd = dev(torch, buf)
    out = empty(torch, (3, dh, dw), torch.float32)
    ok(lib, lib.dav2_hip_preprocess_bgra8_nearest(ptr(bd), width, height, stride, dw, dh, ptr(out),
                                                  stream(torch)))
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))


def test_preprocess_argument_checks(gpu, lib):
    torch = gpu
    buf = empty(torch, (4096,), torch.uint8)
    out = empty(torch, (3 * 14 * 14,), torch.float32)
    s = stream(torch)
    assert lib.dav2_hip_preprocess_bgr8(ptr(buf), 10, 10, 29, 14, 14, ptr(out), s) != 0  # stride < 3 * width
    assert lib.dav2_hip_preprocess_bgr8(ptr(buf), 0, 10, 30, 14, 14, ptr(out), s) != 0
    assert lib.dav2_hip_preprocess_bgr8(None, 10, 10, 30, 14, 14, ptr(out), s) != 0
    assert lib.dav2_hip_preprocess_bgra8_nearest(ptr(buf), 10, 10, 42, 14, 14, ptr(out), s) != 0  # not 4-aligned
    assert lib.dav2_hip_preprocess_bgra8_nearest(ptr(buf), 10, 10, 36, 14, 14, ptr(out), s) != 0  # < 4 * width


@pytest.mark.parametrize("n,constant", [(1000, False), (518 * 518, False), (4096, True)])
def test_normalize_span_bit_exact(gpu, lib, oracle, n, constant):
    torch = gpu
    _announce("normalize_span", n, constant)
    rng = np.random.default_rng(n)
    d = np.full(n, 3.25, np.float32) if constant else (rng.standard_normal(n) * 2 + 5).astype(np.float32)
    dd = dev(torch, d)
    rng_d = empty(torch, (2,), torch.float32)
    part = empty(torch, (2 * lib.dav2_hip_minmax_partials(n),), torch.float32)
    out = empty(torch, (n,), torch.float32)
    s = stream(torch)
    ok(lib, lib.dav2_hip_reduce_minmax(ptr(dd), n, ptr(rng_d), ptr(part), s))
    ok(lib, lib.dav2_hip_normalize_span(ptr(dd), ptr(rng_d), n, ptr(out), s))
    assert np.array_equal(host(torch, out), oracle.normalize_span(d))


@pytest.fixture(scope="module")
def vits_model(pkg, tmp_path_factory):
    p = tmp_path_factory.mktemp("img_models") / "vits.dav2"
    pkg.dav2_format.write_synthetic_model(p, "vits", seed=SEED + 1)
    return p


def _oracle_depth(oracle, model, chw, width, height):
    h = oracle.load_model(model, 0)
    try:
        depth, _, _ = oracle.infer(h, chw, width, height, attention="exact")
    finally:
        oracle.free_model(h)
    return depth


# pad 7: rows uploaded with their padding; pad 360 (stride twice the row):
# rows packed on the host before the upload
@pytest.mark.parametrize("width,height,input_size,pad",
                         [(300, 200, 140, 0), (97, 131, 112, 7), (140, 140, 140, 0), (120, 90, 70, 360)])
def test_infer_bgr8_end_to_end(gpu, pkg, lib, oracle, vits_model, width, height, input_size, pad):
    # dav2.cpp:630-665: network_shape -> preprocess -> inference -> bilinear
    # (align corners) back to the image size; int8 mode is bit-exact.
    stride = width * 3 + pad
    nw, nh = oracle.network_shape(width, height, input_size)
    _announce("infer_bgr8", width, height, stride, input_size, nw, nh)
    buf = _image(width + 3 * height, width, height, 3, stride)
    with pkg.Context(str(vits_model), "vits") as ctx:
        got = ctx.infer_bgr8_rows(buf, width, height, stride, input_size)
        got2 = ctx.infer_bgr8_rows(buf, width, height, stride, input_size)  # arena reuse
    chw = oracle.preprocess_bgr8(buf, width, height, stride, nw, nh)
    depth = _oracle_depth(oracle, vits_model, chw, nw, nh)
    want = depth if (nw, nh) == (width, height) else oracle.bilinear(depth[None], width, height)[0]
    assert got.shape == (height, width) and np.isfinite(got).all()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(got, got2)


def test_inferbridge_bgra8_end_to_end(gpu, pkg, lib, oracle, vits_model):
    # dav2.cpp:754-802: nearest resize to the transposed network shape, depth
    # min/max normalised at that size.
    width, height, input_size = 180, 120, 112
    uw, uh = oracle.network_shape(width, height, input_size)
    nw, nh = uh, uw
    _announce("inferbridge_bgra8", width, height, nw, nh)
    rng = np.random.default_rng(9)
    img = rng.integers(0, 256, size=(height, width, 4), dtype=np.uint8)
    with pkg.Context(str(vits_model), "vits") as ctx:
        got = ctx.inferbridge_bgra8(img, input_size)
    chw = oracle.preprocess_bgra8_nearest(img, width, height, width * 4, nw, nh)
    want = oracle.normalize_span(_oracle_depth(oracle, vits_model, chw, nw, nh)).reshape(nh, nw)
    assert got.shape == (nh, nw)
    assert np.array_equal(got, want)


def test_inferbridge_bgra8_strides(gpu, pkg, lib, vits_model):
    # The same pixels with row padding kept (stride % 4 == 0) and packed on
    # the host (odd stride; large padding) give the same output.
    width, height, input_size = 70, 56, 56
    rng = np.random.default_rng(11)
    img = rng.integers(0, 256, size=(height, width * 4), dtype=np.uint8)
    shape = pkg.ImageShape()
    import ctypes as C
    assert lib.dav2_get_inferbridge_shape(width, height, input_size, C.byref(shape)) == 0
    outs = []
    with pkg.Context(str(vits_model), "vits") as ctx:
        for pad in (0, 8, 3, width * 4):
            stride = width * 4 + pad
            buf = np.zeros((height, stride), np.uint8)
            buf[:, : width * 4] = img
            out = np.empty(shape.width * shape.height, np.float32)
            _announce("inferbridge stride", stride)
            assert lib.dav2_inferbridge_bgra8_f32(ctx.handle, buf.ctypes.data, width, height, stride, input_size,
                                                  out.ctypes.data, out.size) == 0
            outs.append(out)
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


def test_image_entry_argument_checks(gpu, pkg, lib, vits_model):
    import ctypes as C
    buf = np.zeros(64 * 64 * 4, np.uint8)
    out = np.zeros(64 * 64, np.float32)
    big = np.zeros(140 * 140, np.float32)
    with pkg.Context(str(vits_model), "vits") as ctx:
        f = lib.dav2_infer_bgr8
        assert f(ctx.handle, buf.ctypes.data, 64, 64, 191, 140, out.ctypes.data, out.size) == 1  # short stride
        assert f(ctx.handle, buf.ctypes.data, 64, 64, 192, 140, out.ctypes.data, out.size - 1) == 7
        assert f(ctx.handle, buf.ctypes.data, 64, 64, 192, 0, out.ctypes.data, out.size) == 1  # input_size
        assert f(ctx.handle, buf.ctypes.data, 0, 64, 192, 140, out.ctypes.data, out.size) == 1
        assert f(ctx.handle, None, 64, 64, 192, 140, out.ctypes.data, out.size) == 1
        assert lib.dav2_last_error() == b"null inference argument"
        g = lib.dav2_inferbridge_bgra8_f32
        assert g(ctx.handle, buf.ctypes.data, 64, 64, 256, 140, big.ctypes.data, big.size - 1) == 7
        assert g(ctx.handle, buf.ctypes.data, 64, 64, 255, 140, big.ctypes.data, big.size) == 1
        assert g(ctx.handle, buf.ctypes.data, 64, 64, 256, 140, big.ctypes.data, big.size) == 0
        assert np.isfinite(big).all() and big.min() >= 0.0 and big.max() <= 1.0
        shape = pkg.ImageShape()
        assert lib.dav2_get_inferbridge_shape(64, 64, 140, C.byref(shape)) == 0
        assert (shape.width, shape.height) == (140, 140)

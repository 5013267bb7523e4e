"""The operator surface (include/dav2_ops.h -> dav2::HipOperators, mirroring
the reference's VulkanOperators) vs the CPU oracle, plus the reference's own
int8-vs-fp32 operator tests (tests/vulkan_smoke.cpp:143-240) and its size
validation behaviour (src/operators.cpp:93-102)."""

import numpy as np
import pytest
import torch.nn.functional as F

from gpu_util import db, dev, empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(gpu, lib):
    h = lib.dav2_ops_create(0)
    assert h, lib.dav2_ops_last_error()
    yield h
    lib.dav2_ops_destroy(h)


def run(lib, rc):
    assert rc == 0, f"status {rc}: {lib.dav2_ops_last_error().decode()}"


def sync(lib, ops):
    run(lib, lib.dav2_ops_synchronize(ops))


def _weight(torch, oracle, w):
    """int8 weights in the reference GpuModel layout: [rows][K] bytes
    (gpu_model.cpp:241-284), exactly K bytes per row whatever K % 64."""
    q, s = oracle.quantize_weight_rows(w)
    return dev(torch, np.ascontiguousarray(q)), dev(torch, s), q, s


@pytest.mark.parametrize("rows,ic,oc,gelu", [(1370, 384, 1152, False), (1370, 1024, 4096, True), (5, 588, 384, False),
                                             (1369, 1536, 384, False), (1369, 588, 384, False), (77, 432, 48, True),
                                             (3, 36, 5, False)])
def test_linear_int8(gpu, pkg, lib, oracle, ops, rows, ic, oc, gelu):
    torch = gpu
    rng = np.random.default_rng(rows + ic + oc)
    x = rng.standard_normal((rows, ic)).astype(np.float32)
    w = (rng.standard_normal((oc, ic)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(oc) * 0.01).astype(np.float32)
    wd, sd, q, s = _weight(torch, oracle, w)
    xd, bd = dev(torch, x), dev(torch, b)
    out = empty(torch, (rows, oc), torch.float32)
    run(lib, lib.dav2_ops_linear_int8(ops, db(pkg, out), db(pkg, xd), db(pkg, wd), db(pkg, sd), db(pkg, bd), rows, ic,
                                      oc, int(gelu), 0))
    sync(lib, ops)
    ref = oracle.linear_int8(x, q, s, b, gelu=gelu)
    got = host(torch, out)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("rows,ic,oc,gelu", [(1370, 1024, 3072, False), (1370, 1024, 4096, True),
                                             (300, 4096, 1024, False), (130, 588, 100, True), (3, 36, 5, False)])
def test_linear_int8_weight_transposed(gpu, pkg, lib, oracle, ops, rows, ic, oc, gelu):
    # linear_int8(..., weight_transposed=true) with the reference's
    # int8_transposed_buffer ([K][N] bytes, gpu_model.cpp:241-258): the same
    # bits as the oracle's linear on the [N][K] weight.
    torch = gpu
    print("case: linear_int8 transposed", rows, ic, oc, gelu, flush=True)
    rng = np.random.default_rng(rows * 7 + ic + oc)
    x = rng.standard_normal((rows, ic)).astype(np.float32)
    w = (rng.standard_normal((oc, ic)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(oc) * 0.01).astype(np.float32)
    q, s = oracle.quantize_weight_rows(w)
    qt = dev(torch, np.ascontiguousarray(q.T))  # [K][N] bytes
    xd, bd, sd = dev(torch, x), dev(torch, b), dev(torch, s)
    out = empty(torch, (rows, oc), torch.float32)
    out.fill_(float("nan"))
    torch.cuda.current_stream().synchronize()
    run(lib, lib.dav2_ops_linear_int8(ops, db(pkg, out), db(pkg, xd), db(pkg, qt), db(pkg, sd), db(pkg, bd), rows, ic,
                                      oc, int(gelu), 1))
    sync(lib, ops)
    ref = oracle.linear_int8(x, q, s, b, gelu=gelu)
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))
    # a transposed buffer one byte short is rejected
    run_rc = lib.dav2_ops_linear_int8(ops, db(pkg, out), db(pkg, xd), db(pkg, qt, ic * oc - 1), db(pkg, sd),
                                      db(pkg, bd), rows, ic, oc, int(gelu), 1)
    assert run_rc == 1 and b"transposed INT8 weight" in lib.dav2_ops_last_error()


def test_linear_int8_validation(gpu, pkg, lib, ops):
    torch = gpu
    x = empty(torch, (4, 64), torch.float32)
    w = empty(torch, (8, 64), torch.int8)
    s = empty(torch, (8,), torch.float32)
    out = empty(torch, (4, 8), torch.float32)
    # K not a multiple of 4 (operators.cpp:785-788)
    assert lib.dav2_ops_linear_int8(ops, db(pkg, out), db(pkg, x), db(pkg, w), db(pkg, s), db(pkg, s), 4, 62, 8, 0,
                                    0) == 1
    # output buffer too small (require_bytes)
    assert lib.dav2_ops_linear_int8(ops, db(pkg, out, 64), db(pkg, x), db(pkg, w), db(pkg, s), db(pkg, s), 4, 64, 8,
                                    0, 0) == 1
    assert b"too small" in lib.dav2_ops_last_error()
    # zero rows
    assert lib.dav2_ops_linear_int8(ops, db(pkg, out), db(pkg, x), db(pkg, w), db(pkg, s), db(pkg, s), 0, 64, 8, 0,
                                    0) == 1


def test_conv2d_int8_reference_kat(gpu, pkg, lib, oracle, ops):
    # tests/vulkan_smoke.cpp:143-186: 4x4x5 input, 5 outputs, k=3, pad 1;
    # int8 within 0.006 of the fp32 convolution.
    torch = gpu
    width, height, channels, outputs, k = 5, 4, 4, 5, 3
    values = ((np.arange(width * height * channels) % 23 - 11) * 0.03125).astype(np.float32)
    weights = ((np.arange(outputs * channels * 9) % 19 - 9) * 0.015625).astype(np.float32)
    biases = (np.arange(outputs) * 0.01).astype(np.float32)
    x = values.reshape(channels, height, width)
    w4 = weights.reshape(outputs, channels, k, k)
    wd, sd, q, s = _weight(torch, oracle, w4)
    xd, bd = dev(torch, x), dev(torch, biases)
    out = empty(torch, (outputs, height, width), torch.float32)
    run(lib, lib.dav2_ops_conv2d_int8(ops, db(pkg, out), db(pkg, xd), db(pkg, wd), db(pkg, sd), db(pkg, bd), width,
                                      height, channels, outputs, k, 1, 1, 1))
    sync(lib, ops)
    got = host(torch, out)
    fp32 = F.conv2d(torch.from_numpy(x)[None], torch.from_numpy(w4), torch.from_numpy(biases), padding=1)[0].numpy()
    assert np.abs(got - fp32).max() <= 0.006
    ref = oracle.conv2d_int8(x, q, s, biases, outputs, k, 1, 1)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("c,h,w,oc,k,stride,pad,bias", [
    (256, 37, 37, 256, 3, 1, 1, True), (1024, 19, 19, 256, 3, 1, 1, False), (1024, 37, 37, 1024, 3, 2, 1, True),
    (256, 74, 74, 256, 1, 1, 0, True), (128, 130, 130, 32, 3, 1, 1, True), (32, 130, 130, 1, 1, 1, 0, True),
    (96, 23, 29, 64, 3, 1, 1, True), (48, 37, 37, 64, 3, 1, 1, True), (48, 21, 17, 96, 3, 2, 1, False)])
def test_conv2d_int8_vs_oracle(gpu, pkg, lib, oracle, ops, c, h, w, oc, k, stride, pad, bias):
    torch = gpu
    print("case: conv2d", c, h, w, oc, k, stride, pad, flush=True)
    rng = np.random.default_rng(c * h + oc)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    wt = rng.uniform(-1, 1, (oc, c, k, k)).astype(np.float32) / np.sqrt(c * k * k)
    b = rng.uniform(-0.1, 0.1, oc).astype(np.float32)
    wd, sd, q, s = _weight(torch, oracle, wt)
    xd, bd = dev(torch, x), dev(torch, b if bias else np.zeros(1, np.float32))
    ow, oh = (w + 2 * pad - k) // stride + 1, (h + 2 * pad - k) // stride + 1
    out = empty(torch, (oc, oh, ow), torch.float32)
    run(lib, lib.dav2_ops_conv2d_int8(ops, db(pkg, out), db(pkg, xd), db(pkg, wd), db(pkg, sd), db(pkg, bd), w, h, c,
                                      oc, k, stride, pad, int(bias)))
    sync(lib, ops)
    ref = oracle.conv2d_int8(x, q, s, b if bias else None, oc, k, stride, pad, has_bias=bias)
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))


def test_conv_transpose_reference_kat(gpu, pkg, lib, oracle, ops):
    # tests/vulkan_smoke.cpp:187-240: 3x2x4 input, 3 outputs, k=2; int8 within
    # 0.004 of the fp32 transposed convolution.
    torch = gpu
    width, height, inputs, outputs, k = 3, 2, 4, 3, 2
    values = ((np.arange(width * height * inputs) % 17 - 8) * 0.03125).astype(np.float32).reshape(inputs, height, width)
    weights = ((np.arange(inputs * outputs * k * k) % 13 - 6) * 0.02).astype(np.float32).reshape(inputs, outputs, k, k)
    biases = np.zeros(outputs, np.float32)
    q, s = oracle.quantize_convT_weight(weights)
    wd, sd, bd, xd = dev(torch, q), dev(torch, s), dev(torch, biases), dev(torch, values)
    out = empty(torch, (outputs, height * k, width * k), torch.float32)
    run(lib, lib.dav2_ops_conv_transpose_nonoverlap_int8(ops, db(pkg, out), db(pkg, xd), db(pkg, wd), db(pkg, sd),
                                                         db(pkg, bd), width, height, inputs, outputs, k))
    sync(lib, ops)
    got = host(torch, out)
    fp32 = F.conv_transpose2d(torch.from_numpy(values)[None], torch.from_numpy(weights), stride=k)[0].numpy()
    assert np.abs(got - fp32).max() <= 0.004
    ref = oracle.conv_transpose_int8(values, q, s, biases, outputs, k)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("c,h,w,k", [(256, 37, 37, 4), (512, 37, 37, 2), (96, 25, 19, 4)])
def test_conv_transpose_vs_oracle(gpu, pkg, lib, oracle, ops, c, h, w, k):
    torch = gpu
    rng = np.random.default_rng(c + k)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    wt = rng.uniform(-1, 1, (c, c, k, k)).astype(np.float32) / np.sqrt(c * k * k)
    b = rng.uniform(-0.1, 0.1, c).astype(np.float32)
    q, s = oracle.quantize_convT_weight(wt)
    wd, sd, bd, xd = dev(torch, q), dev(torch, s), dev(torch, b), dev(torch, x)
    out = empty(torch, (c, h * k, w * k), torch.float32)
    run(lib, lib.dav2_ops_conv_transpose_nonoverlap_int8(ops, db(pkg, out), db(pkg, xd), db(pkg, wd), db(pkg, sd),
                                                         db(pkg, bd), w, h, c, c, k))
    sync(lib, ops)
    ref = oracle.conv_transpose_int8(x, q, s, b, c, k)
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("pw,ph,dim,oc", [(37, 37, 1024, 256), (25, 19, 384, 48)])
def test_project_tokens_int8(gpu, pkg, lib, oracle, ops, pw, ph, dim, oc):
    torch = gpu
    rng = np.random.default_rng(dim + oc)
    tokens = rng.standard_normal((pw * ph + 1, dim)).astype(np.float32)
    w = rng.uniform(-1, 1, (oc, dim, 1, 1)).astype(np.float32) / np.sqrt(dim)
    b = rng.uniform(-0.1, 0.1, oc).astype(np.float32)
    wd, sd, q, s = _weight(torch, oracle, w)
    td, bd = dev(torch, tokens), dev(torch, b)
    out = empty(torch, (oc, ph, pw), torch.float32)
    run(lib, lib.dav2_ops_project_tokens_int8(ops, db(pkg, out), db(pkg, td), db(pkg, wd), db(pkg, sd), db(pkg, bd),
                                              pw, ph, dim, oc))
    sync(lib, ops)
    ref = oracle.project_tokens_int8(tokens, q, s, b, pw, ph, dim, oc)
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("width,height,dim", [(518, 518, 384), (350, 266, 1024), (42, 28, 64)])
def test_prepare_tokens_int8(gpu, pkg, lib, oracle, ops, width, height, dim):
    torch = gpu
    fmt = pkg.dav2_format
    rng = np.random.default_rng(dim + width)
    image = fmt.imagenet_input(width, height, seed=dim)[0]
    w = (rng.standard_normal((dim, 3, 14, 14)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(dim) * 0.01).astype(np.float32)
    cls = (rng.standard_normal(dim) * 0.02).astype(np.float32)
    pos = (rng.standard_normal((1370, dim)) * 0.02).astype(np.float32)
    wd, sd, q, s = _weight(torch, oracle, w)
    imd, bd, cd, pd = dev(torch, image), dev(torch, b), dev(torch, cls), dev(torch, pos)
    t = (width // 14) * (height // 14) + 1
    out = empty(torch, (t, dim), torch.float32)
    run(lib, lib.dav2_ops_prepare_tokens(ops, db(pkg, out), db(pkg, imd), db(pkg, wd), db(pkg, sd), db(pkg, bd),
                                         db(pkg, cd), db(pkg, pd), width, height, dim))
    sync(lib, ops)
    ref = oracle.prepare_tokens_int8(image, q, s, b, cls, pos, width, height, dim)
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))


def test_prepare_tokens_reference_kat(gpu, pkg, lib, oracle, ops):
    # tests/vulkan_smoke.cpp:630-754: zero image and weights, so every patch
    # token is bias + bicubic position (closed form, 2e-6) and the class token
    # is class + position[0] exactly.
    torch = gpu
    width, height, dim = 42, 28, 3
    bias = np.array([0.25, -0.5, 0.75], np.float32)
    cls = np.array([1.0, 2.0, 3.0], np.float32)
    pos = ((np.arange(1370 * dim) % 31 - 15) * 0.015625).astype(np.float32).reshape(1370, dim)
    image = np.zeros((3, height, width), np.float32)
    wq, ws = oracle.quantize_weight_rows(np.zeros((dim, 3, 14, 14), np.float32))
    out = empty(torch, (7, dim), torch.float32)
    # Every device tensor stays referenced until the call is synchronised: a
    # temporary would go back to torch's caching allocator and the next
    # upload could reuse its memory.
    held = [dev(torch, a) for a in (image, wq, ws, bias, cls, pos)]
    run(lib, lib.dav2_ops_prepare_tokens(ops, db(pkg, out), *[db(pkg, t) for t in held], width, height, dim))
    sync(lib, ops)
    tokens = host(torch, out)
    assert np.array_equal(tokens[0], cls + pos[0])

    def c1(x):
        a = -0.75
        return ((a + 2) * x - (a + 3)) * x * x + 1

    def c2(x):
        a = -0.75
        return ((a * x - 5 * a) * x + 8 * a) * x - 4 * a

    pw, ph = width // 14, height // 14
    for py in range(ph):
        for px in range(pw):
            sx = (px + 0.5) * (37.0 / (pw + 0.1)) - 0.5
            sy = (py + 0.5) * (37.0 / (ph + 0.1)) - 0.5
            bx, by = int(np.floor(sx)), int(np.floor(sy))
            fx, fy = sx - bx, sy - by
            cx = [c2(fx + 1), c1(fx), c1(1 - fx), c2(2 - fx)]
            cy = [c2(fy + 1), c1(fy), c1(1 - fy), c2(2 - fy)]
            expect = bias.astype(np.float64).copy()
            for r in range(4):
                y = min(max(by - 1 + r, 0), 36)
                row = np.zeros(dim)
                for cc in range(4):
                    x = min(max(bx - 1 + cc, 0), 36)
                    row += pos[1 + y * 37 + x] * cx[cc]
                expect += row * cy[r]
            np.testing.assert_allclose(tokens[1 + py * pw + px], expect, atol=2e-6)


def test_layer_norm_add_scaled_kats(gpu, pkg, lib, ops):
    # tests/vulkan_smoke.cpp:436-538
    torch = gpu
    rows, cols = 4, 17
    x = ((np.arange(rows * cols) % 23 - 10) * 0.125).astype(np.float32).reshape(rows, cols)
    w, b = np.ones(cols, np.float32), np.zeros(cols, np.float32)
    out = empty(torch, (rows, cols), torch.float32)
    held = [dev(torch, a) for a in (x, w, b)]
    run(lib, lib.dav2_ops_layer_norm(ops, db(pkg, out), *[db(pkg, t) for t in held], rows, cols, 1e-6))
    sync(lib, ops)
    mean = x.mean(axis=1, keepdims=True)
    var = np.maximum((x * x).mean(axis=1, keepdims=True) - mean * mean, 0)
    np.testing.assert_allclose(host(torch, out), (x - mean) / np.sqrt(var + 1e-6), atol=1e-5)
    residual = (np.arange(15) * 0.125).astype(np.float32)
    addend = ((np.arange(15) + 2) * -0.0625).astype(np.float32)
    scale = ((np.arange(5) + 1) * 0.25).astype(np.float32)
    o2 = empty(torch, (15,), torch.float32)
    held2 = [dev(torch, a) for a in (residual, addend, scale)]
    run(lib, lib.dav2_ops_add_scaled(ops, db(pkg, o2), *[db(pkg, t) for t in held2], 15, 5))
    sync(lib, ops)
    assert np.array_equal(host(torch, o2), residual + addend * scale[np.arange(15) % 5])
    assert lib.dav2_ops_add_scaled(ops, db(pkg, o2), db(pkg, o2), db(pkg, o2), db(pkg, o2), 15, 4) == 1


@pytest.mark.parametrize("tokens,heads,precision", [(1370, 16, 0), (1370, 16, 1), (257, 6, 1)])
def test_attention_head64_surface(gpu, pkg, lib, oracle, ops, tokens, heads, precision):
    torch = gpu
    rng = np.random.default_rng(tokens + heads)
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * 0.5).astype(np.float32)
    out = empty(torch, (tokens, heads * 64), torch.float32)
    qkv_d = dev(torch, qkv)
    run(lib, lib.dav2_ops_attention_head64(ops, db(pkg, out), db(pkg, qkv_d), tokens, heads, db(pkg, None),
                                           precision))
    sync(lib, ops)
    ref = oracle.attention(qkv, tokens, heads, fp16=bool(precision))
    # the reference shaders' arithmetic order: bit for bit
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))
    # a caller-provided scratch of exactly the reference's size
    # (operators.cpp:1112-1119: H*T*T floats, or H*T*ceil(T/2) half2 words)
    nbytes = heads * tokens * ((tokens + 1) // 2 * 4 if precision else tokens * 4)
    scratch = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out2 = empty(torch, (tokens, heads * 64), torch.float32)
    run(lib, lib.dav2_ops_attention_head64(ops, db(pkg, out2), db(pkg, qkv_d), tokens, heads, db(pkg, scratch),
                                           precision))
    sync(lib, ops)
    assert np.array_equal(host(torch, out2).view(np.uint32), ref.view(np.uint32))
    small = empty(torch, (16,), torch.float32)
    assert lib.dav2_ops_attention_head64(ops, db(pkg, out), db(pkg, qkv_d), tokens, heads, db(pkg, small),
                                         precision) == 1


def test_bilinear_minmax_normalize_surface(gpu, pkg, lib, oracle, ops):
    torch = gpu
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, 296, 296)).astype(np.float32)
    out = empty(torch, (1, 518, 518), torch.float32)
    x_d = dev(torch, x)
    run(lib, lib.dav2_ops_bilinear_align_true(ops, db(pkg, out), db(pkg, x_d), 296, 296, 518, 518, 1))
    rng_d = empty(torch, (2,), torch.float32)
    run(lib, lib.dav2_ops_reduce_minmax(ops, db(pkg, out), db(pkg, rng_d), 518 * 518))
    run(lib, lib.dav2_ops_normalize_relative(ops, db(pkg, out), db(pkg, rng_d), 518 * 518))
    sync(lib, ops)
    ref = oracle.bilinear(x, 518, 518)
    r = oracle.reduce_minmax(ref)
    ref = oracle.normalize_relative(ref, r)
    assert np.array_equal(host(torch, out).view(np.uint32), ref.reshape(1, 518, 518).view(np.uint32))
    assert lib.dav2_ops_reduce_minmax(ops, db(pkg, out), db(pkg, rng_d), 0) == 1

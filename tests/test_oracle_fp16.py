"""Pins the CPU oracle's fp16 precision mode (CPU only).

The native binary16 operators (prepare_tokens_fp16.glsl, project_tokens and
conv_transpose_nonoverlap with NATIVE_FP16) are checked against loop-for-loop
numpy restatements of the shaders (numpy's float16 multiply is the IEEE
binary16 product: the exact product of two binary16 values fits a float32,
which numpy rounds once), and by hand vectors in which rounding each product,
or the order of the fp32 sum, changes the result. The cooperative-matrix
linear is checked against float64 products of the binary16-rounded operands,
and by hand vectors that fail if an operand is not rounded."""

import numpy as np
import pytest

F16, F32 = np.float16, np.float32


def _h(x):
    return np.asarray(x, F32).astype(F16)


def _h16_products_numpy(a, b):
    """out[i][j] = sum over k ascending of float32(f16(a) * f16(b))."""
    a16, b16 = _h(a), _h(b)
    m, k = a16.shape
    out = np.zeros((m, b16.shape[0]), F32)
    for kk in range(k):
        prod = (a16[:, kk:kk + 1] * b16[None, :, kk]).astype(F32)  # binary16 products, widened
        out = (out + prod).astype(F32)
    return out


@pytest.mark.parametrize("m,n,k", [(1, 1, 4), (7, 5, 36), (33, 17, 96)])
def test_gemm_h16_products_matches_restatement(oracle, m, n, k):
    rng = np.random.default_rng(m * 100 + n * 10 + k)
    a = (rng.standard_normal((m, k)) * 3).astype(F32)
    b = (rng.standard_normal((n, k)) * 0.2).astype(F32)
    got = oracle.gemm_h16_products(a, b)
    want = _h16_products_numpy(a, b)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gemm_h16_products_round_each_product_and_sum_in_order(oracle):
    # (1 + 2^-10)^2 = 1 + 2^-9 + 2^-20 exactly; binary16 rounds the product to
    # 1 + 2^-9, and the next term removes it: 0 with rounded products, 2^-20
    # with exact ones.
    a = np.array([[1 + 2.0 ** -10, -(1 + 2.0 ** -9)]], F32)
    b = np.array([[1 + 2.0 ** -10, 1.0]], F32)
    assert oracle.gemm_h16_products(a, b)[0, 0] == 0.0
    # fp32 sum in k order: 2^14 + 2^-10 rounds to 2^14 (ulp 2^-9, tie to even),
    # then -2^14 gives 0; the reversed order would give 2^-10.
    a = np.array([[2.0 ** 14, 2.0 ** -10, -(2.0 ** 14)]], F32)
    b = np.ones((1, 3), F32)
    assert oracle.gemm_h16_products(a, b)[0, 0] == 0.0
    assert oracle.gemm_h16_products(a[:, ::-1].copy(), b)[0, 0] == F32(2.0 ** -10)
    # operands are rounded to binary16 first: 1 + 2^-12 is 1 in binary16
    a = np.array([[1 + 2.0 ** -12]], F32)
    assert oracle.gemm_h16_products(a, np.ones((1, 1), F32))[0, 0] == 1.0


@pytest.mark.parametrize("gelu,half_output", [(False, False), (True, True)])
def test_linear_f16_is_rounded_operands_in_fp32(oracle, gelu, half_output):
    rng = np.random.default_rng(7 + gelu)
    x = rng.standard_normal((19, 64)).astype(F32)
    w = (rng.standard_normal((24, 64)) * 0.1).astype(F32)
    b = rng.standard_normal(24).astype(F32)
    got = oracle.linear_f16(x, w, b, gelu=gelu, half_output=half_output)
    exact = _h(x).astype(np.float64) @ _h(w).astype(np.float64).T + b
    if gelu:
        exact = oracle.gelu(exact.astype(F32)).astype(np.float64)
    tol = 2.0 ** -10 * np.abs(exact).max() if half_output else 1e-6 * np.abs(exact).max()
    assert np.abs(got - exact).max() <= tol
    if half_output:
        assert np.array_equal(got, got.astype(F16).astype(F32))  # binary16 values
    # unrounded operands would give 1 + 2^-12 + 2^-12
    x1 = np.array([[1 + 2.0 ** -12, 1.0]], F32)
    w1 = np.array([[1.0, 2.0 ** -12]], F32)
    assert oracle.linear_f16(x1, w1, None)[0, 0] == F32(1 + 2.0 ** -12)


def test_project_tokens_f16_matches_restatement(oracle):
    rng = np.random.default_rng(11)
    pw, ph, d, c = 5, 3, 32, 12
    tokens = rng.standard_normal((pw * ph + 1, d)).astype(F32)
    w = (rng.standard_normal((c, d)) * 0.2).astype(F32)
    b = rng.standard_normal(c).astype(F32)
    got = oracle.project_tokens_f16(tokens, w, b, pw, ph)
    # project_tokens_common.glsl: CLS skipped, sums over the embedding in order
    want = (_h16_products_numpy(tokens[1:], w) + b).T.reshape(c, ph, pw).astype(F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("k", [2, 4])
def test_conv_transpose_f16_matches_restatement(oracle, k):
    rng = np.random.default_rng(13 + k)
    ic, oc, ih, iw = 8, 6, 3, 4
    x = rng.standard_normal((ic, ih, iw)).astype(F32)
    w = (rng.standard_normal((ic, oc, k, k)) * 0.3).astype(F32)
    b = rng.standard_normal(oc).astype(F32)
    got = oracle.conv_transpose_f16(x, w, b)
    want = np.zeros((oc, ih * k, iw * k), F32)
    x16, w16 = _h(x), _h(w)
    for o in range(oc):
        for oy in range(ih * k):
            for ox in range(iw * k):
                s = F32(0)
                for c in range(ic):
                    s = F32(s + F32(x16[c, oy // k, ox // k] * w16[c, o, oy % k, ox % k]))
                want[o, oy, ox] = F32(s + b[o])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_prepare_tokens_f16_matches_restatement(oracle):
    rng = np.random.default_rng(17)
    width, height, d = 28, 14, 8
    image = rng.standard_normal((3, height, width)).astype(F32)
    w = (rng.standard_normal((d, 3, 14, 14)) * 0.05).astype(F32)
    b = rng.standard_normal(d).astype(F32)
    cls = rng.standard_normal(d).astype(F32)
    pos = rng.standard_normal((1370, d)).astype(F32)
    got = oracle.prepare_tokens_f16(image, w.reshape(d, -1), b, cls, pos, width, height)
    # prepare_tokens_fp16.glsl: patch rows in (channel, ky, kx) order, then
    # the position embedding as the fp32 path adds it
    pw, ph = width // 14, height // 14
    patches = np.stack([image[:, py * 14:(py + 1) * 14, px * 14:(px + 1) * 14].reshape(-1)
                        for py in range(ph) for px in range(pw)])
    sums = (_h16_products_numpy(patches, w.reshape(d, -1)) + b).astype(F32)
    base = oracle.prepare_tokens_f32(image, np.zeros_like(w.reshape(d, -1)), np.zeros(d, F32), cls, pos, width,
                                     height)  # class token + positions alone
    want = base.copy()
    want[1:] = (sums + base[1:]).astype(F32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))

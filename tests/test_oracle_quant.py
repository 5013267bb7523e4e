"""Pins the oracle's quantizers and int8 GEMM (CPU only).

quantize_rows_int8_fused.glsl:20-55, im2col_quantize_int8.glsl:26-83,
gpu_model.cpp:207-284, linear_int8_tiled.glsl:40-117. Checks are hand-derived
vectors (power-of-two scales so every quotient is exact), invariants, torch's
unfold for the im2col column order, and exact int64 matmul for the GEMM.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F


def test_quantize_rows_hand_vectors(oracle):
    x = np.array([
        [127.0, -63.5, 0.5, 1.5, -0.5, 2.5, -127.0, 0.0],  # scale 1: RNE ties, clamp edges
        [0.0] * 8,                                           # empty row -> 1e-8, zeros
        [1e-10, -2e-10, 0, 0, 0, 0, 0, 0],                   # tiny row -> scale floor 1e-8
        [254.0, 1.0, 2.0, 3.0, -5.0, 7.0, -254.0, 0.25],     # scale 2
    ], dtype=np.float32)
    q, s = oracle.quantize_rows(x)
    assert s.tolist() == [np.float32(1.0), np.float32(1e-8), np.float32(1e-8), np.float32(2.0)]
    assert q[0].tolist() == [127, -64, 0, 2, 0, 2, -127, 0]
    assert q[1].tolist() == [0] * 8
    assert q[2].tolist() == [0] * 8
    assert q[3].tolist() == [127, 0, 1, 2, -2, 4, -127, 0]


def near_tie_rows(rows: int, cols: int, seed: int) -> np.ndarray:
    """Rows whose quotients x / s fall within a few ulps of half-integers:
    column 0 holds the row maximum A (s = A / 127), the others are
    fl((k + 1/2) s) moved by -4..4 ulps, k in [-126, 125]."""
    rng = np.random.default_rng(seed)
    x = np.empty((rows, cols), np.float32)
    for r in range(rows):
        a = np.float32(rng.uniform(0.01, 50.0) * 2.0 ** rng.integers(-20, 20))
        s = np.float32(max(a / np.float32(127.0), np.float32(1e-8)))
        k = rng.integers(-126, 126, cols).astype(np.float32)
        base = ((k + np.float32(0.5)) * s).astype(np.float32)
        m = rng.integers(-4, 5, cols)
        v = base.copy()
        for step in range(4):
            v = np.where(m > step, np.nextafter(v, np.float32(np.inf)), v)
            v = np.where(m < -step, np.nextafter(v, np.float32(-np.inf)), v)
        v = np.clip(v, -a, a)
        v[0] = a
        x[r] = v
    return x


def test_quantize_by_product_with_guard_equals_quotient():
    # The GPU quantizers compute rne(clamp(x / s)) from x * fl(1 / s) and
    # divide only where that product lies within 2^-14 of a half-integer
    # (common.h quantize_div). Restated in float32 numpy against the IEEE
    # quotient on rows built to sit at ties and a few ulps beside them.
    x = near_tie_rows(64, 1024, 5)
    absmax = np.abs(x).max(axis=1)
    s = np.maximum(absmax / np.float32(127.0), np.float32(1e-8)).astype(np.float32)[:, None]
    want = np.rint(np.clip(x / s, -127, 127))
    inv = (np.float32(1.0) / s).astype(np.float32)
    y = (x * inv).astype(np.float32)
    n = np.rint(y)
    slow = np.abs(y - n) > np.float32(0.5) - np.float32(2.0 ** -14)
    got = np.where(slow, want, np.clip(n, -127, 127))
    assert np.array_equal(got, want)
    assert slow.mean() > 0.3  # the rows do exercise the division path
    # without the guard the product alone rounds some of them the other way
    assert not np.array_equal(np.clip(n, -127, 127), want)


def test_quantize_rows_input_offset_skips_prefix(oracle):
    # project_tokens_int8 passes input_offset = D to skip the class token
    # (operators.cpp:1514-1522).
    x = np.arange(3 * 8, dtype=np.float32).reshape(3, 8) - 7
    q_all, s_all = oracle.quantize_rows(x)
    q, s = oracle.quantize_rows(x, rows=2, columns=8, input_offset=8)
    assert np.array_equal(q, q_all[1:]) and np.array_equal(s, s_all[1:])


def test_quantize_rows_invariants(oracle):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal((257, 384)) * rng.uniform(0.01, 100, (257, 1))).astype(np.float32)
    q, s = oracle.quantize_rows(x)
    assert np.abs(q.astype(np.int32)).max() <= 127
    # the row maximum maps to +-127
    assert np.all(np.abs(q.astype(np.int32)).max(axis=1) == 127)
    np.testing.assert_array_equal(s, np.maximum(np.abs(x).max(axis=1) / np.float32(127), np.float32(1e-8)))
    # dequantization error at most half a step
    err = np.abs(q.astype(np.float64) * s[:, None] - x)
    assert np.all(err <= 0.5 * s[:, None] * (1 + 1e-5))


def test_weight_quantizer_matches_row_rule(oracle):
    # gpu_model.cpp:241-264 uses the same rule as the activation rows (w/s, RNE).
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((64, 96)) * 0.02).astype(np.float32)
    qw, sw = oracle.quantize_weight_rows(w)
    qr, sr = oracle.quantize_rows(w)
    assert np.array_equal(qw, qr) and np.array_equal(sw, sr)


def test_convT_weight_row_order(oracle):
    # gpu_model.cpp:226-240: row (ky*k+kx)*OC + oc holds w[:, oc, ky, kx].
    ic, oc, k = 8, 3, 2
    w = np.arange(ic * oc * k * k, dtype=np.float32).reshape(ic, oc, k, k) - 40.0
    q, s = oracle.quantize_convT_weight(w)
    rows = w.transpose(2, 3, 1, 0).reshape(k * k * oc, ic)
    q2, s2 = oracle.quantize_weight_rows(rows)
    assert np.array_equal(q, q2) and np.array_equal(s, s2)


@pytest.mark.parametrize("c,h,w,k,stride,pad", [(2, 5, 7, 3, 1, 1), (3, 28, 42, 14, 14, 0), (4, 9, 11, 3, 2, 1),
                                                (8, 6, 5, 1, 1, 0)])
def test_im2col_quantize_against_unfold(oracle, c, h, w, k, stride, pad):
    rng = np.random.default_rng(c * 100 + k)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    q, s = oracle.im2col_quantize(x, k, stride, pad)
    cols = F.unfold(torch.from_numpy(x)[None], kernel_size=k, padding=pad, stride=stride)[0].T.numpy()
    assert q.shape == cols.shape
    np.testing.assert_array_equal(s, np.maximum(np.abs(cols).max(axis=1) / np.float32(127), np.float32(1e-8)))
    err = np.abs(q.astype(np.float64) * s[:, None] - cols)
    assert np.all(err <= 0.5 * s[:, None] * (1 + 1e-5) + 1e-12)
    # zero padding taps quantize to exactly zero
    assert np.all(q[cols == 0] == 0)


def test_im2col_uses_reciprocal_multiply(oracle):
    # im2col_quantize_int8.glsl:68 multiplies by 1/s; pick a row where x*(1/s)
    # and x/s round differently: s = 3/127, x = 1.5 -> x/s vs x*(1/s).
    x = np.zeros((1, 1, 4), np.float32)
    vals = np.float32([3.0, 1.5, 0.75, -1.5])
    x[0, 0, :] = vals
    q, s = oracle.im2col_quantize(x, 1, 1, 0)  # rows = pixels, K = 1
    inv = np.float32(1.0) / s
    expect = np.rint(np.clip(vals * inv, -127, 127)).astype(np.int8)
    assert np.array_equal(q[:, 0], expect)


def test_gemm_int32_exact(oracle):
    rng = np.random.default_rng(11)
    for m, n, k in [(1, 1, 4), (37, 65, 588), (130, 96, 1152), (3, 200, 9216)]:
        a = rng.integers(-127, 128, (m, k), dtype=np.int8)
        b = rng.integers(-127, 128, (n, k), dtype=np.int8)
        acc = oracle.gemm_i8(a, b)
        ref = a.astype(np.int64) @ b.astype(np.int64).T
        assert np.array_equal(acc.astype(np.int64), ref)
    # extreme accumulator: K = 9216 of 127*127 stays below 2^31
    a = np.full((2, 9216), 127, np.int8)
    b = np.full((2, 9216), -127, np.int8)
    assert oracle.gemm_i8(a, b)[0, 0] == -9216 * 127 * 127


def test_linear_epilogue_layouts(oracle):
    rng = np.random.default_rng(5)
    acc = rng.integers(-10**6, 10**6, (6, 5)).astype(np.int32)
    si = rng.uniform(0.001, 0.1, 6).astype(np.float32)
    sw = rng.uniform(0.001, 0.1, 5).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    ref = acc.astype(np.float64) * si[:, None] * sw[None, :] + b[None, :]
    row = oracle.linear_epilogue(acc, si, sw, b, out_rows=7, row_offset=1).reshape(7, 5)
    assert np.all(row[0] == 0)
    np.testing.assert_allclose(row[1:], ref, rtol=3e-7, atol=1e-7)
    tr = oracle.linear_epilogue(acc, si, sw, b, out_rows=6, row_offset=0, row_stride=6, transposed=True)
    np.testing.assert_allclose(tr.reshape(5, 6).T, ref, rtol=3e-7, atol=1e-7)
    nob = oracle.linear_epilogue(acc, si, sw, None, out_rows=6).reshape(6, 5)
    np.testing.assert_allclose(nob, ref - b[None, :], rtol=3e-7, atol=1e-7)


def test_linear_int8_close_to_fp32(oracle):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((50, 256)).astype(np.float32)
    w = (rng.standard_normal((96, 256)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(96) * 0.01).astype(np.float32)
    wq, ws = oracle.quantize_weight_rows(w)
    y = oracle.linear_int8(x, wq, ws, b)
    ref = x.astype(np.float64) @ w.T.astype(np.float64) + b
    assert np.abs(y - ref).max() < 0.02 * np.abs(ref).max()
    g = oracle.linear_int8(x, wq, ws, b, gelu=True)
    np.testing.assert_allclose(g, F.gelu(torch.from_numpy(y)).numpy(), rtol=2e-6, atol=2e-7)

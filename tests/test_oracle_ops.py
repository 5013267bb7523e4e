"""Pins the CPU oracle's floating-point operators (CPU only): the reference's
own known-answer tests (tests/vulkan_smoke.cpp), float64 closed forms and
library routines (numpy, math.erf, torch.nn.functional), and invariants that a
dropped term, a wrong sign or index or a transposed operand would break."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle_py import pad_rows


def _ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


# --- exp (Cody-Waite + degree-7 Taylor) ------------------------------------------
def test_exp_within_one_ulp_of_float64(oracle):
    x = np.concatenate([np.linspace(-85.9, 88.7, 400001, dtype=np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 0.5, -0.5, 1.0, -1.0], np.float32)])
    got = oracle.exp(x)
    exact = np.exp(x.astype(np.float64)).astype(np.float32)  # correctly rounded reference
    assert _ulps(got, exact).max() <= 1
    assert oracle.exp(np.float32([0.0]))[0] == 1.0


def test_exp_range_ends(oracle):
    x = np.float32([-86.0, -100.0, -np.inf, 88.8, np.inf, np.nan])
    got = oracle.exp(x)
    assert got[0] == 0.0 and got[1] == 0.0 and got[2] == 0.0
    assert np.isinf(got[3]) and np.isinf(got[4]) and np.isnan(got[5])


# --- GELU (gelu.glsl: erfc fit) ------------------------------------------------
def test_gelu_matches_exact_erf_formula(oracle):
    x = np.concatenate([np.linspace(-12, 12, 100001, dtype=np.float32),
                        np.float32([0.0, 1e-20, -1e-20, 30.0, -30.0])])
    got = oracle.gelu(x).astype(np.float64)
    xd = x.astype(np.float64)
    exact = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in xd])
    # the fit's erf error is below 1.3e-7; the rest is float rounding
    assert np.all(np.abs(got - exact) <= 1.5e-7 * np.maximum(1.0, np.abs(xd)))
    assert oracle.gelu(np.float32([0.0]))[0] == 0.0


# --- LayerNorm (layer_norm.glsl) -----------------------------------------------
def test_layer_norm_reference_kat(oracle):
    # tests/vulkan_smoke.cpp:436-493
    rows, cols = 4, 17
    x = ((np.arange(rows * cols) % 23 - 10) * 0.125).astype(np.float32).reshape(rows, cols)
    got = oracle.layer_norm(x, np.ones(cols, np.float32), np.zeros(cols, np.float32))
    mean = x.sum(1, keepdims=True) / cols
    var = np.maximum((x * x).sum(1, keepdims=True) / cols - mean * mean, 0)
    assert np.abs(got - (x - mean) / np.sqrt(var + 1e-6)).max() <= 1e-5


def test_layer_norm_vs_torch_float64(oracle):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((300, 1024)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 1024).astype(np.float32)
    b = rng.uniform(-0.2, 0.2, 1024).astype(np.float32)
    got = oracle.layer_norm(x, w, b)
    ref = F.layer_norm(torch.from_numpy(x).double(), (1024,), torch.from_numpy(w).double(),
                       torch.from_numpy(b).double(), eps=1e-6).numpy()
    assert np.abs(got - ref).max() <= 2e-5


# --- add_scaled / add / relu -------------------------------------------------------
def test_add_scaled_reference_kat(oracle):
    # tests/vulkan_smoke.cpp:495-538: exact
    residual = (np.arange(15) * 0.125).astype(np.float32)
    addend = ((np.arange(15) + 2) * -0.0625).astype(np.float32)
    scale = ((np.arange(5) + 1) * 0.25).astype(np.float32)
    got = oracle.add_scaled(residual, addend, scale)
    assert np.array_equal(got, residual + addend * scale[np.arange(15) % 5])


def test_add_relu_exact(oracle):
    rng = np.random.default_rng(2)
    a, b = rng.standard_normal(1001).astype(np.float32), rng.standard_normal(1001).astype(np.float32)
    assert np.array_equal(oracle.add(a, b), a + b)
    assert np.array_equal(oracle.relu(a), np.maximum(a, 0))


# --- softmax / attention -------------------------------------------------------------
def test_softmax_rows_vs_float64(oracle):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((50, 1370)) * 4).astype(np.float32)
    got = oracle.softmax_rows(x)
    xd = x.astype(np.float64)
    ref = np.exp(xd - xd.max(1, keepdims=True))
    ref /= ref.sum(1, keepdims=True)
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=1e-9)
    assert np.abs(got.astype(np.float64).sum(1) - 1).max() <= 1e-5


def _attention_f64(qkv, tokens, heads):
    d = heads * 64
    q = qkv[:, :d].reshape(tokens, heads, 64).astype(np.float64)
    k = qkv[:, d:2 * d].reshape(tokens, heads, 64).astype(np.float64)
    v = qkv[:, 2 * d:].reshape(tokens, heads, 64).astype(np.float64)
    sc = np.einsum("ihf,jhf->hij", q * 0.125, k)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("hij,jhf->ihf", p, v).reshape(tokens, d)


def test_attention_reference_kat(oracle):
    # tests/vulkan_smoke.cpp:540-628: fp32 within 2e-6 of the closed form,
    # binary16 within 3e-4 of fp32
    tokens, heads = 5, 2
    qkv = ((np.arange(tokens * 3 * heads * 64) % 29 - 14) * 0.0078125).astype(np.float32)
    qkv = qkv.reshape(tokens, 3 * heads * 64)
    exact = _attention_f64(qkv, tokens, heads)
    out32 = oracle.attention(qkv, tokens, heads)
    assert np.abs(out32 - exact).max() <= 2e-6
    assert np.abs(oracle.attention(qkv, tokens, heads, fp16=True) - out32).max() <= 3e-4
    assert np.abs(oracle.attention(qkv, tokens, heads, fused=True) - exact).max() <= 3e-4


@pytest.mark.parametrize("tokens,heads", [(77, 4), (1370, 2)])
def test_attention_modes_vs_float64(oracle, tokens, heads):
    rng = np.random.default_rng(tokens)
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * 0.5).astype(np.float32)
    exact = _attention_f64(qkv, tokens, heads)
    assert np.abs(oracle.attention(qkv, tokens, heads) - exact).max() <= 2e-6
    assert np.abs(oracle.attention(qkv, tokens, heads, fp16=True) - exact).max() <= 1e-3
    assert np.abs(oracle.attention(qkv, tokens, heads, fused=True) - exact).max() <= 1e-4


def test_attention_exact_mode_is_order_free(oracle):
    # every sum of the integer-exact attention is an exact integer: permuting
    # the keys together with their values changes no bit of the output
    tokens, heads = 200, 3
    rng = np.random.default_rng(9)
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * 0.7).astype(np.float32)
    base = oracle.attention(qkv, tokens, heads, fused=True)
    perm = rng.permutation(tokens)
    d = heads * 64
    shuffled = qkv.copy()
    shuffled[:, d:] = qkv[perm, d:]  # keys and values move, queries stay
    assert np.array_equal(oracle.attention(shuffled, tokens, heads, fused=True).view(np.uint32),
                          base.view(np.uint32))


# --- binary16 attention (mode 1): the reference's int8-mode default ----------------
F16, F32 = np.float16, np.float32


def _coop_scores_numpy(q16_row, k16):
    """bmm_score_coop_fp16.glsl as the oracle states it: the exact products
    q16 * k16 summed in float64 in feature order, rounded to float32 (the
    accumulator's type), then to binary16."""
    s = np.zeros(k16.shape[0], np.float64)
    for f in range(64):
        s = s + np.float64(q16_row[f]) * k16[:, f].astype(np.float64)
    return s.astype(F32).astype(F16)


def _binary16_attention_numpy(oracle, qkv, tokens, heads, coop=False):
    """bmm_score_fp16.glsl (coop: bmm_score_coop_fp16.glsl as above),
    softmax_lastdim_half.glsl and bmm_value_fp16.glsl written loop for loop
    with numpy's IEEE float16 / float32 types (one query row at a time, every
    sum in the shaders' order). exp is the oracle's exp_cw (GLSL leaves exp's
    precision open; exp_cw is pinned against float64 in test_exp_cw_*)."""
    d = heads * 64
    out = np.zeros((tokens, d), F32)
    for h in range(heads):
        q16 = (qkv[:, h * 64:h * 64 + 64].astype(F32) * F32(0.125)).astype(F16)
        k16 = qkv[:, d + h * 64:d + h * 64 + 64].astype(F16)
        v16 = qkv[:, 2 * d + h * 64:2 * d + h * 64 + 64].astype(F16)
        for i in range(tokens):
            if coop:
                row = _coop_scores_numpy(q16[i], k16).astype(F32)
            else:
                # scores: s[j] += float(q16 * k16) for features 0..63 in order
                s = np.zeros(tokens, F32)
                for f in range(64):
                    s = (s + (q16[i, f].astype(F32) * k16[:, f].astype(F32)).astype(F16).astype(F32)).astype(F32)
                row = s.astype(F16).astype(F32)
            # softmax: 128 lanes over words (2w, 2w+1), then the halving tree
            m = row.max()
            e = oracle.exp((row - m).astype(F32))
            words = (tokens + 1) // 2
            part = np.zeros(128, F32)
            for lane in range(128):
                acc = F32(0)
                for w in range(lane, words, 128):
                    ex = e[2 * w]
                    ey = e[2 * w + 1] if 2 * w + 1 < tokens else F32(0)
                    acc = F32(acc + F32(ex + ey))
                part[lane] = acc
            stride = 64
            while stride:
                part[:stride] = (part[:stride] + part[stride:2 * stride]).astype(F32)
                stride //= 2
            inv = F32(F32(1) / max(part[0], F32(1e-20)))
            p16 = (e.astype(F16).astype(F32) * inv).astype(F16)
            # values: o[f] += float(p16[j] * v16[j][f]) for tokens j in order
            o = np.zeros(64, F32)
            for j in range(tokens):
                o = (o + (p16[j].astype(F32) * v16[j].astype(F32)).astype(F16).astype(F32)).astype(F32)
            out[i, h * 64:h * 64 + 64] = o
    return out


def test_round_half_product_matches_numpy(oracle):
    rng = np.random.default_rng(31)
    a = rng.standard_normal(1 << 20).astype(F16)
    b = (rng.standard_normal(1 << 20) * np.exp2(rng.integers(-14, 6, 1 << 20))).astype(F16)
    a[:8] = [F16(2.0 ** -12), F16(-1.0), F16(65504), F16(2.0 ** -14), 0, F16(1 + 2.0 ** -10), F16(3), F16(-0.0)]
    b[:8] = [F16(2.0 ** -12), F16(1 + 2.0 ** -9), F16(2), F16(2.0 ** -11), F16(-5), F16(1 + 2.0 ** -10), F16(1e-7), 1]
    want = (a.astype(F32) * b.astype(F32)).astype(F16).astype(F32)
    got = oracle.round_half_product(a.astype(F32), b.astype(F32))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _qkv_with(features_q, features_k, tokens=2, heads=1):
    """qkv rows for a score between query 0 and key 1 with the given q*0.125
    and k feature values (everything else zero)."""
    qkv = np.zeros((tokens, 3 * heads * 64), F32)
    for f, (q, k) in enumerate(zip(features_q, features_k)):
        qkv[0, f] = 8.0 * q
        qkv[1, heads * 64 + f] = k
    return qkv


def test_binary16_scores_round_each_product(oracle):
    # q*0.125 = 1 + 2^-10 times k = 1 + 2^-10 is 1 + 2^-9 + 2^-20 exactly, which
    # binary16 rounds to 1 + 2^-9; the second feature adds -(1 + 2^-9). Binary16
    # products give the score 0 exactly; exact products would give 2^-20 (a
    # binary16 subnormal, so the stored score would keep it).
    qkv = _qkv_with([1 + 2.0 ** -10, -1.0], [1 + 2.0 ** -10, 1 + 2.0 ** -9])
    s = oracle.scores_binary16(qkv, 2, 1)
    assert s[0, 0, 1] == 0.0
    assert F16(2.0 ** -20) != 0.0  # the exact-product score would survive storage
    # Feature order of the fp32 sum: 1, 2^-24, -1 in order gives 1 + 2^-24 = 1
    # (tie to even), then 0; the reversed order would give 2^-24 (the smallest
    # binary16 subnormal).
    qkv = _qkv_with([1.0, 2.0 ** -12, -1.0], [1.0, 2.0 ** -12, 1.0])
    assert oracle.scores_binary16(qkv, 2, 1)[0, 0, 1] == 0.0
    qkv = _qkv_with([-1.0, 2.0 ** -12, 1.0], [1.0, 2.0 ** -12, 1.0])  # -1 first: -1 + 2^-24 is exact
    assert oracle.scores_binary16(qkv, 2, 1)[0, 0, 1] == F16(2.0 ** -24)
    # the score is rounded to binary16 when stored: 1 + 2^-11 + 2^-12 -> 1 + 2^-10
    qkv = _qkv_with([1.0, 2.0 ** -11, 2.0 ** -12], [1.0, 1.0, 1.0])
    assert oracle.scores_binary16(qkv, 2, 1)[0, 0, 1] == F16(1 + 2.0 ** -10)


@pytest.mark.parametrize("tokens,heads", [(2, 1), (37, 2), (258, 1)])
def test_binary16_attention_matches_shader_restatement(oracle, tokens, heads):
    # T = 258: 129 packed words, so lane 0 of the softmax sums two words
    rng = np.random.default_rng(tokens + 100 * heads)
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * 1.5).astype(F32)
    want = _binary16_attention_numpy(oracle, qkv, tokens, heads)
    got = oracle.attention(qkv, tokens, heads, fp16=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_coop_scores_keep_exact_products(oracle):
    # bmm_score_coop_fp16.glsl multiplies binary16 operands without rounding
    # the products: (1 + 2^-10)^2 - (1 + 2^-9) = 2^-20, a binary16 subnormal
    # the stored score keeps (the per-product shader gives 0 here)
    qkv = _qkv_with([1 + 2.0 ** -10, -1.0], [1 + 2.0 ** -10, 1 + 2.0 ** -9])
    assert oracle.scores_coop(qkv, 2, 1)[0, 0, 1] == F16(2.0 ** -20)
    assert oracle.scores_binary16(qkv, 2, 1)[0, 0, 1] == 0.0
    # the sum passes through the fp32 accumulator before binary16: 1 + 2^-11
    # + 2^-30 is 1 + 2^-11 in fp32, a binary16 tie that rounds to even (1.0);
    # rounding the exact sum straight to binary16 would give 1 + 2^-10
    qkv = _qkv_with([1.0, 2.0 ** -11, 2.0 ** -15], [1.0, 1.0, 2.0 ** -15])
    assert oracle.scores_coop(qkv, 2, 1)[0, 0, 1] == F16(1.0)
    assert np.float64(1 + 2.0 ** -11 + 2.0 ** -30).astype(F16) == F16(1 + 2.0 ** -10)
    # the sign of a cancelling product pair: exact products cancel to 0
    qkv = _qkv_with([3.0, -3.0], [1 + 2.0 ** -10, 1 + 2.0 ** -10])
    assert oracle.scores_coop(qkv, 2, 1)[0, 0, 1] == 0.0


@pytest.mark.parametrize("tokens,heads", [(5, 1), (37, 2), (129, 1)])
def test_coop_scores_match_numpy(oracle, tokens, heads):
    rng = np.random.default_rng(tokens * 11 + heads)
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * 2.0).astype(F32)
    got = oracle.scores_coop(qkv, tokens, heads)
    d = heads * 64
    for h in range(heads):
        q16 = (qkv[:, h * 64:h * 64 + 64] * F32(0.125)).astype(F16)
        k16 = qkv[:, d + h * 64:d + h * 64 + 64].astype(F16)
        want = np.stack([_coop_scores_numpy(q16[i], k16) for i in range(tokens)])
        assert np.array_equal(got[h].view(np.uint16), want.view(np.uint16))
    # scores of magnitude ~10 differ from the per-product shader's somewhere
    assert (got != oracle.scores_binary16(qkv, tokens, heads)).any()


@pytest.mark.parametrize("tokens,heads", [(2, 1), (37, 2), (258, 1)])
def test_coop_attention_matches_shader_restatement(oracle, tokens, heads):
    rng = np.random.default_rng(tokens + 300 * heads)
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * 1.5).astype(F32)
    want = _binary16_attention_numpy(oracle, qkv, tokens, heads, coop=True)
    got = oracle.attention(qkv, tokens, heads, fp16=True, coop=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.abs(got - _attention_f64(qkv, tokens, heads)).max() <= 2e-2


def test_binary16_attention_differs_from_exact_products(oracle):
    # the binary16 rounding of every product is visible at this size: the
    # outputs are not those of exact products accumulated in fp32 (a
    # restatement that drops the product rounding fails here)
    tokens, heads = 64, 1
    rng = np.random.default_rng(77)
    qkv = (rng.standard_normal((tokens, 192)) * 2.0).astype(F32)
    got = oracle.attention(qkv, tokens, heads, fp16=True)
    d = 64
    q16 = (qkv[:, :64] * F32(0.125)).astype(F16).astype(np.float64)
    k16 = qkv[:, 64:128].astype(F16).astype(np.float64)
    exact_scores = (q16 @ k16.T).astype(F32).astype(F16).astype(F32)
    # scores alone already differ somewhere in binary16
    binary16_scores = np.zeros_like(exact_scores)
    for i in range(tokens):
        s = np.zeros(tokens, F32)
        for f in range(d):
            s = (s + (F32(q16[i, f]) * k16[:, f].astype(F32)).astype(F16).astype(F32)).astype(F32)
        binary16_scores[i] = s.astype(F16).astype(F32)
    assert (binary16_scores != exact_scores).any()
    # binary16 scores of magnitude up to ~30 carry 2^-6 steps: a loose sanity
    # bound against float64 attention
    assert np.abs(got - _attention_f64(qkv, tokens, heads)).max() <= 2e-2


def test_numerator21_vs_float64(oracle):
    # E(x) = rint(min(2^x 2^21, 2^21 - 1)) up to the polynomial's rounding:
    # within 0.5 + 2.5e-7 * 2^(x+21) of the float64 value, exact integers,
    # 0 below -100 and for -inf, 2^21 - 1 at the top
    x = np.concatenate([np.linspace(-40.0, 0.0, 400001), -np.logspace(-9, 0, 2001),
                        np.linspace(-0.5, 0.5, 1001)]).astype(np.float32)
    e = oracle.numerator21(x)
    want = np.minimum(np.exp2(x.astype(np.float64) + 21.0), 2097151.0)
    assert np.all(e == np.rint(e))
    assert np.all(np.abs(e - want) <= 0.5 + 2.5e-7 * want)
    assert np.abs(e - want).max() >= 0.4  # the test sees real roundings
    far = np.array([-100.5, -1e4, -3e38, -np.inf], np.float32)
    assert np.all(oracle.numerator21(far) == 0.0)
    assert np.all(oracle.numerator21(np.array([0.0, 1e-6, 0.03], np.float32)) == 2097151.0)


def test_numerator21_vector_form_matches_scalar(oracle):
    # The eight-wide form the oracle's attention uses for speed gives the
    # scalar numerator21's bits: dense and random arguments, half-integers
    # (ties of the rounding to an integer exponent), the clamp at -100,
    # -inf and NaN.
    rng = np.random.default_rng(21)
    x = np.concatenate([np.linspace(-101.0, 0.5, 2000003), rng.uniform(-110.0, 0.6, 2000000),
                        np.arange(-100.5, 1.0, 0.5), np.nextafter(np.arange(-100.5, 1.0, 0.5), 0.0),
                        np.nextafter(np.arange(-100.5, 1.0, 0.5), -1.0),
                        [-np.inf, np.nan, -3e38, 0.0, -0.0, 1e-30]]).astype(np.float32)
    scalar = oracle.numerator21(x)
    vec = np.empty_like(x)
    oracle.lib.orc_numerator21_x8(x.ctypes.data, x.size, vec.ctypes.data)
    assert np.array_equal(vec.view(np.uint32), scalar.view(np.uint32))


def test_attention_exact_mode_uniform_keys(oracle):
    # identical keys: every probability is 1/T, the output is the mean of the
    # (15-bit block floating point) values
    tokens, heads = 64, 1
    rng = np.random.default_rng(4)
    qkv = rng.standard_normal((tokens, 192)).astype(np.float32)
    qkv[:, 64:128] = qkv[0, 64:128]
    out, p = oracle.attention(qkv, tokens, heads, fused=True, probabilities=True)
    assert np.all(p == p[0, 0, 0])
    assert np.abs(out - qkv[:, 128:].mean(0)).max() <= 2e-4 * np.abs(qkv[:, 128:]).max()


# --- resize, min/max, normalisation, position -----------------------------------------
@pytest.mark.parametrize("ih,iw,oh,ow", [(37, 37, 74, 74), (296, 296, 518, 518), (19, 23, 37, 41), (5, 5, 5, 5)])
def test_bilinear_align_corners_vs_torch(oracle, ih, iw, oh, ow):
    rng = np.random.default_rng(ih + ow)
    x = rng.standard_normal((3, ih, iw)).astype(np.float32)
    got = oracle.bilinear(x, ow, oh)
    ref = F.interpolate(torch.from_numpy(x)[None].double(), size=(oh, ow), mode="bilinear",
                        align_corners=True)[0].numpy()
    # the shader forms the source coordinate in fp32: an error of up to about
    # one ulp of the coordinate times the largest neighbour difference
    step = max(np.abs(np.diff(x, axis=1)).max(), np.abs(np.diff(x, axis=2)).max()) if min(ih, iw) > 1 else 0.0
    assert np.abs(got - ref).max() <= 2e-6 + 4 * step * max(ih, iw) * 2.0 ** -23


def test_minmax_normalize_reference_kat(oracle):
    # tests/vulkan_smoke.cpp:119-139
    d = np.float32([2.0, 3.0, 5.0, 10.0])
    r = oracle.reduce_minmax(d)
    assert r.tolist() == [2.0, 10.0]
    assert np.abs(oracle.normalize_relative(d, r) - [0.0, 0.125, 0.375, 1.0]).max() <= 1e-6
    rng = np.random.default_rng(8)
    x = rng.standard_normal(268324).astype(np.float32)
    r = oracle.reduce_minmax(x)
    assert r[0] == x.min() and r[1] == x.max()
    n = oracle.normalize_relative(x, r)
    assert n.min() == 0.0 and n.max() == 1.0
    assert np.abs(n - (x.astype(np.float64) - r[0]) / (r[1] - r[0])).max() <= 1e-6


@pytest.mark.parametrize("pw,ph", [(37, 37), (21, 21), (74, 74), (25, 19)])
def test_position_bicubic_vs_torch(oracle, pw, ph):
    # upstream interpolate_pos_encoding: bicubic, scale_factor (P + 0.1) / 37,
    # align_corners=False; the reference copies the grid unchanged at 37x37
    dim = 6
    rng = np.random.default_rng(pw * ph)
    pos = rng.standard_normal((1370, dim)).astype(np.float32)
    got = oracle.position_bicubic(pos, pw, ph, dim)
    grid = torch.from_numpy(pos[1:]).double().reshape(1, 37, 37, dim).permute(0, 3, 1, 2)
    if pw == 37 and ph == 37:
        assert np.array_equal(got, pos[1:].T.reshape(dim, 37, 37))
        return
    ref = F.interpolate(grid, scale_factor=((ph + 0.1) / 37, (pw + 0.1) / 37), mode="bicubic",
                        align_corners=False)[0].numpy()
    assert ref.shape == got.shape
    assert np.abs(got - ref).max() <= 2e-5


# --- int8 operators vs fp32 -------------------------------------------------------------
def test_conv2d_int8_reference_kat(oracle):
    # tests/vulkan_smoke.cpp:143-186: within 0.006 of the fp32 convolution
    width, height, channels, outputs, k = 5, 4, 4, 5, 3
    x = ((np.arange(width * height * channels) % 23 - 11) * 0.03125).astype(np.float32).reshape(channels, height,
                                                                                               width)
    w = ((np.arange(outputs * channels * 9) % 19 - 9) * 0.015625).astype(np.float32).reshape(outputs, channels, k, k)
    b = (np.arange(outputs) * 0.01).astype(np.float32)
    q, s = oracle.quantize_weight_rows(w)
    got = oracle.conv2d_int8(x, q, s, b, outputs, k, 1, 1)
    ref = F.conv2d(torch.from_numpy(x)[None], torch.from_numpy(w), torch.from_numpy(b), padding=1)[0].numpy()
    assert np.abs(got - ref).max() <= 0.006


def test_conv_transpose_int8_reference_kat(oracle):
    # tests/vulkan_smoke.cpp:187-240: within 0.004 of the fp32 transposed convolution
    width, height, inputs, outputs, k = 3, 2, 4, 3, 2
    x = ((np.arange(width * height * inputs) % 17 - 8) * 0.03125).astype(np.float32).reshape(inputs, height, width)
    w = ((np.arange(inputs * outputs * k * k) % 13 - 6) * 0.02).astype(np.float32).reshape(inputs, outputs, k, k)
    q, s = oracle.quantize_convT_weight(w)
    got = oracle.conv_transpose_int8(x, q, s, np.zeros(outputs, np.float32), outputs, k)
    ref = F.conv_transpose2d(torch.from_numpy(x)[None], torch.from_numpy(w), stride=k)[0].numpy()
    assert np.abs(got - ref).max() <= 0.004


@pytest.mark.parametrize("c,h,w,oc,k,stride,pad", [(32, 13, 11, 24, 3, 1, 1), (64, 9, 9, 16, 3, 2, 1),
                                                   (48, 7, 5, 8, 1, 1, 0)])
def test_conv2d_int8_close_to_fp32(oracle, c, h, w, oc, k, stride, pad):
    rng = np.random.default_rng(c + oc)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    wt = (rng.uniform(-1, 1, (oc, c, k, k)) / np.sqrt(c * k * k)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, oc).astype(np.float32)
    q, s = oracle.quantize_weight_rows(wt)
    got = oracle.conv2d_int8(x, q, s, b, oc, k, stride, pad)
    ref = F.conv2d(torch.from_numpy(x)[None], torch.from_numpy(wt), torch.from_numpy(b), stride=stride,
                   padding=pad)[0].numpy()
    # per-row activation and per-channel weight quantization: a few percent of the output scale
    assert np.abs(got - ref).max() <= 0.03 * np.abs(ref).max()
    # a transposed weight layout or a shifted window would not come close
    assert np.abs(got - ref).mean() <= 0.005 * np.abs(ref).max()


def test_prepare_tokens_reference_kat(oracle):
    # tests/vulkan_smoke.cpp:630-754: zero image and weights, so every patch
    # token is bias + bicubic position and the class token is class + position[0]
    width, height, dim = 42, 28, 3
    bias = np.float32([0.25, -0.5, 0.75])
    cls = np.float32([1.0, 2.0, 3.0])
    pos = ((np.arange(1370 * dim) % 31 - 15) * 0.015625).astype(np.float32).reshape(1370, dim)
    wq, ws = oracle.quantize_weight_rows(np.zeros((dim, 3, 14, 14), np.float32))
    tokens = oracle.prepare_tokens_int8(np.zeros((3, height, width), np.float32), wq, ws, bias, cls, pos, width,
                                        height, dim)
    assert np.array_equal(tokens[0], cls + pos[0])
    interp = oracle.position_bicubic(pos, width // 14, height // 14, dim)
    assert np.array_equal(tokens[1:], (interp.reshape(dim, -1).T + bias).astype(np.float32))


def test_project_tokens_int8_layout(oracle):
    # the class token is skipped and the output is channel-major [C][ph][pw]
    pw, ph, dim, ch = 5, 3, 64, 8
    rng = np.random.default_rng(6)
    tokens = rng.standard_normal((pw * ph + 1, dim)).astype(np.float32)
    w = (rng.standard_normal((ch, dim)) * 0.1).astype(np.float32)
    b = rng.standard_normal(ch).astype(np.float32) * 0.1
    q, s = oracle.quantize_weight_rows(w)
    got = oracle.project_tokens_int8(tokens, q, s, b, pw, ph, dim, ch)
    ref = (tokens[1:] @ w.T + b).T.reshape(ch, ph, pw)
    assert np.abs(got - ref).max() <= 0.03 * np.abs(ref).max()
    assert np.array_equal(got, oracle.linear_int8(tokens[1:], pad_rows(q)[:, :dim], s, b).T.reshape(ch, ph, pw))

"""The oracle's fp32 precision-mode operators (src/operators.cpp:882-955,
:1211-1452, :1528-1676, :1807-1861) against independent float64
implementations: numpy products and torch's CPU convolutions."""

import numpy as np
import pytest

torch = pytest.importorskip("torch")
F = torch.nn.functional


def _rel(got, want):
    return float(np.abs(got - want).max() / max(np.abs(want).max(), 1e-30))


def test_linear_f32(oracle):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((37, 96)).astype(np.float32)
    w = (rng.standard_normal((80, 96)) * 0.1).astype(np.float32)
    b = rng.standard_normal(80).astype(np.float32)
    got = oracle.linear_f32(x, w, b)
    want = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert _rel(got, want) < 1e-5
    g = oracle.linear_f32(x, w, b, gelu=True)
    assert np.array_equal(g, oracle.gelu(got))  # GELU on the same fp32 sums
    assert np.array_equal(oracle.linear_f32(x, w, None), oracle.linear_f32(x, w, np.zeros(80, np.float32)))


@pytest.mark.parametrize("c,oc,k,stride,pad,h,w", [(8, 12, 3, 1, 1, 11, 9), (16, 8, 3, 2, 1, 13, 10),
                                                   (8, 4, 1, 1, 0, 7, 7), (3, 16, 14, 14, 0, 28, 42)])
def test_conv2d_f32_matches_torch(oracle, c, oc, k, stride, pad, h, w):
    rng = np.random.default_rng(c * 10 + k)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c, k, k)) * 0.2).astype(np.float32)
    b = rng.standard_normal(oc).astype(np.float32)
    got = oracle.conv2d_f32(x, wt, b, stride, pad)
    want = F.conv2d(torch.from_numpy(x).double()[None], torch.from_numpy(wt).double(), torch.from_numpy(b).double(),
                    stride=stride, padding=pad)[0].numpy()
    assert got.shape == want.shape and _rel(got, want) < 1e-5
    nob = oracle.conv2d_f32(x, wt, None, stride, pad)
    assert _rel(nob, want - b[:, None, None]) < 1e-5


@pytest.mark.parametrize("k", [2, 4])
def test_conv_transpose_f32_matches_torch(oracle, k):
    rng = np.random.default_rng(k)
    x = rng.standard_normal((12, 5, 7)).astype(np.float32)
    wt = (rng.standard_normal((12, 6, k, k)) * 0.2).astype(np.float32)
    b = rng.standard_normal(6).astype(np.float32)
    got = oracle.conv_transpose_f32(x, wt, b)
    want = F.conv_transpose2d(torch.from_numpy(x).double()[None], torch.from_numpy(wt).double(),
                              torch.from_numpy(b).double(), stride=k)[0].numpy()
    assert got.shape == want.shape and _rel(got, want) < 1e-5


def test_project_tokens_f32(oracle):
    rng = np.random.default_rng(5)
    pw, ph, d, c = 6, 4, 32, 10
    tokens = rng.standard_normal((pw * ph + 1, d)).astype(np.float32)
    w = rng.standard_normal((c, d)).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    got = oracle.project_tokens_f32(tokens, w, b, pw, ph)
    want = (tokens[1:].astype(np.float64) @ w.T.astype(np.float64) + b).T.reshape(c, ph, pw)
    assert _rel(got, want) < 1e-5


def test_prepare_tokens_f32(oracle):
    # patch conv (k = s = 14) + class token + bicubic position, composed from
    # independently pinned parts
    rng = np.random.default_rng(6)
    width, height, d = 42, 28, 16
    image = rng.standard_normal((3, height, width)).astype(np.float32)
    w = (rng.standard_normal((d, 3, 14, 14)) * 0.05).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    cls = rng.standard_normal(d).astype(np.float32)
    pos = rng.standard_normal((1370, d)).astype(np.float32)
    got = oracle.prepare_tokens_f32(image, w, b, cls, pos, width, height)
    pw, ph = width // 14, height // 14
    patches = oracle.conv2d_f32(image, w, b, 14, 0).reshape(d, -1).T
    interp = oracle.position_bicubic(pos, pw, ph, d).reshape(d, -1).T
    assert np.array_equal(got[0], cls + pos[0])
    assert np.array_equal(got[1:], patches + interp)

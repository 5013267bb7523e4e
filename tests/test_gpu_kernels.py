"""HIP kernels vs the CPU oracle, through the C-ABI launchers (include/dav2_hip.h).

Integer stages (int8 bytes, scales, int32 accumulators) must match bit for
bit; fp32 stages whose GPU code evaluates the same expression order match
bit for bit too, the rest within the stated tolerances.
"""

import ctypes as C
import sys

import numpy as np
import pytest

from gpu_util import dev, empty, host, ok, ptr, stream
from oracle_py import pack_conv_weights, pad_rows

pytestmark = pytest.mark.gpu


def _announce(*what):
    print("case:", *what, flush=True)
    sys.stdout.flush()


# ---------------------------------------------------------------------------
# quantize_rows_int8_fused.glsl
@pytest.mark.parametrize("rows,cols,offset_rows", [(1370, 384, 0), (1370, 1024, 0), (1369, 4096, 0), (7, 8, 0),
                                                   (3, 8192, 0), (1369, 1024, 1), (1, 1536, 0),
                                                   # many rows: the row-looping kernel (odd wave tails)
                                                   (10960, 1024, 0), (4099, 384, 2), (5000, 100, 0)])
def test_quantize_rows_bit_exact(gpu, lib, oracle, rows, cols, offset_rows):
    torch = gpu
    _announce("quantize_rows", rows, cols, offset_rows)
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows + offset_rows, cols)) * rng.uniform(0.01, 30, (rows + offset_rows, 1))).astype(np.float32)
    if rows > 2:
        x[offset_rows + 1] = 0.0  # an all-zero row
    q_ref, s_ref = oracle.quantize_rows(x, rows, cols, offset_rows * cols)
    ld = (cols + 63) // 64 * 64
    xd = dev(torch, x)
    qd = torch.full((rows, ld), 0x55, dtype=torch.int8, device="cuda")
    sd = empty(torch, (rows,), torch.float32)
    ok(lib, lib.dav2_hip_quantize_rows_i8(ptr(xd), offset_rows * cols, rows, cols, ptr(qd), ld, ptr(sd), stream(torch)))
    q = host(torch, qd)
    assert np.array_equal(q[:, :cols], q_ref)
    assert np.all(q[:, cols:] == 0)
    assert np.array_equal(host(torch, sd).view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("rows,cols,offset_rows", [(37, 4096, 2), (300, 4096, 0), (9, 3072, 1), (17, 1536, 0),
                                                   (5, 1000, 3), (3, 100, 0)])
def test_gelu_quantize_rows_bit_exact(gpu, lib, oracle, rows, cols, offset_rows):
    # the row quantized is gelu(x): the oracle's GELU pass, then its row quantizer
    torch = gpu
    _announce("gelu quantize_rows", rows, cols, offset_rows)
    rng = np.random.default_rng(rows * cols + 7)
    x = (rng.standard_normal((rows + offset_rows, cols)) * rng.uniform(0.01, 12, (rows + offset_rows, 1))).astype(np.float32)
    x[offset_rows] = 0.0  # an all-zero row
    if rows > 2:
        x[offset_rows + 1] = -np.abs(x[offset_rows + 1]) - 20.0  # gelu flushes the whole row to (almost) zero
    g = oracle.gelu(x)
    q_ref, s_ref = oracle.quantize_rows(g, rows, cols, offset_rows * cols)
    ld = (cols + 63) // 64 * 64
    xd = dev(torch, x)
    qd = torch.full((rows, ld), 0x55, dtype=torch.int8, device="cuda")
    sd = empty(torch, (rows,), torch.float32)
    ok(lib, lib.dav2_hip_gelu_quantize_rows_i8(ptr(xd), offset_rows * cols, rows, cols, ptr(qd), ld, ptr(sd),
                                              stream(torch)))
    q = host(torch, qd)
    assert np.array_equal(q[:, :cols], q_ref)
    assert np.all(q[:, cols:] == 0)
    assert np.array_equal(host(torch, sd).view(np.uint32), s_ref.view(np.uint32))
    # rows longer than the register-resident kernel holds are rejected
    assert lib.dav2_hip_gelu_quantize_rows_i8(ptr(xd), 0, 1, 4100, ptr(qd), 4160, ptr(sd), stream(torch)) != 0


def test_quantize_rows_packed_word_byte_order(gpu, lib):
    # quantize_rows_int8_fused.glsl:51: byte k of word w is column 4w+k.
    torch = gpu
    x = np.array([[254.0, 1.0, 2.0, 3.0, -254.0, -2.0, 4.0, 0.0]], np.float32)
    xd = dev(torch, x)
    qd = empty(torch, (1, 64), torch.int8)
    sd = empty(torch, (1,), torch.float32)
    ok(lib, lib.dav2_hip_quantize_rows_i8(ptr(xd), 0, 1, 8, ptr(qd), 64, ptr(sd), stream(torch)))
    words = host(torch, qd).view(np.uint32)[0, :2]
    assert words.tolist() == [0x0201007F, 0x0002FF81]
    assert host(torch, sd)[0] == np.float32(2.0)


@pytest.mark.parametrize("cols", [100, 1024, 2048, 4096, 20000])
def test_quantize_rows_near_ties(gpu, lib, oracle, cols):
    # quotients within a few ulps of half-integers: the kernels' product path
    # must hand these to the IEEE division (bit-exact against the oracle)
    from test_oracle_quant import near_tie_rows
    torch = gpu
    _announce("quantize_rows near ties", cols)
    x = near_tie_rows(24, cols, cols)
    q_ref, s_ref = oracle.quantize_rows(x)
    ld = (cols + 63) // 64 * 64
    xd = dev(torch, x)
    qd = torch.full((24, ld), 0x55, dtype=torch.int8, device="cuda")
    sd = empty(torch, (24,), torch.float32)
    ok(lib, lib.dav2_hip_quantize_rows_i8(ptr(xd), 0, 24, cols, ptr(qd), ld, ptr(sd), stream(torch)))
    assert np.array_equal(host(torch, qd)[:, :cols], q_ref)
    assert np.array_equal(host(torch, sd).view(np.uint32), s_ref.view(np.uint32))


# ---------------------------------------------------------------------------
# im2col_quantize_int8.glsl
@pytest.mark.parametrize("c,h,w,k,s,p", [(3, 518, 518, 14, 14, 0), (3, 266, 350, 14, 14, 0), (64, 37, 37, 3, 1, 1),
                                         (96, 19, 19, 3, 2, 1), (32, 74, 74, 1, 1, 0), (5, 4, 4, 3, 1, 1),
                                         (128, 60, 52, 3, 1, 1), (1024, 10, 10, 3, 2, 1), (1024, 19, 19, 3, 1, 1),
                                         (128, 130, 141, 3, 1, 1), (16, 3, 70, 3, 1, 1), (512, 37, 37, 1, 1, 0),
                                         (48, 5, 7, 1, 1, 0), (256, 150, 150, 3, 1, 1), (64, 100, 100, 1, 1, 0),
                                         (8, 91, 93, 3, 2, 1), (2048, 9, 9, 3, 1, 1), (1024, 38, 38, 3, 1, 1),
                                         (512, 13, 11, 3, 1, 1), (700, 5, 9, 3, 2, 1)])
def test_im2col_quantize_bit_exact(gpu, lib, oracle, c, h, w, k, s, p):
    torch = gpu
    _announce("im2col", c, h, w, k, s, p)
    rng = np.random.default_rng(c + h + k)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    q_ref, s_ref = oracle.im2col_quantize(x, k, s, p)
    ow = (w + 2 * p - k) // s + 1
    oh = (h + 2 * p - k) // s + 1
    kk = c * k * k
    ld = (kk + 63) // 64 * 64
    xd = dev(torch, x)
    n_scratch = lib.dav2_hip_im2col_scratch_floats(w, h, c)
    scratch = empty(torch, (n_scratch,), torch.float32)
    # generic gather kernels (no scratch), then the tiled 3x3 / 1x1 kernels
    for sp, sn in ((None, 0), (ptr(scratch), n_scratch)):
        qd = torch.full((ow * oh, ld), 0x55, dtype=torch.int8, device="cuda")
        sd = empty(torch, (ow * oh,), torch.float32)
        ok(lib, lib.dav2_hip_im2col_quantize_i8(ptr(xd), w, h, c, ow, oh, k, s, p, ptr(qd), ld, ptr(sd), sp, sn,
                                                stream(torch)))
        q = host(torch, qd)
        assert np.array_equal(host(torch, sd).view(np.uint32), s_ref.view(np.uint32))
        assert np.array_equal(q[:, :kk], q_ref)
        assert np.all(q[:, kk:] == 0)


@pytest.mark.parametrize("c,h,w,k", [(256, 37, 37, 3), (1024, 19, 19, 3), (16, 3, 70, 3), (256, 37, 37, 1),
                                     (48, 5, 7, 1), (64, 100, 100, 3), (64, 100, 100, 1)])
def test_im2col_quantize_relu_bit_exact(gpu, lib, oracle, c, h, w, k):
    # the fused ReLU quantizes exactly the rows of max(x, 0)
    torch = gpu
    _announce("im2col relu", c, h, w, k)
    rng = np.random.default_rng(c + h + 3 * k)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    p = (k - 1) // 2
    q_ref, s_ref = oracle.im2col_quantize(np.maximum(x, 0.0), k, 1, p)
    kk = c * k * k
    ld = (kk + 63) // 64 * 64
    xd = dev(torch, x)
    n_scratch = lib.dav2_hip_im2col_scratch_floats(w, h, c)
    scratch = empty(torch, (n_scratch,), torch.float32)
    qd = torch.full((w * h, ld), 0x55, dtype=torch.int8, device="cuda")
    sd = empty(torch, (w * h,), torch.float32)
    ok(lib, lib.dav2_hip_im2col_quantize_relu_i8(ptr(xd), w, h, c, w, h, k, 1, p, ptr(qd), ld, ptr(sd), ptr(scratch),
                                                 n_scratch, stream(torch)))
    q = host(torch, qd)
    assert np.array_equal(host(torch, sd).view(np.uint32), s_ref.view(np.uint32))
    assert np.array_equal(q[:, :kk], q_ref)
    assert np.all(q[:, kk:] == 0)
    # x itself is unchanged. Without scratch, maps of up to 8192 output pixels
    # (the single-pass path) give the same bytes; larger ones refuse.
    assert np.array_equal(host(torch, xd), x)
    qd.fill_(0x55)
    rc = lib.dav2_hip_im2col_quantize_relu_i8(ptr(xd), w, h, c, w, h, k, 1, p, ptr(qd), ld, ptr(sd), None, 0,
                                              stream(torch))
    if w * h <= 8192:
        assert rc == 0
        assert np.array_equal(host(torch, sd).view(np.uint32), s_ref.view(np.uint32))
        assert np.array_equal(host(torch, qd)[:, :kk], q_ref)
    else:
        assert rc != 0


# ---------------------------------------------------------------------------
# implicit-GEMM convolution == im2col_quantize_int8.glsl + linear_int8_tiled.glsl
# (CHW store), bit for bit. Shapes cover every channel-tile configuration the
# launchers pick (256/128/64/32 output channels per workgroup), the two-row
# 3x3 kernel (even widths: tiles of 60 columns, an odd height leaving a tile's
# second row outside, one and three channel blocks) and the one-row kernel
# (odd widths), maps narrower than one tile, one-row maps and 1x1 kernels.
@pytest.mark.parametrize("c,h,w,n,k,has_bias", [(64, 37, 37, 256, 3, True), (128, 9, 150, 32, 3, True),
                                                (256, 166, 180, 256, 3, True), (64, 100, 300, 128, 3, False),
                                                (64, 250, 128, 64, 3, True), (64, 1, 5, 32, 3, True),
                                                (192, 19, 19, 96, 3, True), (64, 37, 37, 96, 1, True),
                                                (128, 100, 330, 128, 1, True), (128, 518, 518, 32, 3, True),
                                                (192, 19, 20, 96, 3, True), (64, 3, 6, 32, 3, True),
                                                (64, 7, 121, 64, 3, True), (256, 75, 74, 256, 3, True),
                                                (128, 4, 62, 128, 3, False), (64, 1, 64, 256, 3, True),
                                                # 128 output channels over >= 512 tiles: single-buffered
                                                (128, 208, 244, 128, 3, False)])
def test_conv2d_i8_matches_im2col_gemm(gpu, pkg, lib, oracle, c, h, w, n, k, has_bias):
    torch = gpu
    _announce("conv2d_i8", c, h, w, n, k, has_bias)
    assert lib.dav2_hip_conv2d_i8_supported(w, h, c, n, k, 1, (k - 1) // 2)
    rng = np.random.default_rng(c * 31 + h + n + k)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    x[:, h // 2, :] *= 40.0  # rows with a larger range, so scales differ between pixels
    kk = c * k * k
    ld = (kk + 63) // 64 * 64
    wq, ws = oracle.quantize_weight_rows(rng.standard_normal((n, kk)).astype(np.float32) * 0.05)
    bias = rng.standard_normal(n).astype(np.float32)
    xd, wqd, wsd, bd = dev(torch, x), dev(torch, pad_rows(wq, ld)), dev(torch, ws), dev(torch, bias)
    s = stream(torch)
    n_scratch = lib.dav2_hip_im2col_scratch_floats(w, h, c)
    scratch = empty(torch, (n_scratch,), torch.float32)

    # reference path: tiled im2col + GEMM with the channel-major epilogue
    rows = h * w
    qd = empty(torch, (rows, ld), torch.int8)
    sd = empty(torch, (rows,), torch.float32)
    ok(lib, lib.dav2_hip_im2col_quantize_i8(ptr(xd), w, h, c, w, h, k, 1, (k - 1) // 2, ptr(qd), ld, ptr(sd),
                                            ptr(scratch), n_scratch, s))
    ref = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    args = _gemm_args(pkg, a=ptr(qd), lda=ld, b=ptr(wqd), ldb=ld, m=rows, n=n, k=ld, epilogue=pkg.GEMM_EPI["transposed"],
                      a_scales=ptr(sd), b_scales=ptr(wsd), bias=ptr(bd) if has_bias else None, out=ptr(ref),
                      out_row_stride=rows)
    ok(lib, lib.dav2_hip_gemm_i8(C.byref(args), s))

    # packed weights: tap-major K (dst k = t*c + ic holds src[o][ic*k*k + t])
    # in 16 x 64-byte MFMA operand fragments
    wt = empty(torch, (n, kk), torch.int8)
    ok(lib, lib.dav2_hip_conv_weights_pack(ptr(wt), ptr(wqd), n, c, k, ld, s))
    assert np.array_equal(host(torch, wt), pack_conv_weights(wq, n, c, k))

    out = torch.full((n, rows), float("nan"), dtype=torch.float32, device="cuda")
    a = pkg.ConvArgs(input=ptr(xd), width=w, height=h, channels=c, kernel=k, weight=ptr(wt), weight_scales=ptr(wsd),
                     bias=ptr(bd) if has_bias else None, out_channels=n, out=ptr(out), scratch=ptr(scratch),
                     scratch_floats=n_scratch)
    ok(lib, lib.dav2_hip_conv2d_i8(C.byref(a), s))
    got, want = host(torch, out), host(torch, ref)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{np.count_nonzero(got.view(np.uint32) != want.view(np.uint32))} of {got.size} outputs differ"


def test_conv2d_i8_matches_oracle(gpu, pkg, lib, oracle):
    # the CPU oracle's conv2d_int8 (im2col + int8 GEMM + CHW epilogue)
    torch = gpu
    _announce("conv2d_i8 oracle")
    rng = np.random.default_rng(5)
    c, h, w, n = 64, 21, 70, 64
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    wq, ws = oracle.quantize_weight_rows(rng.standard_normal((n, c * 9)).astype(np.float32) * 0.05)
    bias = rng.standard_normal(n).astype(np.float32)
    want = oracle.conv2d_int8(x, wq, ws, bias, n, 3, 1, 1).reshape(n, h * w)
    wt = pack_conv_weights(wq, n, c, 3)
    n_scratch = lib.dav2_hip_im2col_scratch_floats(w, h, c)
    scratch = empty(torch, (n_scratch,), torch.float32)
    xd, wtd, wsd, bd = dev(torch, x), dev(torch, wt), dev(torch, ws), dev(torch, bias)
    out = empty(torch, (n, h * w), torch.float32)
    a = pkg.ConvArgs(input=ptr(xd), width=w, height=h, channels=c, kernel=3, weight=ptr(wtd), weight_scales=ptr(wsd),
                     bias=ptr(bd), out_channels=n, out=ptr(out), scratch=ptr(scratch), scratch_floats=n_scratch)
    ok(lib, lib.dav2_hip_conv2d_i8(C.byref(a), stream(torch)))
    assert np.array_equal(host(torch, out).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("flags,with_residual", [(1, False), (2, False), (3, False), (0, True), (2, True)])
@pytest.mark.parametrize("c,h,w,n", [(128, 20, 90, 128), (64, 90, 150, 256), (128, 9, 61, 64)])
def test_conv2d_i8_fusions(gpu, pkg, lib, oracle, flags, with_residual, c, h, w, n):
    # relu(input) -> conv -> + residual -> relu, each step as its own kernel
    # (relu.glsl, add.glsl), against the flags of the fused kernel: the
    # single-buffered 128-channel tiles, the double-buffered 256-channel ones
    # and the one-row kernel of odd widths.
    torch = gpu
    _announce("conv2d_i8 fusions", flags, with_residual, c, h, w, n)
    rng = np.random.default_rng(flags * 7 + with_residual)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    res = rng.standard_normal((n, h * w)).astype(np.float32)
    wq, ws = oracle.quantize_weight_rows(rng.standard_normal((n, c * 9)).astype(np.float32) * 0.05)
    wt = pack_conv_weights(wq, n, c, 3)
    bias = rng.standard_normal(n).astype(np.float32)
    xd, wtd, wsd, bd, rd = dev(torch, x), dev(torch, wt), dev(torch, ws), dev(torch, bias), dev(torch, res)
    s = stream(torch)
    n_scratch = lib.dav2_hip_im2col_scratch_floats(w, h, c)
    scratch = empty(torch, (n_scratch,), torch.float32)

    def conv(inp, out, fl, resid):
        a = pkg.ConvArgs(input=ptr(inp), width=w, height=h, channels=c, kernel=3, weight=ptr(wtd), weight_scales=ptr(wsd),
                         bias=ptr(bd), out_channels=n, out=ptr(out), scratch=ptr(scratch), scratch_floats=n_scratch,
                         flags=fl, residual=ptr(resid) if resid is not None else None)
        ok(lib, lib.dav2_hip_conv2d_i8(C.byref(a), s))

    src = xd
    if flags & 1:
        src = empty(torch, xd.shape, torch.float32)
        ok(lib, lib.dav2_hip_relu(ptr(src), ptr(xd), xd.numel(), s))
    want = empty(torch, (n, h * w), torch.float32)
    conv(src, want, 0, None)
    if with_residual:
        ok(lib, lib.dav2_hip_add(ptr(want), ptr(want), ptr(rd), want.numel(), s))
    if flags & 2:
        ok(lib, lib.dav2_hip_relu(ptr(want), ptr(want), want.numel(), s))
    got = empty(torch, (n, h * w), torch.float32)
    conv(xd, got, flags, rd if with_residual else None)
    assert np.array_equal(host(torch, got).view(np.uint32), host(torch, want).view(np.uint32))


def _group_max(x, relu):
    """Per-pixel maxima over 32-channel groups of a [C][P] map."""
    m = np.maximum(x, 0) if relu else np.abs(x)
    return m.reshape(x.shape[0] // 32, 32, -1).max(axis=1)


@pytest.mark.parametrize("k,n,relu_in,emit", [(3, 256, True, 4), (3, 128, False, 8), (1, 256, False, 8),
                                              (1, 128, True, 4)])
def test_conv2d_i8_group_maxima(gpu, pkg, lib, oracle, k, n, relu_in, emit):
    # EMIT_*: the output's 32-channel group maxima written by the epilogue
    # equal those of the output; partial_in: the same output as maxima
    # computed by the kernel itself.
    torch = gpu
    _announce("conv2d_i8 group maxima", k, n, relu_in, emit)
    c, h, w = 128, 9, 77
    rng = np.random.default_rng(k * n + emit)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    wq, ws = oracle.quantize_weight_rows(rng.standard_normal((n, c * k * k)).astype(np.float32) * 0.05)
    wt = pack_conv_weights(wq, n, c, k)
    bias = rng.standard_normal(n).astype(np.float32)
    xd, wtd, wsd, bd = dev(torch, x), dev(torch, wt), dev(torch, ws), dev(torch, bias)
    s = stream(torch)
    n_scratch = lib.dav2_hip_im2col_scratch_floats(w, h, c)
    scratch = empty(torch, (n_scratch,), torch.float32)
    assert lib.dav2_hip_conv2d_i8_emits(n, k) == 1 and lib.dav2_hip_conv2d_i8_emits(64, k) == 0
    fl = 1 if relu_in else 0

    def conv(out, flags, partial_in=None, partial_out=None):
        a = pkg.ConvArgs(input=ptr(xd), width=w, height=h, channels=c, kernel=k, weight=ptr(wtd),
                         weight_scales=ptr(wsd), bias=ptr(bd), out_channels=n, out=ptr(out), scratch=ptr(scratch),
                         scratch_floats=n_scratch, flags=flags, residual=None,
                         partial_in=ptr(partial_in) if partial_in is not None else None,
                         partial_out=ptr(partial_out) if partial_out is not None else None)
        return lib.dav2_hip_conv2d_i8(C.byref(a), s)

    want = empty(torch, (n, h * w), torch.float32)
    ok(lib, conv(want, fl))
    got = empty(torch, (n, h * w), torch.float32)
    maxima = empty(torch, (n // 32, h * w), torch.float32)
    ok(lib, conv(got, fl | emit, partial_out=maxima))
    ref = host(torch, want)
    assert np.array_equal(host(torch, got).view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(host(torch, maxima), _group_max(ref, relu=(emit == 8)))
    # the input's maxima given by a producer instead of computed here
    pin = dev(torch, _group_max(x.reshape(c, -1), relu=relu_in))
    again = empty(torch, (n, h * w), torch.float32)
    ok(lib, conv(again, fl, partial_in=pin))
    assert np.array_equal(host(torch, again).view(np.uint32), ref.view(np.uint32))
    # both emit modes at once, or an emit without a buffer, are rejected
    assert conv(got, fl | 12, partial_out=maxima) != 0
    assert conv(got, fl | 4) != 0


@pytest.mark.parametrize("c,ih,iw,oh,ow", [(128, 296, 296, 518, 518), (256, 37, 37, 74, 74), (32, 5, 7, 9, 13),
                                           (64, 148, 148, 296, 296), (32, 19, 19, 37, 37), (32, 9, 13, 17, 25),
                                           (32, 10, 10, 10, 10), (32, 1, 1, 5, 3), (32, 7, 3, 7, 200),
                                           (32, 40, 40, 20, 20), (32, 30, 5, 7, 50)])
def test_bilinear_maxima(gpu, lib, c, ih, iw, oh, ow):
    # the 32-channel resize with maxima: the same bits as the plain resize
    # (up- and downsampling, ragged tiles, one-pixel sources)
    torch = gpu
    _announce("bilinear maxima", c, ih, iw, oh, ow)
    x = np.random.default_rng(c + oh).standard_normal((c, ih, iw)).astype(np.float32)
    xd = dev(torch, x)
    plain = empty(torch, (c, oh * ow), torch.float32)
    fused = empty(torch, (c, oh * ow), torch.float32)
    maxima = empty(torch, (c // 32, oh * ow), torch.float32)
    s = stream(torch)
    ok(lib, lib.dav2_hip_bilinear_align_true(ptr(plain), ptr(xd), iw, ih, ow, oh, c, s))
    ok(lib, lib.dav2_hip_bilinear_align_true_maxima(ptr(fused), ptr(maxima), ptr(xd), iw, ih, ow, oh, c, s))
    ref = host(torch, plain)
    assert np.array_equal(host(torch, fused).view(np.uint32), ref.view(np.uint32))
    assert np.array_equal(host(torch, maxima), _group_max(ref, relu=False))


# 32 channels on an even plane take the two-pixel kernel (also with three
# outputs and both ReLUs); odd planes and other channel counts the other
@pytest.mark.parametrize("c,h,w,n,flags", [(32, 518, 518, 1, 2), (32, 20, 33, 1, 0), (32, 6, 10, 3, 3), (32, 7, 9, 4, 3),
                                           (64, 7, 9, 3, 1), (12, 5, 5, 4, 3)])
def test_conv1x1_narrow_matches_im2col_gemm(gpu, pkg, lib, oracle, c, h, w, n, flags):
    torch = gpu
    _announce("conv1x1 narrow", c, h, w, n, flags)
    rng = np.random.default_rng(c + h + n)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    ld = (c + 63) // 64 * 64
    wq, ws = oracle.quantize_weight_rows(rng.standard_normal((n, c)).astype(np.float32) * 0.2)
    bias = rng.standard_normal(n).astype(np.float32)
    xd, wqd, wsd, bd = dev(torch, x), dev(torch, pad_rows(wq, ld)), dev(torch, ws), dev(torch, bias)
    s = stream(torch)
    rows = h * w
    src = xd
    if flags & 1:
        src = empty(torch, xd.shape, torch.float32)
        ok(lib, lib.dav2_hip_relu(ptr(src), ptr(xd), xd.numel(), s))
    qd = empty(torch, (rows, ld), torch.int8)
    sd = empty(torch, (rows,), torch.float32)
    n_scratch = lib.dav2_hip_im2col_scratch_floats(w, h, c)
    scratch = empty(torch, (n_scratch,), torch.float32)
    ok(lib, lib.dav2_hip_im2col_quantize_i8(ptr(src), w, h, c, w, h, 1, 1, 0, ptr(qd), ld, ptr(sd), ptr(scratch),
                                            n_scratch, s))
    want = empty(torch, (n, rows), torch.float32)
    args = _gemm_args(pkg, a=ptr(qd), lda=ld, b=ptr(wqd), ldb=ld, m=rows, n=n, k=ld, epilogue=pkg.GEMM_EPI["transposed"],
                      a_scales=ptr(sd), b_scales=ptr(wsd), bias=ptr(bd), out=ptr(want), out_row_stride=rows)
    ok(lib, lib.dav2_hip_gemm_i8(C.byref(args), s))
    pre = host(torch, want).copy()
    if flags & 2:
        ok(lib, lib.dav2_hip_relu(ptr(want), ptr(want), want.numel(), s))
    got = empty(torch, (n, rows), torch.float32)
    got_pre = empty(torch, (n, rows), torch.float32)
    ok(lib, lib.dav2_hip_conv1x1_narrow_i8(ptr(xd), w, h, c, ptr(wqd), ld, ptr(wsd), ptr(bd), n, ptr(got), ptr(got_pre),
                                           flags, s))
    assert np.array_equal(host(torch, got).view(np.uint32), host(torch, want).view(np.uint32))
    assert np.array_equal(host(torch, got_pre).view(np.uint32), pre.view(np.uint32))


def test_conv2d_i8_rejects_unsupported(gpu, pkg, lib):
    torch = gpu
    for args in [(10, 10, 48, 32, 3, 1, 1), (10, 10, 64, 48, 3, 1, 1), (10, 10, 64, 32, 3, 2, 1), (10, 10, 64, 32, 5, 1, 2),
                 (10, 10, 64, 32, 1, 1, 1)]:
        assert not lib.dav2_hip_conv2d_i8_supported(*args)
    x = torch.zeros(64 * 100, dtype=torch.float32, device="cuda")
    a = pkg.ConvArgs(input=ptr(x), width=10, height=10, channels=48, kernel=3, weight=ptr(x), weight_scales=ptr(x),
                     bias=None, out_channels=32, out=ptr(x), scratch=ptr(x), scratch_floats=100)
    assert lib.dav2_hip_conv2d_i8(C.byref(a), stream(torch)) != 0
    a.channels = 64
    a.scratch_floats = 10  # fewer than width * height * groups
    assert lib.dav2_hip_conv2d_i8(C.byref(a), stream(torch)) != 0


# ---------------------------------------------------------------------------
# int8 GEMM (linear_int8_tiled.glsl), raw int32 accumulators
def _gemm_args(pkg, **kw):
    a = pkg.GemmArgs()
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("m,n,k", [(1370, 1152, 384), (1370, 3072, 1024), (1369, 384, 588), (17, 33, 64),
                                   (4096, 256, 2304), (1370, 1024, 4096), (130, 1, 32), (21904, 256, 2304)])
def test_gemm_int32_bit_exact(gpu, pkg, lib, m, n, k):
    torch = gpu
    _announce("gemm raw", m, n, k)
    rng = np.random.default_rng(m * 7 + n)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    ref = (a.astype(np.int64) @ b.astype(np.int64).T)
    ld = (k + 63) // 64 * 64
    ad, bd = dev(torch, pad_rows(a, ld)), dev(torch, pad_rows(b, ld))
    out = torch.full((m, n), -1, dtype=torch.int32, device="cuda")
    args = _gemm_args(pkg, a=ptr(ad), lda=ld, b=ptr(bd), ldb=ld, m=m, n=n, k=ld, epilogue=pkg.GEMM_EPI["raw"],
                      out_i32=ptr(out))
    ok(lib, lib.dav2_hip_gemm_i8(C.byref(args), stream(torch)))
    assert np.array_equal(host(torch, out).astype(np.int64), ref)


def _random_gemm_case(rng, m, n, k):
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    sa = rng.uniform(1e-3, 5e-2, m).astype(np.float32)
    sb = rng.uniform(1e-4, 2e-3, n).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32) * 0.1
    return a, b, sa, sb, bias


# (4100, 200, 192) and (4097, 1001, 128) take the 64x128 tiles of M >= 4096:
# ragged M, N not a multiple of 128 (200) and not of 4 (1001, element stores),
# a partial K stage (192); (4100, 3100, 192), (4097, 3073, 128) and
# (6000, 4096, 1024) the 128x128 eight-wave tiles of N >= 3072; (1370, 4096,
# 256) and (700, 4100, 192) the 128x64 eight-wave tiles of N >= 4096 below
# M = 4096;
# (1370, 1024, 4096) and (300, 96, 2112): long K (fc2), the second with a
# partial last stage; (4100, 1024, 4096) and (4097, 1020, 4224): the
# 32x32x32 kernel of M >= 4096, K >= 4096 on 192-row tiles (ROW and
# LayerScale; ragged M and N), (4100, 3000, 4096) on 256-row tiles (one round
# of 204 tiles against two of 264); (4097, 1001, 4224): N % 4 != 0, which it
# leaves to gemm_i8_kernel
@pytest.mark.parametrize("m,n,k", [(1370, 384, 384), (1369, 96, 640), (300, 1024, 1024), (5477, 384, 384),
                                   (4100, 200, 192), (4097, 1001, 128), (4100, 3100, 192), (4097, 3073, 128),
                                   (6000, 4096, 1024), (1370, 4096, 256), (700, 4100, 192), (1370, 1024, 4096),
                                   (300, 96, 2112), (4100, 1024, 4096), (4097, 1020, 4224),
                                   (4100, 3000, 4096), (4097, 1001, 4224)])
def test_gemm_row_epilogues(gpu, pkg, lib, oracle, m, n, k):
    torch = gpu
    _announce("gemm epilogues", m, n, k)
    rng = np.random.default_rng(n + k)
    a, b, sa, sb, bias = _random_gemm_case(rng, m, n, k)
    acc = oracle.gemm_i8(a, b)
    ld = (k + 63) // 64 * 64
    ad, bd = dev(torch, pad_rows(a, ld)), dev(torch, pad_rows(b, ld))
    sad, sbd, biasd = dev(torch, sa), dev(torch, sb), dev(torch, bias)
    s = stream(torch)
    base = dict(a=ptr(ad), lda=ld, b=ptr(bd), ldb=ld, m=m, n=n, k=ld, a_scales=ptr(sad), b_scales=ptr(sbd))

    # ROW with bias and a row offset (prepare_tokens writes rows 1..T-1)
    out = torch.zeros((m + 1, n), dtype=torch.float32, device="cuda")
    ok(lib, lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **base, epilogue=1, bias=ptr(biasd), out=ptr(out),
                                                    out_row_offset=1)), s))
    ref = oracle.linear_epilogue(acc, sa, sb, bias, out_rows=m + 1, row_offset=1).reshape(m + 1, n)
    got = host(torch, out)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))

    # ROW without bias
    out0 = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    ok(lib, lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **base, epilogue=1, out=ptr(out0))), s))
    ref0 = oracle.linear_epilogue(acc, sa, sb, None, out_rows=m).reshape(m, n)
    assert np.array_equal(host(torch, out0).view(np.uint32), ref0.view(np.uint32))

    # TRANSPOSED (channel-major, row stride m)
    outt = torch.zeros((n, m), dtype=torch.float32, device="cuda")
    ok(lib, lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **base, epilogue=4, bias=ptr(biasd), out=ptr(outt),
                                                    out_row_stride=m)), s))
    reft = oracle.linear_epilogue(acc, sa, sb, bias, out_rows=m, row_stride=m, transposed=True).reshape(n, m)
    assert np.array_equal(host(torch, outt).view(np.uint32), reft.view(np.uint32))

    # ROW + GELU (erfc fit and exp evaluated by the same IEEE sequence): exact
    outg = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    ok(lib, lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **base, epilogue=2, bias=ptr(biasd), out=ptr(outg))), s))
    refg = oracle.gelu(oracle.linear_epilogue(acc, sa, sb, bias, out_rows=m).reshape(m, n))
    assert np.array_equal(host(torch, outg).view(np.uint32), refg.view(np.uint32))

    # ROW + LayerScale residual, in place (add_scaled.glsl arithmetic)
    resid = rng.standard_normal((m, n)).astype(np.float32)
    gamma = rng.uniform(-1e-3, 1e-3, n).astype(np.float32)
    outr = dev(torch, resid)
    gd = dev(torch, gamma)
    ok(lib, lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **base, epilogue=3, bias=ptr(biasd), out=ptr(outr),
                                                    residual=ptr(outr), gamma=ptr(gd))), s))
    refr = oracle.add_scaled(resid, oracle.linear_epilogue(acc, sa, sb, bias, out_rows=m).reshape(m, n), gamma)
    assert np.array_equal(host(torch, outr).view(np.uint32), refr.view(np.uint32))


@pytest.mark.parametrize("m,n,k,begin", [(1370, 3072, 1024, 1024), (1369, 2304, 384, 768), (300, 1024, 256, 512),
                                         (20, 192, 64, 64), (1, 128, 64, 0)])
def test_gemm_colmax_epilogue(gpu, pkg, lib, oracle, m, n, k, begin):
    # ROW output, plus per row tile the max |out| of each column >= begin
    # (max is exact, so the partials equal numpy's over the same rows).
    torch = gpu
    _announce("gemm colmax", m, n, k, begin)
    rng = np.random.default_rng(m + n + begin)
    a, b, sa, sb, bias = _random_gemm_case(rng, m, n, k)
    acc = oracle.gemm_i8(a, b)
    ld = (k + 63) // 64 * 64
    ad, bd = dev(torch, pad_rows(a, ld)), dev(torch, pad_rows(b, ld))
    sad, sbd, biasd = dev(torch, sa), dev(torch, sb), dev(torch, bias)
    tiles = lib.dav2_hip_gemm_i8_row_tiles(m, n, 6)
    bm = 32 if m <= 32 else (96 if n >= 2048 and m >= 512 else 64)
    assert tiles == -(-m // bm)
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    cmax = torch.full((tiles, n - begin), -1.0, dtype=torch.float32, device="cuda")
    base = dict(a=ptr(ad), lda=ld, b=ptr(bd), ldb=ld, m=m, n=n, k=ld, a_scales=ptr(sad), b_scales=ptr(sbd),
                bias=ptr(biasd), out=ptr(out), epilogue=6)
    ok(lib, lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **base, col_absmax=ptr(cmax), col_absmax_begin=begin)),
                                 stream(torch)))
    ref = oracle.linear_epilogue(acc, sa, sb, bias, out_rows=m).reshape(m, n)
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))
    want = np.stack([np.abs(ref[t * bm:(t + 1) * bm, begin:]).max(axis=0) for t in range(tiles)])
    assert np.array_equal(host(torch, cmax), want)
    for bad in (dict(col_absmax=ptr(cmax), col_absmax_begin=begin + 32), dict(col_absmax=ptr(cmax), col_absmax_begin=n),
                dict(col_absmax=None, col_absmax_begin=begin)):
        assert lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **base, **bad)), stream(torch)) != 0


@pytest.mark.parametrize("m,n,k", [(1369, 256, 2304), (361, 256, 9216), (37, 96, 576)])
def test_gemm_transposed_residual_relu(gpu, pkg, lib, oracle, m, n, k):
    # channel-major output + residual (add.glsl) then max(., 0) (relu.glsl)
    torch = gpu
    _announce("gemm transposed residual relu", m, n, k)
    rng = np.random.default_rng(m + n)
    a, b, sa, sb, bias = _random_gemm_case(rng, m, n, k)
    acc = oracle.gemm_i8(a, b)
    ld = (k + 63) // 64 * 64
    ad, bd = dev(torch, pad_rows(a, ld)), dev(torch, pad_rows(b, ld))
    sad, sbd, biasd = dev(torch, sa), dev(torch, sb), dev(torch, bias)
    conv = oracle.linear_epilogue(acc, sa, sb, bias, out_rows=m, row_stride=m, transposed=True).reshape(n, m)
    resid = (rng.standard_normal((n, m)) * np.abs(conv).mean()).astype(np.float32)
    rd = dev(torch, resid)
    base = dict(a=ptr(ad), lda=ld, b=ptr(bd), ldb=ld, m=m, n=n, k=ld, a_scales=ptr(sad), b_scales=ptr(sbd),
                bias=ptr(biasd), epilogue=4, out_row_stride=m)
    for res, relu in ((True, False), (False, True), (True, True)):
        out = torch.full((n, m), float("nan"), dtype=torch.float32, device="cuda")
        ok(lib, lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **base, out=ptr(out), residual=ptr(rd) if res else None,
                                                        relu_output=int(relu))), stream(torch)))
        want = oracle.add(conv, resid) if res else conv.copy()
        if relu:
            want = oracle.relu(want)
        assert np.array_equal(host(torch, out).view(np.uint32), want.view(np.uint32)), (res, relu)
    # relu_output belongs to the channel-major epilogue only
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    bad = dict(base, epilogue=1)
    assert lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **bad, out=ptr(out), relu_output=1)), stream(torch)) != 0


@pytest.mark.parametrize("m,n,k,split", [(361, 256, 2304, 8), (1369, 256, 9216, 3), (361, 1024, 9216, 3),
                                         (37, 96, 576, 2), (361, 256, 2304, 5), (100, 64, 192, 4)])
def test_gemm_split_k_matches_single_pass(gpu, pkg, lib, oracle, m, n, k, split):
    # K in slices on more workgroups, slices added as int32 (exact): the same
    # bits as one pass, with and without residual / ReLU
    torch = gpu
    _announce("gemm split-k", m, n, k, split)
    rng = np.random.default_rng(m + n + split)
    a, b, sa, sb, bias = _random_gemm_case(rng, m, n, k)
    acc = oracle.gemm_i8(a, b)
    ld = (k + 63) // 64 * 64
    ad, bd = dev(torch, pad_rows(a, ld)), dev(torch, pad_rows(b, ld))
    sad, sbd, biasd = dev(torch, sa), dev(torch, sb), dev(torch, bias)
    conv = oracle.linear_epilogue(acc, sa, sb, bias, out_rows=m, row_stride=m, transposed=True).reshape(n, m)
    resid = (rng.standard_normal((n, m)) * np.abs(conv).mean()).astype(np.float32)
    rd = dev(torch, resid)
    nbytes = lib.dav2_hip_gemm_i8_split_scratch_bytes(m, n, split)
    assert nbytes == split * m * n * 4
    scratch = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda")
    base = dict(a=ptr(ad), lda=ld, b=ptr(bd), ldb=ld, m=m, n=n, k=ld, a_scales=ptr(sad), b_scales=ptr(sbd),
                bias=ptr(biasd), epilogue=4, out_row_stride=m, split_k=split, split_scratch=ptr(scratch))
    for res, relu in ((False, False), (True, True)):
        out = torch.full((n, m), float("nan"), dtype=torch.float32, device="cuda")
        ok(lib, lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **base, out=ptr(out), residual=ptr(rd) if res else None,
                                                        relu_output=int(relu))), stream(torch)))
        want = oracle.add(conv, resid) if res else conv.copy()
        if relu:
            want = oracle.relu(want)
        assert np.array_equal(host(torch, out).view(np.uint32), want.view(np.uint32)), (res, relu)
    # split-K belongs to the channel-major epilogue and needs its scratch
    out = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    assert lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **dict(base, epilogue=1), out=ptr(out))), stream(torch)) != 0
    assert lib.dav2_hip_gemm_i8(C.byref(_gemm_args(pkg, **dict(base, split_scratch=None), out=ptr(out))),
                                stream(torch)) != 0


def test_gemm_rejects_bad_arguments(gpu, pkg, lib):
    torch = gpu
    a = torch.zeros((4, 64), dtype=torch.int8, device="cuda")
    out = torch.zeros((4, 4), dtype=torch.int32, device="cuda")
    bad_k = _gemm_args(pkg, a=ptr(a), lda=64, b=ptr(a), ldb=64, m=4, n=4, k=60, epilogue=0, out_i32=ptr(out))
    assert lib.dav2_hip_gemm_i8(C.byref(bad_k), stream(torch)) != 0
    bad_epi = _gemm_args(pkg, a=ptr(a), lda=64, b=ptr(a), ldb=64, m=4, n=4, k=64, epilogue=9, out_i32=ptr(out))
    assert lib.dav2_hip_gemm_i8(C.byref(bad_epi), stream(torch)) != 0


# ---------------------------------------------------------------------------
# LayerNorm (+ fused quantization)
@pytest.mark.parametrize("rows,cols", [(1370, 384), (1370, 1024), (4, 17), (10, 768), (3, 5000), (2, 4096)])
def test_layer_norm_bit_exact(gpu, lib, oracle, rows, cols):
    torch = gpu
    _announce("layer_norm", rows, cols)
    rng = np.random.default_rng(rows + cols)
    x = (rng.standard_normal((rows, cols)) * 3 + 1).astype(np.float32)
    w = rng.uniform(0.5, 1.5, cols).astype(np.float32)
    b = rng.standard_normal(cols).astype(np.float32) * 0.1
    ref = oracle.layer_norm(x, w, b, 1e-6)
    xd, wd, bd = dev(torch, x), dev(torch, w), dev(torch, b)
    out = empty(torch, (rows, cols), torch.float32)
    ok(lib, lib.dav2_hip_layer_norm(ptr(out), ptr(xd), ptr(wd), ptr(bd), rows, cols, 1e-6, stream(torch)))
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))
    if cols % 4 == 0 and cols <= 4096:
        ld = (cols + 63) // 64 * 64
        qd = torch.full((rows, ld), 0x33, dtype=torch.int8, device="cuda")
        sd = empty(torch, (rows,), torch.float32)
        out2 = empty(torch, (rows, cols), torch.float32)
        ok(lib, lib.dav2_hip_layer_norm_quantize_i8(ptr(qd), ld, ptr(sd), ptr(out2), ptr(xd), ptr(wd), ptr(bd), rows,
                                                     cols, 1e-6, stream(torch)))
        q_ref, s_ref = oracle.quantize_rows(ref)
        q = host(torch, qd)
        assert np.array_equal(q[:, :cols], q_ref) and np.all(q[:, cols:] == 0)
        assert np.array_equal(host(torch, sd).view(np.uint32), s_ref.view(np.uint32))
        assert np.array_equal(host(torch, out2).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("cols", [384, 1024, 1536])
def test_layer_norm_quantize_near_ties(gpu, lib, oracle, cols):
    # weight 0 makes every normalised value the bias exactly, so the quantizer
    # sees quotients within a few ulps of half-integers (CH path for 384 and
    # 1024 columns, the re-reading path for 1536)
    from test_oracle_quant import near_tie_rows
    torch = gpu
    _announce("layer_norm_quantize near ties", cols)
    rows = 6
    b = near_tie_rows(1, cols, cols + 1)[0]
    x = np.random.default_rng(cols).standard_normal((rows, cols)).astype(np.float32)
    w = np.zeros(cols, np.float32)
    ref = oracle.layer_norm(x, w, b, 1e-6)
    assert np.array_equal(ref, np.broadcast_to(b, ref.shape))
    q_ref, s_ref = oracle.quantize_rows(ref)
    ld = (cols + 63) // 64 * 64
    xd, wd, bd = dev(torch, x), dev(torch, w), dev(torch, b)
    qd = torch.full((rows, ld), 0x33, dtype=torch.int8, device="cuda")
    sd = empty(torch, (rows,), torch.float32)
    ok(lib, lib.dav2_hip_layer_norm_quantize_i8(ptr(qd), ld, ptr(sd), 0, ptr(xd), ptr(wd), ptr(bd), rows, cols, 1e-6,
                                                 stream(torch)))
    q = host(torch, qd)
    assert np.array_equal(q[:, :cols], q_ref) and np.all(q[:, cols:] == 0)
    assert np.array_equal(host(torch, sd).view(np.uint32), s_ref.view(np.uint32))


@pytest.mark.parametrize("rows,cols,ld", [(384, 588, 640), (64, 432, 448), (1, 4, 16), (7, 36, 4096), (3, 64, 64)])
def test_pad_rows_i8(gpu, lib, rows, cols, ld):
    # reference GpuModel int8 rows ([rows][cols] bytes) to the GEMM layout
    torch = gpu
    rng = np.random.default_rng(rows + cols)
    q = rng.integers(-127, 128, (rows, cols), dtype=np.int8)
    src = dev(torch, q)
    dst = torch.full((rows, ld), 0x55, dtype=torch.int8, device="cuda")
    ok(lib, lib.dav2_hip_pad_rows_i8(ptr(src), rows, cols, ptr(dst), ld, stream(torch)))
    got = host(torch, dst)
    assert np.array_equal(got[:, :cols], q) and np.all(got[:, cols:] == 0)
    assert lib.dav2_hip_pad_rows_i8(ptr(src), rows, cols, ptr(dst), cols - 4, stream(torch)) != 0


# ---------------------------------------------------------------------------
# attention: scores -> softmax -> values
def _attention_mfma_gpu(torch, lib, qkv, tokens, heads):
    """fp32 attention on the matrix cores (the fp32 precision mode's path)."""
    qd = dev(torch, qkv)
    nbytes = lib.dav2_hip_attention_scratch_bytes(tokens, heads, 1, 0)
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out = empty(torch, (tokens, heads * 64), torch.float32)
    s = stream(torch)
    ok(lib, lib.dav2_hip_attention_scores(ptr(buf), ptr(qd), tokens, heads, 1, 0, s))
    ok(lib, lib.dav2_hip_softmax_rows(ptr(buf), heads * tokens, tokens, tokens, 0, s))
    ok(lib, lib.dav2_hip_attention_values(ptr(out), ptr(buf), ptr(qd), tokens, heads, 1, 0, s))
    probs = host(torch, buf[: heads * tokens * tokens * 4].view(torch.float32).reshape(heads, tokens, tokens))
    return host(torch, out), probs


def _attention_ref_gpu(torch, lib, qkv, tokens, heads, fp16, batch=1, unpacked=True, coop=False):
    """The reference-order kernels (coop: the cooperative-matrix scores);
    returns the output, the probabilities ([batch*H][T][T] as float32) and
    the scores before the softmax (None, None without `unpacked`)."""
    qd = dev(torch, qkv)
    nbytes = lib.dav2_hip_attention_ref_scratch_bytes(tokens, heads, batch, int(fp16))
    words = (tokens + 1) // 2
    assert nbytes == batch * heads * tokens * (words * 4 if fp16 else tokens * 4)  # the reference's size
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    if coop:
        buf.fill_(0xFF)  # every half of the score buffer is written (NaN pattern otherwise)
    out = empty(torch, (batch * tokens, heads * 64), torch.float32)
    s = stream(torch)
    if coop:
        ok(lib, lib.dav2_hip_attention_ref_scores_coop(ptr(buf), ptr(qd), tokens, heads, batch, s))
    else:
        ok(lib, lib.dav2_hip_attention_ref_scores(ptr(buf), ptr(qd), tokens, heads, batch, int(fp16), s))

    def unpack():
        if fp16:
            w = host(torch, buf.view(torch.float16)).reshape(batch * heads, tokens, 2 * words)
            return w[:, :, :tokens].astype(np.float32), w[:, :, tokens:]
        return host(torch, buf.view(torch.float32)).reshape(batch * heads, tokens, tokens), None

    scores = probs = None
    if unpacked:
        scores, pad = unpack()
        if fp16 and tokens % 2:
            assert np.all(pad == 0)  # the high half of a row's last word is 0
    ok(lib, lib.dav2_hip_attention_ref_softmax(ptr(buf), batch * heads * tokens, tokens, int(fp16), s))
    if unpacked:
        probs, pad = unpack()
        if fp16 and tokens % 2:
            assert np.all(pad == 0)
    ok(lib, lib.dav2_hip_attention_ref_values(ptr(out), ptr(buf), ptr(qd), tokens, heads, batch, int(fp16), s))
    return host(torch, out), probs, scores


@pytest.mark.parametrize("tokens,heads,batch", [(1, 1, 1), (5, 2, 1), (65, 3, 1), (258, 2, 2), (1370, 6, 1),
                                                (1370, 16, 1)])
def test_attention_ref_fp32_bit_exact(gpu, lib, oracle, tokens, heads, batch):
    # bmm.glsl + softmax_lastdim.glsl order (mode 0 of the oracle), bit for bit
    torch = gpu
    _announce("attention ref fp32", tokens, heads, batch)
    rng = np.random.default_rng(tokens + heads)
    qkv = rng.standard_normal((batch * tokens, 3 * heads * 64)).astype(np.float32)
    out, p, _ = _attention_ref_gpu(torch, lib, qkv, tokens, heads, False, batch)
    for b in range(batch):
        rows = slice(b * tokens, (b + 1) * tokens)
        ref, p_ref = oracle.attention(qkv[rows], tokens, heads, fp16=False, probabilities=True)
        assert np.array_equal(p[b * heads:(b + 1) * heads].view(np.uint32), p_ref.view(np.uint32))
        assert np.array_equal(out[rows].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("tokens,heads,batch", [(1, 1, 1), (2, 1, 1), (5, 2, 1), (77, 4, 1), (258, 2, 2),
                                                (1369, 3, 1), (1370, 16, 1), (3101, 1, 1), (6200, 1, 1),
                                                (100, 2, 1), (1500, 1, 1), (3073, 1, 1), (3074, 2, 1),
                                                (5477, 1, 1)])
def test_attention_ref_fp16_bit_exact(gpu, lib, oracle, tokens, heads, batch):
    # bmm_score_fp16 + softmax_lastdim_half + bmm_value_fp16 (mode 1 of the
    # oracle: every product rounded to binary16), bit for bit: the binary16
    # scores, the probabilities and the output
    torch = gpu
    _announce("attention ref fp16", tokens, heads, batch)
    rng = np.random.default_rng(tokens * 3 + heads)
    qkv = (rng.standard_normal((batch * tokens, 3 * heads * 64)) * 1.5).astype(np.float32)
    out, p, scores = _attention_ref_gpu(torch, lib, qkv, tokens, heads, True, batch)
    for b in range(batch):
        rows = slice(b * tokens, (b + 1) * tokens)
        hs = slice(b * heads, (b + 1) * heads)
        s_ref = oracle.scores_binary16(qkv[rows], tokens, heads).astype(np.float32)
        assert np.array_equal(scores[hs].view(np.uint32), s_ref.view(np.uint32))
        ref, p_ref = oracle.attention(qkv[rows], tokens, heads, fp16=True, probabilities=True)
        assert np.array_equal(p[hs].view(np.uint32), p_ref.view(np.uint32))
        assert np.array_equal(out[rows].view(np.uint32), ref.view(np.uint32))


def _attention_ref16_fused_gpu(torch, lib, qkv, tokens, heads, batch=1, coop=False):
    qd = dev(torch, qkv)
    nbytes = lib.dav2_hip_attention_ref16_fused_scratch_bytes(tokens, heads, batch)
    assert nbytes == 2 * batch * heads * ((tokens + 63) // 64) * 8192
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out = empty(torch, (batch * tokens, heads * 64), torch.float32)
    out.fill_(float("nan"))
    run = lib.dav2_hip_attention_ref16_fused_coop if coop else lib.dav2_hip_attention_ref16_fused
    ok(lib, run(ptr(out), ptr(qd), tokens, heads, batch, ptr(buf), nbytes, stream(torch)))
    # one byte short of the binary16 keys and values is rejected before any launch
    assert run(ptr(out), ptr(qd), tokens, heads, batch, ptr(buf), nbytes - 1, stream(torch)) == 1
    return host(torch, out)


@pytest.mark.parametrize("tokens,heads,batch", [(1, 1, 1), (2, 1, 1), (5, 2, 1), (63, 1, 1), (64, 2, 1), (65, 3, 1),
                                                (77, 4, 2), (129, 2, 1), (1369, 3, 1), (1370, 16, 1), (1407, 2, 1),
                                                (1409, 2, 1), (2240, 2, 1)])
def test_attention_ref16_fused_bit_exact(gpu, lib, oracle, tokens, heads, batch):
    # The fused binary16 kernel (16 query rows per workgroup, T up to 2240)
    # against the oracle's mode 1 (bmm_score_fp16 + softmax_lastdim_half +
    # bmm_value_fp16), bit for bit
    torch = gpu
    _announce("attention ref16 fused", tokens, heads, batch)
    rng = np.random.default_rng(tokens * 5 + heads + batch)
    qkv = (rng.standard_normal((batch * tokens, 3 * heads * 64)) * 1.5).astype(np.float32)
    out = _attention_ref16_fused_gpu(torch, lib, qkv, tokens, heads, batch)
    for b in range(batch):
        rows = slice(b * tokens, (b + 1) * tokens)
        ref = oracle.attention(qkv[rows], tokens, heads, fp16=True)
        assert np.array_equal(out[rows].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("tokens,heads,batch,sigma", [(1370, 16, 2, 0.64), (1370, 16, 8, 3.0), (2240, 16, 1, 1.0)])
def test_attention_ref16_fused_matches_three_kernels(gpu, lib, tokens, heads, batch, sigma):
    # Batches of ViT-L rows and the fused kernel's longest rows against the
    # three materialised kernels, themselves bit-exact with the oracle's mode
    # 1 up to 6200 tokens: the same bits
    torch = gpu
    _announce("attention ref16 fused vs three kernels", tokens, heads, batch, sigma)
    rng = np.random.default_rng(tokens + heads + int(10 * sigma))
    qkv = (rng.standard_normal((batch * tokens, 3 * heads * 64)) * sigma).astype(np.float32)
    out = _attention_ref16_fused_gpu(torch, lib, qkv, tokens, heads, batch)
    ref, _, _ = _attention_ref_gpu(torch, lib, qkv, tokens, heads, True, batch, unpacked=False)
    assert np.isfinite(out).all()
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


def _f16_steps(a, b):
    """Distance in binary16 steps between two float16 arrays."""
    def key(x):
        u = x.view(np.uint16).astype(np.int32)
        return np.where(u & 0x8000, -(u & 0x7FFF), u)
    return np.abs(key(a) - key(b))


@pytest.mark.parametrize("tokens,heads,batch", [(1, 1, 1), (2, 1, 1), (5, 2, 1), (77, 4, 2), (258, 2, 1),
                                                (1370, 16, 1), (2241, 2, 1), (5477, 1, 1)])
def test_attention_coop_scores(gpu, lib, oracle, tokens, heads, batch):
    # bmm_score_coop_fp16.glsl on v_mfma_f32_16x16x32_f16 against the oracle's
    # mode-3 scores (exact products summed in double, rounded to fp32, then
    # binary16). The shader leaves the fp32 sum order to the matrix unit, and
    # any fp32 order of 64 terms is within 63 * 2^-24 * sum|q16 k16| of the
    # exact sum; so a score may differ from the oracle's by one binary16 step
    # plus that bound (near zero, where binary16 steps are finer than the
    # fp32 sums' rounding, that can be several steps), and differs at all only
    # rarely. The scores differ from the per-product shader's (mode 1) in
    # many places.
    torch = gpu
    _announce("attention coop scores", tokens, heads, batch)
    rng = np.random.default_rng(tokens * 13 + heads + batch)
    qkv = (rng.standard_normal((batch * tokens, 3 * heads * 64)) * 1.5).astype(np.float32)
    _, _, scores = _attention_ref_gpu(torch, lib, qkv, tokens, heads, True, batch, coop=True)
    d = heads * 64
    outside = moved = several = total = 0
    for b in range(batch):
        rows = slice(b * tokens, (b + 1) * tokens)
        got = scores[b * heads:(b + 1) * heads].astype(np.float16)
        ref = oracle.scores_coop(qkv[rows], tokens, heads)
        for h in range(heads):
            q16 = (qkv[rows, h * 64:h * 64 + 64] * np.float32(0.125)).astype(np.float16).astype(np.float64)
            k16 = qkv[rows, d + h * 64:d + h * 64 + 64].astype(np.float16).astype(np.float64)
            bound = 63 * 2.0 ** -24 * (np.abs(q16) @ np.abs(k16).T)
            step = np.spacing(np.abs(ref[h])).astype(np.float64)
            diff = np.abs(got[h].astype(np.float64) - ref[h].astype(np.float64))
            outside += int((diff > step + bound).sum())
        steps = _f16_steps(got, ref)
        moved += int((steps > 0).sum())
        several += int((steps > 1).sum())
        total += steps.size
        if tokens >= 64:
            assert (got != oracle.scores_binary16(qkv[rows], tokens, heads)).any()
    print(f"coop scores T={tokens}: {moved} of {total} differ from the oracle ({several} by more than one "
          f"binary16 step)", flush=True)
    assert outside == 0
    assert moved <= max(2, 1e-3 * total)


@pytest.mark.parametrize("tokens,heads,batch,sigma", [(1, 1, 1, 1.0), (65, 3, 1, 1.5), (77, 3, 2, 1.5),
                                                      (1370, 16, 2, 0.64), (1370, 16, 1, 3.0), (2240, 16, 1, 1.0)])
def test_attention_coop_fused_matches_three_kernels(gpu, lib, tokens, heads, batch, sigma):
    # the fused kernel issues the same two MFMAs per 16 x 16 score block as
    # the materialised score kernel, then the binary16 softmax and values of
    # the fused binary16 kernel: the same bits as scores + softmax + values
    torch = gpu
    _announce("attention coop fused vs three kernels", tokens, heads, batch, sigma)
    rng = np.random.default_rng(tokens + 7 * heads + int(10 * sigma))
    qkv = (rng.standard_normal((batch * tokens, 3 * heads * 64)) * sigma).astype(np.float32)
    out = _attention_ref16_fused_gpu(torch, lib, qkv, tokens, heads, batch, coop=True)
    ref, _, _ = _attention_ref_gpu(torch, lib, qkv, tokens, heads, True, batch, unpacked=False, coop=True)
    assert np.isfinite(out).all()
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("tokens,heads,sigma", [(77, 4, 1.5), (1370, 16, 0.64), (1370, 16, 2.0), (5477, 2, 0.64)])
def test_attention_coop_against_oracle(gpu, lib, oracle, tokens, heads, sigma):
    # The whole cooperative-matrix pipeline against the oracle's mode 3 and
    # against float64 attention. Only scores one binary16 step apart
    # (test_attention_coop_scores) separate it from mode 3, so the outputs
    # agree to a few binary16 steps of the values; both stay within the
    # per-product pipeline's distance of float64 attention.
    torch = gpu
    _announce("attention coop vs oracle", tokens, heads, sigma)
    rng = np.random.default_rng(tokens * 17 + heads + int(10 * sigma))
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * sigma).astype(np.float32)
    if lib.dav2_hip_attention_ref16_fused_scratch_bytes(tokens, heads, 1):
        out = _attention_ref16_fused_gpu(torch, lib, qkv, tokens, heads, coop=True)
    else:
        out, _, _ = _attention_ref_gpu(torch, lib, qkv, tokens, heads, True, unpacked=False, coop=True)
    ref = oracle.attention(qkv, tokens, heads, fp16=True, coop=True)
    per_product = oracle.attention(qkv, tokens, heads, fp16=True)
    f64 = _attention_f64_gpu(torch, qkv, tokens, heads)
    d = np.abs(out.astype(np.float64) - ref)
    scale = float(np.abs(qkv[:, 2 * heads * 64:]).max())
    e_coop, e_mode1 = np.abs(out - f64).max(), np.abs(per_product - f64).max()
    print(f"coop vs oracle T={tokens} sigma={sigma}: max {d.max():.3g}, mean {d.mean():.3g}, "
          f"equal {np.mean(out == ref):.4f}; max|coop - f64| {e_coop:.3g}, max|per-product - f64| {e_mode1:.3g}",
          flush=True)
    assert d.max() <= 4e-3 * scale
    assert d.mean() <= 1e-5 * scale
    assert e_coop <= 1.25 * e_mode1


def test_attention_ref16_fused_limits(gpu, lib):
    # beyond 2240 tokens the fused kernel reports no scratch size and refuses
    # to run; the three kernels serve those lengths
    assert lib.dav2_hip_attention_ref16_fused_scratch_bytes(2240, 1, 1) > 0
    assert lib.dav2_hip_attention_ref16_fused_scratch_bytes(2241, 1, 1) == 0
    assert lib.dav2_hip_attention_ref16_fused(None, None, 2241, 1, 1, None, 0, None) == 1


def test_attention_ref_hand_vectors(gpu, lib):
    # Scores that only the shader's arithmetic gives (see the oracle tests):
    # binary16 products cancel exactly; 1, 2^-24, -1 in feature order sum to
    # 0 while -1, 2^-24, 1 keep 2^-24.
    torch = gpu
    qkv = np.zeros((3, 192), np.float32)
    qkv[0, 0:2] = 8.0 * np.float32([1 + 2.0 ** -10, -1.0])
    qkv[1, 64:66] = [1 + 2.0 ** -10, 1 + 2.0 ** -9]
    qkv[2, 64:67] = [-1.0, 2.0 ** -12, 1.0]
    _, _, scores = _attention_ref_gpu(torch, lib, qkv, 3, 1, True)
    assert scores[0, 0, 1] == 0.0
    qkv[0, 0:3] = 8.0 * np.float32([1.0, 2.0 ** -12, -1.0])
    qkv[1, 64:67] = [1.0, 2.0 ** -12, 1.0]
    qkv[2, 64:67] = [1.0, 2.0 ** -12, 1.0]
    _, _, scores = _attention_ref_gpu(torch, lib, qkv, 3, 1, True)
    assert scores[0, 0, 1] == 0.0
    qkv[0, 0:3] = 8.0 * np.float32([-1.0, 2.0 ** -12, 1.0])
    _, _, scores = _attention_ref_gpu(torch, lib, qkv, 3, 1, True)
    assert scores[0, 0, 1] == np.float32(2.0 ** -24)


@pytest.mark.parametrize("tokens,heads", [(5, 2), (65, 3), (1370, 6), (1370, 16)])
def test_attention_mfma_fp32(gpu, lib, oracle, tokens, heads):
    # the matrix-core fp32 path of the fp32 precision mode: its own sum order,
    # within tolerance of the reference order
    torch = gpu
    _announce("attention mfma fp32", tokens, heads)
    rng = np.random.default_rng(tokens + heads)
    qkv = rng.standard_normal((tokens, 3 * heads * 64)).astype(np.float32)
    ref, p_ref = oracle.attention(qkv, tokens, heads, fp16=False, probabilities=True)
    out, p = _attention_mfma_gpu(torch, lib, qkv, tokens, heads)
    np.testing.assert_allclose(p, p_ref, rtol=2e-5, atol=2e-7)
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=2e-6)


def test_attention_reference_kat(gpu, lib):
    # tests/vulkan_smoke.cpp:540-628: 5 tokens x 2 heads, qkv[i] = (i%29-14)/128;
    # fp32 within 2e-6 of the closed form, fp16 within 3e-4 of fp32.
    torch = gpu
    tokens, heads = 5, 2
    d = heads * 64
    qkv = ((np.arange(tokens * 3 * d) % 29 - 14) * 0.0078125).astype(np.float32).reshape(tokens, 3 * d)
    q = qkv[:, :d].reshape(tokens, heads, 64).astype(np.float64)
    k = qkv[:, d:2 * d].reshape(tokens, heads, 64).astype(np.float64)
    v = qkv[:, 2 * d:].reshape(tokens, heads, 64).astype(np.float64)
    sc = np.einsum("ihf,jhf->hij", q * 0.125, k)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    expect = np.einsum("hij,jhf->ihf", p, v).reshape(tokens, d)
    out32, _, _ = _attention_ref_gpu(torch, lib, qkv, tokens, heads, False)
    assert np.abs(out32 - expect).max() <= 2e-6
    out16, _, _ = _attention_ref_gpu(torch, lib, qkv, tokens, heads, True)
    assert np.abs(out16 - out32).max() <= 3e-4
    outm, _ = _attention_mfma_gpu(torch, lib, qkv, tokens, heads)
    assert np.abs(outm - expect).max() <= 2e-6


def _attention_fused_gpu(torch, lib, qkv, tokens, heads, batch):
    qd = dev(torch, qkv)
    nbytes = lib.dav2_hip_attention_fused_scratch_bytes(tokens, heads, batch)
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out = empty(torch, (batch * tokens, heads * 64), torch.float32)
    ok(lib, lib.dav2_hip_attention_fused(ptr(out), ptr(qd), tokens, heads, batch, ptr(buf), nbytes, stream(torch)))
    # one byte short of the packed operands is rejected before any launch
    assert lib.dav2_hip_attention_fused(ptr(out), ptr(qd), tokens, heads, batch, ptr(buf), nbytes - 1,
                                        stream(torch)) == 1
    return host(torch, out)


@pytest.mark.parametrize("tokens,heads,batch", [(1, 1, 1), (5, 2, 1), (64, 3, 1), (77, 4, 2), (257, 6, 1),
                                                (1370, 16, 1), (1370, 6, 3), (1500, 3, 2), (1536, 2, 1),
                                                (1537, 2, 1), (2000, 2, 1)])
def test_attention_fused(gpu, lib, oracle, tokens, heads, batch):
    # Integer-exact kernel vs the oracle's restatement: every sum is an exact
    # integer and every rounding the same IEEE operation, so bit for bit; and
    # within 2e-4 of float64 attention.
    torch = gpu
    _announce("attention fused", tokens, heads, batch)
    rng = np.random.default_rng(tokens * 7 + heads + batch)
    qkv = (rng.standard_normal((batch * tokens, 3 * heads * 64)) * 0.5).astype(np.float32)
    out = _attention_fused_gpu(torch, lib, qkv, tokens, heads, batch)
    for b in range(batch):
        rows = slice(b * tokens, (b + 1) * tokens)
        ref = oracle.attention(qkv[rows], tokens, heads, fused=True)
        assert np.array_equal(out[rows].view(np.uint32), ref.view(np.uint32))
        q = qkv[rows, :heads * 64].reshape(tokens, heads, 64).astype(np.float64)
        k = qkv[rows, heads * 64:2 * heads * 64].reshape(tokens, heads, 64).astype(np.float64)
        v = qkv[rows, 2 * heads * 64:].reshape(tokens, heads, 64).astype(np.float64)
        sc = np.einsum("ihf,jhf->hij", q * 0.125, k)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        exact = np.einsum("hij,jhf->ihf", p, v).reshape(tokens, heads * 64)
        assert np.abs(out[rows] - exact).max() <= 2e-4


def _attention_colmax_gpu(torch, lib, qkv, tokens, heads, partial_rows):
    # column maxima of |k| | |v| over `partial_rows` row chunks, as the qkv
    # GEMM's ROW_COLMAX epilogue leaves them
    D = heads * 64
    bounds = np.linspace(0, tokens, partial_rows + 1).astype(int)
    cm = np.zeros((partial_rows, 2 * D), np.float32)
    for p in range(partial_rows):
        if bounds[p + 1] > bounds[p]:
            cm[p] = np.abs(qkv[bounds[p]:bounds[p + 1], D:]).max(axis=0)
    qd, cmd = dev(torch, qkv), dev(torch, cm)
    nbytes = lib.dav2_hip_attention_fused_scratch_bytes(tokens, heads, 1)
    buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    out = empty(torch, (tokens, D), torch.float32)
    ok(lib, lib.dav2_hip_attention_fused_colmax(ptr(out), ptr(qd), tokens, heads, ptr(cmd), partial_rows, ptr(buf),
                                                nbytes, stream(torch)))
    assert lib.dav2_hip_attention_fused_colmax(ptr(out), ptr(qd), tokens, heads, None, partial_rows, ptr(buf),
                                               nbytes, stream(torch)) != 0
    assert lib.dav2_hip_attention_fused_colmax(ptr(out), ptr(qd), tokens, heads, ptr(cmd), 0, ptr(buf),
                                               nbytes, stream(torch)) != 0
    return host(torch, out)


@pytest.mark.parametrize("tokens,heads,partial_rows", [(1, 1, 1), (5, 2, 3), (64, 3, 1), (77, 4, 2), (1370, 16, 15),
                                                       (1370, 6, 22), (2000, 2, 7)])
def test_attention_fused_colmax(gpu, lib, oracle, tokens, heads, partial_rows):
    # One-pass digit packing from column maxima: the same bits as the
    # two-pass packing and the oracle.
    torch = gpu
    _announce("attention fused colmax", tokens, heads, partial_rows)
    rng = np.random.default_rng(tokens * 5 + heads)
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * 0.5).astype(np.float32)
    got = _attention_colmax_gpu(torch, lib, qkv, tokens, heads, partial_rows)
    two_pass = _attention_fused_gpu(torch, lib, qkv, tokens, heads, 1)
    assert np.array_equal(got.view(np.uint32), two_pass.view(np.uint32))
    ref = oracle.attention(qkv, tokens, heads, fused=True)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("colmax", [False, True])
def test_attention_fused_peaked_and_zero_rows(gpu, lib, oracle, colmax):
    # Peaked rows (|s| up to ~60, most numerators underflow to 0), an all-zero
    # query row, an all-zero key row and an all-zero value column.
    torch = gpu
    tokens, heads = 300, 2
    rng = np.random.default_rng(11)
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * 2.0).astype(np.float32)
    qkv[7, :64] = 0.0
    qkv[9, heads * 64:heads * 64 + 64] = 0.0
    qkv[:, 2 * heads * 64 + 5] = 0.0
    out = (_attention_colmax_gpu(torch, lib, qkv, tokens, heads, 4) if colmax
           else _attention_fused_gpu(torch, lib, qkv, tokens, heads, 1))
    ref = oracle.attention(qkv, tokens, heads, fused=True)
    assert np.isfinite(out).all()
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    assert np.all(out[:, 5] == 0.0)


def _attention_f64_gpu(torch, qkv, tokens, heads):
    # float64 attention on the device (head by head), the exact reference
    q = torch.from_numpy(qkv).to("cuda", torch.float64)
    d = heads * 64
    out = torch.empty((tokens, d), dtype=torch.float64, device="cuda")
    for h in range(heads):
        qh = q[:, h * 64:(h + 1) * 64] * 0.125
        kh = q[:, d + h * 64:d + (h + 1) * 64].contiguous()
        vh = q[:, 2 * d + h * 64:2 * d + (h + 1) * 64].contiguous()
        p = torch.softmax(qh @ kh.T.contiguous(), dim=-1)
        out[:, h * 64:(h + 1) * 64] = p @ vh
    return host(torch, out)


@pytest.mark.parametrize("tokens,heads,sigma", [(1370, 16, 0.64), (1370, 16, 2.0), (5477, 16, 0.64)])
def test_attention_fused_against_reference_arithmetic(gpu, lib, tokens, heads, sigma):
    # The int8 mode's default attention (integer-exact, this build's own
    # arithmetic) against the reference's int8-mode arithmetic
    # (bmm_score_fp16.glsl / softmax_lastdim_half.glsl / bmm_value_fp16.glsl:
    # the binary16 kernels, bit-exact with the oracle's mode 1 in
    # test_attention_ref_fp16_bit_exact) and float64 attention, on the same
    # qkv at ViT-L width (16 heads) for 518x518 (T = 1370) and 1036x1036
    # (T = 5477). sigma 0.64 is the spread of a random-init ViT-L's qkv; 2.0
    # gives peaked rows. Asserted:
    #   max|fused - f64| <= max|binary16 - f64| (the default is no less
    #     accurate than the reference's arithmetic), and so is the per-row
    #     maximum on at least 98% of the (token, head) rows;
    #   max|fused - binary16| <= 1.25 max|binary16 - f64|: the default departs
    #     from the reference's arithmetic by no more than that arithmetic
    #     departs from exact attention.
    torch = gpu
    _announce("attention fused vs binary16 vs f64", tokens, heads, sigma)
    rng = np.random.default_rng(tokens + int(sigma * 100))
    qkv = (rng.standard_normal((tokens, 3 * heads * 64)) * sigma).astype(np.float32)
    fused = _attention_fused_gpu(torch, lib, qkv, tokens, heads, 1).astype(np.float64)
    ref16, _, _ = _attention_ref_gpu(torch, lib, qkv, tokens, heads, True, unpacked=False)
    ref16 = ref16.astype(np.float64)
    exact = _attention_f64_gpu(torch, qkv, tokens, heads)
    e_fused, e_ref = np.abs(fused - exact), np.abs(ref16 - exact)
    rows_fused = e_fused.reshape(tokens, heads, 64).max(-1)
    rows_ref = e_ref.reshape(tokens, heads, 64).max(-1)
    gap = np.abs(fused - ref16).max()
    share = float((rows_fused <= rows_ref).mean())
    print(f"attention T={tokens} H={heads} sigma={sigma}: max|fused-f64| {e_fused.max():.3g}, "
          f"max|binary16-f64| {e_ref.max():.3g}, max|fused-binary16| {gap:.3g}, "
          f"rows with fused <= binary16 error {share:.4f}", flush=True)
    assert e_fused.max() <= e_ref.max()
    assert share >= 0.98
    assert gap <= 1.25 * e_ref.max()


def test_softmax_fp32_buffer_off_8_bytes(gpu, lib, oracle):
    # rows of an even number of items on a buffer 4 bytes past an 8-byte
    # boundary: the single-item path, the same bits
    torch = gpu
    rows, cols = 6, 1024
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((rows, cols)) * 4).astype(np.float32)
    ref = oracle.softmax_rows(x)
    buf = torch.zeros(rows * cols + 2, dtype=torch.float32, device="cuda")
    buf[1:1 + rows * cols] = torch.from_numpy(x.reshape(-1)).cuda()
    ok(lib, lib.dav2_hip_attention_ref_softmax(ptr(buf) + 4, rows, cols, 0, stream(torch)))
    got = host(torch, buf)[1:1 + rows * cols].reshape(rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(16 * 1370, 1370), (7, 5477), (3, 64), (5, 9000), (4, 6144), (2, 1),
                                       (3, 2500), (1, 1537), (5, 2), (3, 130), (6, 1024), (9, 1536), (4, 1000),
                                       (3, 1025), (2, 3072), (2, 3073), (2, 5632), (2, 5633), (2, 11264),
                                       (2, 11265), (64 * 5477, 5477), (5, 961), (3, 960), (4, 700)])
def test_softmax_fp32(gpu, lib, oracle, rows, cols):
    # softmax_lastdim.glsl in its lane/tree order: bit for bit (register and
    # streaming forms); the matrix-core path's row softmax within tolerance
    torch = gpu
    _announce("softmax", rows, cols)
    rng = np.random.default_rng(rows)
    x = (rng.standard_normal((rows, cols)) * 4).astype(np.float32)
    ref = oracle.softmax_rows(x)
    xd = dev(torch, x)
    ok(lib, lib.dav2_hip_attention_ref_softmax(ptr(xd), rows, cols, 0, stream(torch)))
    assert np.array_equal(host(torch, xd).view(np.uint32), ref.view(np.uint32))
    xd = dev(torch, x)
    ok(lib, lib.dav2_hip_softmax_rows(ptr(xd), rows, cols, cols, 0, stream(torch)))
    np.testing.assert_allclose(host(torch, xd), ref, rtol=5e-6, atol=1e-9)


# ---------------------------------------------------------------------------
# elementwise, resize, min/max, position
def test_elementwise_exact(gpu, lib, oracle):
    torch = gpu
    rng = np.random.default_rng(1)
    n = 1370 * 1024 + 3
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    ad, bd = dev(torch, a), dev(torch, b)
    out = empty(torch, (n,), torch.float32)
    s = stream(torch)
    ok(lib, lib.dav2_hip_add(ptr(out), ptr(ad), ptr(bd), n, s))
    assert np.array_equal(host(torch, out), oracle.add(a, b))
    ok(lib, lib.dav2_hip_relu(ptr(out), ptr(ad), n, s))
    assert np.array_equal(host(torch, out), oracle.relu(a))
    cols = 1024
    m = (n // cols) * cols
    gamma = rng.uniform(-1e-3, 1e-3, cols).astype(np.float32)
    gd = dev(torch, gamma)
    ok(lib, lib.dav2_hip_add_scaled(ptr(out), ptr(ad), ptr(bd), ptr(gd), m, cols, s))
    assert np.array_equal(host(torch, out)[:m], oracle.add_scaled(a[:m], b[:m], gamma))
    ok(lib, lib.dav2_hip_gelu(ptr(out), ptr(ad), n, s))
    assert np.array_equal(host(torch, out).view(np.uint32), oracle.gelu(a).view(np.uint32))
    # wide sweep through every branch of the exp and erfc evaluation
    w = np.concatenate([np.linspace(-40, 40, 200001, dtype=np.float32),
                        (rng.standard_normal(100000) * 10).astype(np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 13.5, -13.5, 1e4, -1e4, np.inf, 3e38, -3e38, 42.42, -42.42,
                                  42.43, -42.43, 42.44, -42.44, 100.0, -100.0], np.float32),
                        # around 1 + |x|/(2 sqrt 2) = 16, where the reciprocal switches form
                        (42.426407 + np.arange(-64, 64) * 1e-5).astype(np.float32)]).astype(np.float32)
    wd, wo = dev(torch, w), empty(torch, w.shape, torch.float32)
    ok(lib, lib.dav2_hip_gelu(ptr(wo), ptr(wd), w.size, s))
    assert np.array_equal(host(torch, wo).view(np.uint32), oracle.gelu(w).view(np.uint32))
    # -inf: both give NaN (-inf * 0); NaN bit patterns are not compared
    ninf = dev(torch, np.array([-np.inf, np.nan], np.float32))
    no = empty(torch, (2,), torch.float32)
    ok(lib, lib.dav2_hip_gelu(ptr(no), ptr(ninf), 2, s))
    assert np.isnan(host(torch, no)).all() and np.isnan(oracle.gelu(np.array([-np.inf, np.nan], np.float32))).all()


def test_gelu_every_float_below_42(gpu, lib, oracle):
    # Every float x with |x| < 42.5 (2.2e9 values): the range in which the
    # GELU's 1 / (1 + |x|/(2 sqrt 2)) takes the refined hardware reciprocal;
    # bit-exact against the oracle's IEEE division.
    torch = gpu
    s = stream(torch)
    limit, chunk = 0x422A0000, 1 << 26
    for sign in (0, -(2**31)):
        for start in range(0, limit, chunk):
            n = min(chunk, limit - start)
            bits = torch.arange(start, start + n, dtype=torch.int32, device="cuda")
            if sign:
                bits = bits | sign
            x = bits.view(torch.float32)
            out = torch.empty_like(x)
            ok(lib, lib.dav2_hip_gelu(ptr(out), ptr(x), n, s))
            xh = (np.arange(start, start + n, dtype=np.uint32) | np.uint32(sign & 0xFFFFFFFF)).view(np.float32)
            got = host(torch, out)
            if not np.array_equal(got.view(np.uint32), oracle.gelu(xh).view(np.uint32)):
                bad = np.nonzero(got.view(np.uint32) != oracle.gelu(xh).view(np.uint32))[0][:4]
                pytest.fail(f"GELU differs at x = {xh[bad]}")


@pytest.mark.parametrize("c,ih,iw,oh,ow", [(256, 19, 19, 37, 37), (256, 148, 148, 296, 296), (128, 296, 296, 518, 518),
                                           (3, 5, 7, 1, 1), (2, 1, 1, 4, 3), (64, 25, 19, 50, 38), (13, 9, 11, 20, 21)])
def test_bilinear_bit_exact(gpu, lib, oracle, c, ih, iw, oh, ow):
    torch = gpu
    _announce("bilinear", c, ih, iw, oh, ow)
    rng = np.random.default_rng(c + oh)
    x = rng.standard_normal((c, ih, iw)).astype(np.float32)
    ref = oracle.bilinear(x, ow, oh)
    xd = dev(torch, x)
    out = empty(torch, (c, oh, ow), torch.float32)
    ok(lib, lib.dav2_hip_bilinear_align_true(ptr(out), ptr(xd), iw, ih, ow, oh, c, stream(torch)))
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("n", [4, 1000, 518 * 518, 1036 * 1036 + 5])
def test_minmax_normalize(gpu, lib, oracle, n):
    torch = gpu
    rng = np.random.default_rng(n)
    d = (rng.standard_normal(n) * 3 + 7).astype(np.float32)
    if n == 4:
        d = np.array([2.0, 3.0, 5.0, 10.0], np.float32)  # tests/vulkan_smoke.cpp:121-142
    dd = dev(torch, d)
    rng_d = empty(torch, (2,), torch.float32)
    part = empty(torch, (2 * lib.dav2_hip_minmax_partials(n),), torch.float32)
    s = stream(torch)
    ok(lib, lib.dav2_hip_reduce_minmax(ptr(dd), n, ptr(rng_d), ptr(part), s))
    r = host(torch, rng_d)
    assert np.array_equal(r, oracle.reduce_minmax(d))
    ok(lib, lib.dav2_hip_normalize_relative(ptr(dd), ptr(rng_d), n, s))
    got = host(torch, dd)
    assert np.array_equal(got.view(np.uint32), oracle.normalize_relative(d, r).view(np.uint32))
    if n == 4:
        np.testing.assert_allclose(got, [0.0, 0.125, 0.375, 1.0], atol=1e-6)


@pytest.mark.parametrize("pw,ph,dim", [(37, 37, 384), (74, 74, 64), (25, 19, 96), (3, 2, 3)])
def test_position_bicubic_and_tokens(gpu, lib, oracle, pw, ph, dim):
    torch = gpu
    rng = np.random.default_rng(pw * ph)
    pos = (rng.standard_normal((1370, dim)) * 0.02).astype(np.float32)
    ref = oracle.position_bicubic(pos, pw, ph, dim)
    pd = dev(torch, pos)
    out = empty(torch, (dim, ph, pw), torch.float32)
    s = stream(torch)
    ok(lib, lib.dav2_hip_position_bicubic(ptr(out), ptr(pd), pw, ph, dim, s))
    interp = host(torch, out)
    assert np.array_equal(interp.view(np.uint32), ref.view(np.uint32))
    if pw == 37 and ph == 37:
        assert np.array_equal(interp, pos[1:].T.reshape(dim, 37, 37))  # exact copy (operators.cpp:1351-1357)
    # class token + position add for a batch of two token matrices
    t = pw * ph + 1
    tokens = rng.standard_normal((2, t, dim)).astype(np.float32)
    cls = rng.standard_normal(dim).astype(np.float32)
    td, cd = dev(torch, tokens), dev(torch, cls)
    ok(lib, lib.dav2_hip_finish_tokens(ptr(td), ptr(out), ptr(pd), ptr(cd), pw, ph, dim, 2, s))
    got = host(torch, td)
    exp = tokens.copy()
    exp[:, 0] = cls + pos[0]
    exp[:, 1:] = tokens[:, 1:] + interp.reshape(dim, -1).T[None]
    assert np.array_equal(got, exp)

"""The fp32 precision mode (DAV2_CREATE_FORCE_FP32): the fp32 MFMA GEMM and
im2col kernels against float64 products and torch's unfold, the fp32
operators (src/operators.cpp:882-955, :1211-1452, :1528-1676, :1807-1861)
against the oracle, and whole models against the oracle's fp32 graph.

fp32 sums in a different order than the oracle's: the gate is the depth
tolerance, max|gpu - cpu| <= 1e-3 of the depth range; the operators are held
to 1e-5 of their output's magnitude."""

import ctypes as C

import numpy as np
import pytest
import torch.nn.functional as F

from gpu_util import db, dev, empty, host, ok, ptr, stream

pytestmark = pytest.mark.gpu

SEED = 0xDA20000
ENC = {"vits": 0, "vitb": 1, "vitl": 2}
EPI = {"row": 1, "gelu": 2, "layerscale": 3, "transposed": 4, "convt": 5}


def _announce(*args):
    print("case:", *args, flush=True)


def _rel(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.fixture(scope="module")
def ops(gpu, lib):
    h = lib.dav2_ops_create(0)
    assert h, lib.dav2_ops_last_error()
    yield h
    lib.dav2_ops_destroy(h)


def _resident(torch, *arrays):
    """Device copies, complete before the operator set's own stream reads them
    (the copies run on torch's stream) and held until the caller drops them."""
    out = [dev(torch, a) for a in arrays]
    torch.cuda.synchronize()
    return out


def run(lib, rc):
    assert rc == 0, f"status {rc}: {lib.dav2_ops_last_error().decode()}"


@pytest.mark.parametrize("m,n,k", [(37, 80, 96), (1370, 1024, 1024), (200, 33, 588), (1, 5, 4)])
@pytest.mark.parametrize("epi", ["row", "gelu", "layerscale", "transposed"])
def test_gemm_f32_epilogues(gpu, pkg, lib, oracle, m, n, k, epi):
    torch = gpu
    _announce("gemm_f32", m, n, k, epi)
    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    gamma = rng.standard_normal(n).astype(np.float32)
    v = a.astype(np.float64) @ b.astype(np.float64).T + bias
    ad, bd, biasd, gd = dev(torch, a), dev(torch, b), dev(torch, bias), dev(torch, gamma)
    args = pkg.GemmF32Args()
    args.a, args.lda, args.b, args.ldb = ptr(ad), k, ptr(bd), k
    args.m, args.n, args.k, args.epilogue, args.bias = m, n, k, EPI[epi], ptr(biasd)
    if epi == "transposed":
        res = rng.standard_normal((n, m + 3)).astype(np.float32)
        out = dev(torch, res.copy())
        args.out, args.out_row_stride, args.out_row_offset = ptr(out), m + 3, 2
        resd = dev(torch, res)
        args.residual, args.relu_output = ptr(resd), 1
        want = res.astype(np.float64).copy()
        want[:, 2:2 + m] = np.maximum(v.T + res[:, 2:2 + m], 0.0)
    else:
        res = rng.standard_normal((m + 1, n)).astype(np.float32)
        out = dev(torch, res)
        args.out, args.out_row_offset = ptr(out), 1
        want = res.astype(np.float64).copy()
        if epi == "row":
            want[1:] = v
        elif epi == "gelu":
            want[1:] = oracle.gelu(v.astype(np.float32))
        else:
            args.residual, args.gamma = ptr(out), ptr(gd)
            want[1:] = res[1:] + v * gamma
    ok(lib, lib.dav2_hip_gemm_f32(C.byref(args), stream(torch)))
    got = host(torch, out)
    assert _rel(got, want) < 1e-5


def test_gemm_f32_rejects(gpu, pkg, lib):
    torch = gpu
    a = empty(torch, (8, 8), torch.float32)
    args = pkg.GemmF32Args()
    args.a, args.lda, args.b, args.ldb, args.m, args.n, args.k = ptr(a), 8, ptr(a), 8, 8, 8, 6  # k % 4
    args.epilogue, args.out = 1, ptr(a)
    assert lib.dav2_hip_gemm_f32(C.byref(args), stream(torch)) != 0
    args.k, args.epilogue = 8, 6  # ROW_COLMAX is int8 only
    assert lib.dav2_hip_gemm_f32(C.byref(args), stream(torch)) != 0


@pytest.mark.parametrize("c,h,w,k,s,p,relu", [(8, 11, 9, 3, 1, 1, False), (16, 13, 10, 3, 2, 1, True),
                                              (3, 28, 42, 14, 14, 0, False), (4, 5, 7, 1, 1, 0, True)])
def test_im2col_f32_matches_unfold(gpu, lib, c, h, w, k, s, p, relu):
    torch = gpu
    _announce("im2col_f32", c, h, w, k, s, p, relu)
    x = np.random.default_rng(c + h).standard_normal((c, h, w)).astype(np.float32)
    ow, oh = (w + 2 * p - k) // s + 1, (h + 2 * p - k) // s + 1
    ld = (c * k * k + 3) // 4 * 4 + 4
    xd = dev(torch, x)
    out = empty(torch, (ow * oh, ld), torch.float32)
    ok(lib, lib.dav2_hip_im2col_f32(ptr(xd), w, h, c, ow, oh, k, s, p, int(relu), ptr(out), ld, stream(torch)))
    src = torch.from_numpy(np.maximum(x, 0) if relu else x)[None]
    want = F.unfold(src, k, padding=p, stride=s)[0].T.numpy()
    got = host(torch, out)
    assert np.array_equal(got[:, : c * k * k], want)
    assert not got[:, c * k * k:].any()


def test_ops_linear(gpu, pkg, lib, oracle, ops):
    torch = gpu
    rng = np.random.default_rng(3)
    rows, ic, oc = 333, 384, 1536
    x = rng.standard_normal((rows, ic)).astype(np.float32)
    w = (rng.standard_normal((oc, ic)) * 0.05).astype(np.float32)
    b = rng.standard_normal(oc).astype(np.float32)
    xd, wd, bd = _resident(torch, x, w, b)
    for gelu in (False, True):
        out = empty(torch, (rows, oc), torch.float32)
        run(lib, lib.dav2_ops_linear(ops, db(pkg, out), db(pkg, xd), db(pkg, wd), db(pkg, bd), rows, ic, oc,
                                     int(gelu)))
        run(lib, lib.dav2_ops_synchronize(ops))
        assert _rel(host(torch, out), oracle.linear_f32(x, w, b, gelu=gelu)) < 1e-5
    bad = empty(torch, (rows, oc - 1), torch.float32)
    assert lib.dav2_ops_linear(ops, db(pkg, bad), db(pkg, xd), db(pkg, wd), db(pkg, bd), rows, ic, oc, 0) == 1


@pytest.mark.parametrize("c,oc,h,w,k,s,p", [(64, 64, 37, 37, 3, 1, 1), (32, 16, 20, 24, 3, 2, 1),
                                            (64, 32, 9, 11, 1, 1, 0)])
def test_ops_conv2d(gpu, pkg, lib, oracle, ops, c, oc, h, w, k, s, p):
    torch = gpu
    _announce("conv2d fp32", c, oc, h, w, k, s, p)
    rng = np.random.default_rng(c + oc + h)
    x = rng.standard_normal((c, h, w)).astype(np.float32)
    wt = (rng.standard_normal((oc, c, k, k)) * 0.05).astype(np.float32)
    b = rng.standard_normal(oc).astype(np.float32)
    ow, oh = (w + 2 * p - k) // s + 1, (h + 2 * p - k) // s + 1
    out = empty(torch, (oc, oh, ow), torch.float32)
    xd, wd, bd = _resident(torch, x, wt, b)
    run(lib, lib.dav2_ops_conv2d(ops, db(pkg, out), db(pkg, xd), db(pkg, wd), db(pkg, bd), w, h, c, oc, k, s, p, 1))
    run(lib, lib.dav2_ops_synchronize(ops))
    assert _rel(host(torch, out), oracle.conv2d_f32(x, wt, b, s, p)) < 1e-5


@pytest.mark.parametrize("k", [2, 4])
def test_ops_conv_transpose(gpu, pkg, lib, oracle, ops, k):
    torch = gpu
    rng = np.random.default_rng(k)
    ic, oc, h, w = 32, 24, 7, 9
    x = rng.standard_normal((ic, h, w)).astype(np.float32)
    wt = (rng.standard_normal((ic, oc, k, k)) * 0.1).astype(np.float32)
    b = rng.standard_normal(oc).astype(np.float32)
    rows = wt.transpose(2, 3, 1, 0).reshape(k * k * oc, ic)  # row (ky k + kx) OC + oc, column ic
    out = empty(torch, (oc, h * k, w * k), torch.float32)
    xd, rd, bd = _resident(torch, x, np.ascontiguousarray(rows), b)
    run(lib, lib.dav2_ops_conv_transpose_nonoverlap(ops, db(pkg, out), db(pkg, xd), db(pkg, rd), db(pkg, bd), w, h,
                                                    ic, oc, k))
    run(lib, lib.dav2_ops_synchronize(ops))
    assert _rel(host(torch, out), oracle.conv_transpose_f32(x, wt, b)) < 1e-5


def test_ops_project_tokens(gpu, pkg, lib, oracle, ops):
    torch = gpu
    rng = np.random.default_rng(8)
    pw, ph, d, c = 19, 11, 64, 48
    tokens = rng.standard_normal((pw * ph + 1, d)).astype(np.float32)
    w = rng.standard_normal((c, d)).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32)
    out = empty(torch, (c, ph, pw), torch.float32)
    td, wd, bd = _resident(torch, tokens, w, b)
    run(lib, lib.dav2_ops_project_tokens(ops, db(pkg, out), db(pkg, td), db(pkg, wd), db(pkg, bd), pw, ph, d, c))
    run(lib, lib.dav2_ops_synchronize(ops))
    assert _rel(host(torch, out), oracle.project_tokens_f32(tokens, w, b, pw, ph)) < 1e-5


def test_ops_prepare_tokens_f32(gpu, pkg, lib, oracle, ops):
    torch = gpu
    rng = np.random.default_rng(9)
    pw, ph, d = 9, 6, 32
    width, height = 14 * pw, 14 * ph
    image = rng.standard_normal((3, height, width)).astype(np.float32)
    w = (rng.standard_normal((d, 3, 14, 14)) * 0.05).astype(np.float32)
    b = rng.standard_normal(d).astype(np.float32)
    cls = rng.standard_normal(d).astype(np.float32)
    pos = rng.standard_normal((1370, d)).astype(np.float32)
    toks = empty(torch, (pw * ph + 1, d), torch.float32)
    imd, wd, bd, cd, pd = _resident(torch, image, w, b, cls, pos)
    run(lib, lib.dav2_ops_prepare_tokens_f32(ops, db(pkg, toks), db(pkg, imd), db(pkg, wd), db(pkg, bd), db(pkg, cd),
                                             db(pkg, pd), width, height, d))
    run(lib, lib.dav2_ops_synchronize(ops))
    want = oracle.prepare_tokens_f32(image, w, b, cls, pos, width, height)
    assert _rel(host(torch, toks), want) < 1e-5


@pytest.fixture(scope="module")
def models(pkg, tmp_path_factory):
    root = tmp_path_factory.mktemp("fp32_models")
    paths = {}
    for enc in ("vits", "vitb"):
        p = root / f"{enc}.dav2"
        pkg.dav2_format.write_synthetic_model(p, enc, seed=SEED + ENC[enc] + 1)
        paths[enc] = p
    return paths


def _span_err(got, ref):
    span = float(ref.max() - ref.min())
    return float(np.abs(got - ref).max()) / (span if span > 0 else 1.0)


@pytest.mark.parametrize("enc,width,height", [("vits", 266, 266), ("vits", 350, 266), ("vitb", 196, 252)])
def test_fp32_mode_depth_parity(gpu, pkg, lib, oracle, models, enc, width, height):
    torch = gpu
    _announce("fp32 model", enc, width, height)
    x = pkg.dav2_format.imagenet_input(width, height, seed=SEED + width + 1)[0]
    with pkg.Context(str(models[enc]), enc, pkg.FORCE_FP32) as ctx:
        depth = ctx.infer(x, width, height)
        xd = dev(torch, x)
        d2 = empty(torch, (height, width), torch.float32)
        logits = empty(torch, (height, width), torch.float32)
        assert lib.dav2_infer_tensor_f32_device_logits(ctx.handle, xd.data_ptr(), width, height, d2.data_ptr(),
                                                       logits.data_ptr(), stream(torch)) == 0
        d2, logits = host(torch, d2), host(torch, logits)
    h = oracle.load_model(models[enc], ENC[enc])
    try:
        ref_depth, ref_logits = oracle.infer_fp32(h, x, width, height)
    finally:
        oracle.free_model(h)
    assert np.isfinite(depth).all() and np.array_equal(depth, d2)
    e_depth, e_logits = _span_err(depth, ref_depth), _span_err(logits, ref_logits)
    print(f"fp32 parity {enc} {width}x{height}: depth {e_depth:.3g}, logits {e_logits:.3g}", flush=True)
    assert e_depth <= 1e-3 and e_logits <= 1e-3

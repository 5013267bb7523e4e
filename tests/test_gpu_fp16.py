"""The fp16 precision mode (DAV2_CREATE_FORCE_FP16): the native binary16
product GEMM bit for bit against the oracle (prepare_tokens_fp16.glsl,
project_tokens_fp16.glsl, conv_transpose_nonoverlap_fp16.glsl sum in k order),
the half-operand fp32 GEMM (the cooperative-matrix linears) against float64
products of the rounded operands, the binary16 weight rounding against numpy,
and whole models against the oracle's fp16 graph.

The cooperative-matrix linears and the DPT convolutions sum in the GEMM's own
order: the model gate is the north-star tolerance, max|gpu - cpu| <= 1e-3 of
the depth range (and of the pre-ReLU logits' range)."""

import ctypes as C

import numpy as np
import pytest

from gpu_util import dev, empty, host, ptr, stream

pytestmark = pytest.mark.gpu

SEED = 0xDA21600
ENC = {"vits": 0, "vitb": 1, "vitl": 2}
EPI = {"row": 1, "transposed": 4, "convt": 5}


def _announce(*args):
    print("case:", *args, flush=True)


def _gemm_args(pkg, **kw):
    a = pkg.GemmF32Args()
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("m,n,k,epi", [(37, 80, 96, "row"), (1369, 64, 588, "row"), (200, 33, 64, "transposed"),
                                       (1, 5, 4, "row"), (64, 64, 32, "transposed"), (49, 48, 12, "convt")])
def test_gemm_h16_products_bit_exact(gpu, pkg, lib, oracle, m, n, k, epi):
    torch = gpu
    _announce("gemm_h16_products", m, n, k, epi)
    rng = np.random.default_rng(m * 7 + n + k)
    a = (rng.standard_normal((m, k)) * 2).astype(np.float32)
    b = (rng.standard_normal((n, k)) * 0.1).astype(np.float32)
    bias_n = n // 4 if epi == "convt" else n
    bias = rng.standard_normal(bias_n).astype(np.float32)
    acc = oracle.gemm_h16_products(a, b)  # [m][n], k-order fp32 sums of binary16 products
    ad, bd, biasd = dev(torch, a), dev(torch, b), dev(torch, bias)
    args = _gemm_args(pkg, a=ptr(ad), lda=k, b=ptr(bd), ldb=k, m=m, n=n, k=k, epilogue=EPI[epi], bias=ptr(biasd))
    if epi == "row":
        out = torch.full((m + 1, n), float("nan"), dtype=torch.float32, device="cuda")
        args.out, args.out_row_offset = ptr(out), 1
        want = (acc + bias).astype(np.float32)
    elif epi == "transposed":
        out = torch.full((n, m), float("nan"), dtype=torch.float32, device="cuda")
        args.out, args.out_row_stride = ptr(out), m
        want = (acc + bias).astype(np.float32).T
    else:
        # 2x2 kernel, 7x7 input pixels, 12 output channels: column n = (ky*2 + kx)*12 + oc
        kk, w, h, c = 2, 7, 7, n // 4
        out = torch.full((c, h * kk, w * kk), float("nan"), dtype=torch.float32, device="cuda")
        args.out, args.convt_kernel, args.convt_width, args.convt_height, args.convt_channels = ptr(out), kk, w, h, c
        want = np.empty((c, h * kk, w * kk), np.float32)
        for col in range(n):
            kidx, oc = divmod(col, c)
            ky, kx = divmod(kidx, kk)
            want[oc, ky::kk, kx::kk] = (acc[:, col] + bias[oc]).astype(np.float32).reshape(h, w)
    assert lib.dav2_hip_gemm_h16_products(C.byref(args), stream(torch)) == 0
    got = host(torch, out)[1:] if epi == "row" else host(torch, out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), \
        f"{np.count_nonzero(got.view(np.uint32) != want.view(np.uint32))} of {got.size} differ"


def test_gemm_h16_products_rejects(gpu, pkg, lib):
    torch = gpu
    a = torch.zeros((4, 8), dtype=torch.float32, device="cuda")
    out = torch.zeros((4, 4), dtype=torch.float32, device="cuda")
    base = dict(a=ptr(a), lda=8, b=ptr(a), ldb=8, m=4, n=4, k=8, out=ptr(out))
    # GELU / LayerScale epilogues are not native binary16 shaders
    assert lib.dav2_hip_gemm_h16_products(C.byref(_gemm_args(pkg, epilogue=2, **base)), stream(torch)) != 0
    # k not a multiple of 4
    bad = dict(base, k=6)
    assert lib.dav2_hip_gemm_h16_products(C.byref(_gemm_args(pkg, epilogue=1, **bad)), stream(torch)) != 0


@pytest.mark.parametrize("m,n,k", [(1370, 384, 384), (77, 96, 1536), (5, 3, 4)])
def test_gemm_f32_half_operands(gpu, pkg, lib, m, n, k):
    torch = gpu
    _announce("gemm_f32 half operands", m, n, k)
    rng = np.random.default_rng(m + 3 * n + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    exact = (a.astype(np.float16).astype(np.float64) @ b.astype(np.float16).astype(np.float64).T) + bias
    ad, bd, biasd = dev(torch, a), dev(torch, b), dev(torch, bias)
    out = torch.empty((m, n), dtype=torch.float32, device="cuda")
    args = _gemm_args(pkg, a=ptr(ad), lda=k, b=ptr(bd), ldb=k, m=m, n=n, k=k, epilogue=1, bias=ptr(biasd),
                      out=ptr(out), half_operands=1)
    assert lib.dav2_hip_gemm_f32(C.byref(args), stream(torch)) == 0
    got = host(torch, out).astype(np.float64)
    # fp32 sums of exact products: within k * 2^-24 of the magnitude sum
    mag = np.abs(a.astype(np.float16).astype(np.float64)) @ np.abs(b.astype(np.float16).astype(np.float64)).T
    assert (np.abs(got - exact) <= k * 2.0 ** -24 * (mag + np.abs(bias)) + 1e-30).all()
    # without the rounding the result differs (the operands are not binary16 values)
    args.half_operands = 0
    assert lib.dav2_hip_gemm_f32(C.byref(args), stream(torch)) == 0
    assert not np.array_equal(host(torch, out).astype(np.float64), got)


def test_round_half_matches_numpy(gpu, lib):
    torch = gpu
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(100003).astype(np.float32) * 10.0 ** rng.integers(-8, 6, 100003),
                        np.float32([0.0, -0.0, 65504.0, 65520.0, 1e6, -1e6, 2.0 ** -25, 2.0 ** -24, 6e-8])])
    x = x.astype(np.float32)
    xd = dev(torch, x)
    assert lib.dav2_hip_round_half(ptr(xd), x.size, stream(torch)) == 0
    got = host(torch, xd)
    want = x.astype(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.fixture(scope="module")
def models(pkg, tmp_path_factory):
    root = tmp_path_factory.mktemp("fp16_models")
    paths = {}
    for enc in ("vits", "vitb", "vitl"):
        p = root / f"{enc}.dav2"
        pkg.dav2_format.write_synthetic_model(p, enc, seed=SEED + ENC[enc] + 1)
        paths[enc] = p
    return paths


def _span_err(got, ref):
    span = float(ref.max() - ref.min())
    return float(np.abs(got - ref).max()) / (span if span > 0 else 1.0)


@pytest.mark.parametrize("enc,width,height,attention", [
    ("vits", 266, 266, "binary16"), ("vits", 350, 266, "binary16"), ("vits", 266, 266, "fp32"),
    ("vitb", 196, 252, "binary16"), ("vitl", 518, 518, "binary16"), ("vits", 350, 266, "coop"),
    ("vitl", 518, 518, "coop")])
def test_fp16_mode_depth_parity(gpu, pkg, lib, oracle, models, enc, width, height, attention):
    # coop: the fp16 mode with the cooperative-matrix score shader
    # (REFERENCE_FP16_COOP_ATTENTION) against the oracle's fp16 graph with
    # mode-3 attention, the same 1e-3 bound
    torch = gpu
    _announce("fp16 model", enc, width, height, attention)
    flags = pkg.FORCE_FP16 | {"fp32": pkg.FORCE_FP32_ATTENTION, "coop": pkg.REFERENCE_FP16_COOP_ATTENTION}.get(attention, 0)
    x = pkg.dav2_format.imagenet_input(width, height, seed=SEED + width + 1)[0]
    with pkg.Context(str(models[enc]), enc, flags) as ctx:
        depth = ctx.infer(x, width, height)
        xd = dev(torch, x)
        d2 = empty(torch, (height, width), torch.float32)
        logits = empty(torch, (height, width), torch.float32)
        assert lib.dav2_infer_tensor_f32_device_logits(ctx.handle, xd.data_ptr(), width, height, d2.data_ptr(),
                                                       logits.data_ptr(), stream(torch)) == 0
        d2, logits = host(torch, d2), host(torch, logits)
    h = oracle.load_model(models[enc], ENC[enc])
    try:
        ref_depth, ref_logits = oracle.infer_fp16(h, x, width, height, attention=attention)
    finally:
        oracle.free_model(h)
    assert np.isfinite(depth).all() and np.array_equal(depth, d2)
    e_depth, e_logits = _span_err(depth, ref_depth), _span_err(logits, ref_logits)
    print(f"fp16 parity {enc} {width}x{height} {attention}: depth {e_depth:.3g}, logits {e_logits:.3g}", flush=True)
    assert e_depth <= 1e-3 and e_logits <= 1e-3

"""Pins the oracle's whole int8 graph (orc_model_infer: encoder.cpp:322-597,
dpt.cpp:628-863 with every DPT convolution on the int8 path) against an
independent PyTorch restatement of the DepthAnythingV2 architecture
(depth_anything_v2/dinov2.py: prepare_tokens, Block, get_intermediate_layers;
depth_anything_v2/dpt.py: DPTHead, FeatureFusionBlock, ResidualConvUnit),
evaluated in float64 with int8 fake quantization at the same points (per-row
activations, per-output-channel weights). The two differ only by rounding, so
features agree to int8 resolution; a miswired graph does not (checked by
planting wiring mistakes in the restatement). CPU only."""

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

SEED = 0xDA20000
ENC = {"vits": 0, "vitb": 1, "vitl": 2}
CAPTURE = {"vits": (2, 5, 8, 11), "vitb": (2, 5, 8, 11), "vitl": (4, 11, 17, 23)}


def _fq_rows(x):
    """Per-row symmetric int8 (quantize_rows_int8_fused.glsl): returns q (as
    float64 integers) and the fp32 scales."""
    x32 = np.asarray(x, np.float32)
    s = np.maximum(np.abs(x32).max(axis=1) / np.float32(127.0), np.float32(1e-8)).astype(np.float32)
    q = np.rint(np.clip(x32 / s[:, None], -127, 127))
    return q.astype(np.float64), s.astype(np.float64)


def _linear(x, w, b):
    qx, sx = _fq_rows(x)
    qw, sw = _fq_rows(w)
    y = (qx @ qw.T) * sx[:, None] * sw[None, :]
    return y + (0.0 if b is None else b.astype(np.float64))


def _conv(x, w, b, stride=1, pad=0):
    """conv2d_int8: im2col rows (column c*k*k + ky*k + kx) quantized per pixel."""
    oc, c, k, _ = w.shape
    cols = F.unfold(torch.from_numpy(np.asarray(x, np.float32))[None], k, padding=pad, stride=stride)[0].T.numpy()
    oh = (x.shape[1] + 2 * pad - k) // stride + 1
    ow = (x.shape[2] + 2 * pad - k) // stride + 1
    y = _linear(cols, w.reshape(oc, -1), b)
    return y.T.reshape(oc, oh, ow)


def _conv_transpose(x, w, b):
    """stride == kernel ConvTranspose2d: input pixel rows quantized over C, weight
    rows (ky, kx, oc) quantized over the input channels."""
    c, h, wd = x.shape
    _, oc, k, _ = w.shape
    rows = np.asarray(x, np.float32).reshape(c, -1).T
    wr = w.transpose(2, 3, 1, 0).reshape(k * k * oc, c)
    y = _linear(rows, wr, None).reshape(h, wd, k, k, oc)
    return y.transpose(4, 0, 2, 1, 3).reshape(oc, h * k, wd * k) + b.astype(np.float64)[:, None, None]


def _ln(x, w, b):
    return F.layer_norm(torch.from_numpy(x).double(), (x.shape[1],), torch.from_numpy(w).double(),
                        torch.from_numpy(b).double(), eps=1e-6).numpy()


def _attention(qkv, heads):
    t, d = qkv.shape[0], heads * 64
    q = qkv[:, :d].reshape(t, heads, 64)
    k = qkv[:, d:2 * d].reshape(t, heads, 64)
    v = qkv[:, 2 * d:].reshape(t, heads, 64)
    sc = np.einsum("ihf,jhf->hij", q * 0.125, k)
    p = np.exp(sc - sc.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    return np.einsum("hij,jhf->ihf", p, v).reshape(t, d)


def _gelu(x):
    return F.gelu(torch.from_numpy(x)).numpy()


def _bilinear(x, oh, ow):
    return F.interpolate(torch.from_numpy(x)[None], size=(oh, ow), mode="bilinear", align_corners=True)[0].numpy()


def _reference(st, enc, image, width, height, miswire=None):
    """float64 DepthAnythingV2 with int8 fake quantization; returns (features,
    pre-ReLU logits)."""
    p = "pretrained."
    d = st[p + "cls_token"].shape[-1]
    heads = d // 64
    pw, ph = width // 14, height // 14
    # prepare_tokens: patch embedding, class token, bicubic position embedding
    patches = F.unfold(torch.from_numpy(image)[None], 14, stride=14)[0].T.numpy()
    tok = _linear(patches, st[p + "patch_embed.proj.weight"].reshape(d, -1), st[p + "patch_embed.proj.bias"])
    pos = st[p + "pos_embed"][0].astype(np.float64)
    grid = torch.from_numpy(pos[1:]).reshape(1, 37, 37, d).permute(0, 3, 1, 2)
    if (pw, ph) != (37, 37):
        grid = F.interpolate(grid, scale_factor=((ph + 0.1) / 37, (pw + 0.1) / 37), mode="bicubic",
                             align_corners=False)
    x = np.concatenate([st[p + "cls_token"][0].astype(np.float64) + pos[:1],
                        tok + grid[0].reshape(d, -1).T.numpy()])
    feats = []
    for i in range(len([k for k in st if k.endswith(".norm1.weight")])):
        b = f"{p}blocks.{i}."
        h = _ln(x, st[b + "norm1.weight"], st[b + "norm1.bias"])
        a = _attention(_linear(h, st[b + "attn.qkv.weight"], st[b + "attn.qkv.bias"]), heads)
        x = x + st[b + "ls1.gamma"] * _linear(a, st[b + "attn.proj.weight"], st[b + "attn.proj.bias"])
        h = _ln(x, st[b + "norm2.weight"], st[b + "norm2.bias"])
        m = _gelu(_linear(h, st[b + "mlp.fc1.weight"], st[b + "mlp.fc1.bias"]))
        mlp = st[b + "ls2.gamma"] * _linear(m, st[b + "mlp.fc2.weight"], st[b + "mlp.fc2.bias"])
        x = x + (0.0 if miswire == "drop_mlp" else mlp)
        if i in CAPTURE[enc]:
            feats.append(_ln(x, st[p + "norm.weight"], st[p + "norm.bias"]))
    # DPT head
    h = "depth_head."
    s = h + "scratch."
    layers = []
    for i, f in enumerate(feats):
        y = _linear(f[1:], st[f"{h}projects.{i}.weight"][:, :, 0, 0], st[f"{h}projects.{i}.bias"])
        y = y.T.reshape(-1, ph, pw)
        if i < 2:
            y = _conv_transpose(y, st[f"{h}resize_layers.{i}.weight"], st[f"{h}resize_layers.{i}.bias"])
        elif i == 3:
            y = _conv(y, st[h + "resize_layers.3.weight"], st[h + "resize_layers.3.bias"], stride=2, pad=1)
        layers.append(_conv(y, st[f"{s}layer{i + 1}_rn.weight"], None, pad=1))
    if miswire == "swap_skips":
        layers[1], layers[2] = layers[2], layers[1]

    def rcu(x, name):
        out = _conv(np.maximum(x, 0), st[name + ".conv1.weight"], st[name + ".conv1.bias"], pad=1)
        out = _conv(np.maximum(out, 0), st[name + ".conv2.weight"], st[name + ".conv2.bias"], pad=1)
        return out + x

    def fusion(path, skip, name, size):
        if skip is not None:
            path = path + rcu(skip, name + ".resConfUnit1")
        path = rcu(path, name + ".resConfUnit2")
        path = _bilinear(path, *size)
        return _conv(path, st[name + ".out_conv.weight"], st[name + ".out_conv.bias"])

    path = fusion(layers[3], None, s + "refinenet4", layers[2].shape[1:])
    path = fusion(path, layers[2], s + "refinenet3", layers[1].shape[1:])
    path = fusion(path, layers[1], s + "refinenet2", layers[0].shape[1:])
    path = fusion(path, layers[0], s + "refinenet1", (2 * layers[0].shape[1], 2 * layers[0].shape[2]))
    out = _conv(path, st[s + "output_conv1.weight"], st[s + "output_conv1.bias"], pad=1)
    out = _bilinear(out, height, width)
    out = np.maximum(_conv(out, st[s + "output_conv2.0.weight"], st[s + "output_conv2.0.bias"], pad=1), 0)
    out = _conv(out, st[s + "output_conv2.2.weight"], st[s + "output_conv2.2.bias"])
    return np.stack(feats), out[0]


@pytest.fixture(scope="module")
def graph_case(pkg, oracle, tmp_path_factory):
    enc, width, height = "vits", 98, 84
    st = pkg.dav2_format.synthetic_state(enc, SEED + 17)
    # LayerScale 0.5 instead of 1e-5 so that attention and the MLP shape the features
    for k in st:
        if k.endswith("ls1.gamma") or k.endswith("ls2.gamma"):
            st[k][:] = 0.5
    path = tmp_path_factory.mktemp("graph") / "vits.dav2"
    pkg.dav2_format.write_model(path, enc, st)
    image = pkg.dav2_format.imagenet_input(width, height, SEED + 5)[0]
    h = oracle.load_model(Path(path), ENC[enc])
    try:
        depth, logits, feats = oracle.infer(h, image, width, height, attention="exact", dim=384)
    finally:
        oracle.free_model(h)
    return st, enc, image, width, height, feats, logits


def _rel(a, b):
    return float(np.abs(a - b).max() / (np.abs(b).max() + 1e-30))


def test_encoder_features_match_restatement(graph_case):
    st, enc, image, width, height, feats, _ = graph_case
    ref_feats, _ = _reference(st, enc, image, width, height)
    # int8 rounding differences compound over the 12 blocks: about 2 %
    for i in range(4):
        assert _rel(feats[i], ref_feats[i]) <= 4e-2, i


def test_depth_logits_match_restatement(graph_case):
    st, enc, image, width, height, _, logits = graph_case
    _, ref = _reference(st, enc, image, width, height)
    span = ref.max() - ref.min()
    assert np.abs(logits - ref).max() <= 0.06 * span


@pytest.mark.parametrize("mistake", ["drop_mlp", "swap_skips"])
def test_planted_wiring_mistakes_are_detected(graph_case, mistake):
    st, enc, image, width, height, feats, logits = graph_case
    ref_feats, ref = _reference(st, enc, image, width, height, miswire=mistake)
    span = ref.max() - ref.min()
    feat_err = max(_rel(feats[i], ref_feats[i]) for i in range(4))
    # correct wiring: features within 4 %, logits within 6 % of the range
    assert feat_err > 0.25 or np.abs(logits - ref).max() > 0.25 * span

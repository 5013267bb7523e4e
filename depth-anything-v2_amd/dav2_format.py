"""The .dav2 model file: a seeded writer and a reader.

Format (fixed by the reference's loader, src/model.cpp:27-69, and converter,
tools/export_model.py:21-38): a 64-byte header, one 192-byte record per tensor
(names sorted), an optional 128-byte derivation record, then float32 payloads
at 64-byte aligned offsets, each with the CRC-32 of its bytes.

No checkpoints are available offline, so `write_synthetic_model` fills the
official Depth-Anything-V2 tensor names and shapes with seeded random values:
linear/qkv/proj/fc weights, patch-embed weight, class token and position
embedding ~ N(0, 0.02); patch-embed bias ~ N(0, 0.01); LayerNorm weight 1 and
bias 0; LayerScale gamma 1e-5; transformer biases 0; DPT convolution weights
and biases ~ U(+-1/sqrt(fan_in)) (PyTorch's default Kaiming-uniform).
"""

from __future__ import annotations

import struct
import zlib
from dataclasses import dataclass
from pathlib import Path

import numpy as np

MAGIC = b"DAV2MOD\0"
FORMAT_VERSION = 1
ENDIAN_TAG = 0x01020304
DTYPE_FLOAT32 = 1
HEADER = struct.Struct("<8sIIIIQQQQQ")
RECORD = struct.Struct("<112sII4QQQQIIQ")
METADATA = struct.Struct("<8sIIIIII32s64s")
ALIGNMENT = 64
ENCODERS = {"vits": 0, "vitb": 1, "vitl": 2}
RELATIVE_CONVERTER = b"dav2-export-pytorch-v1"
METRIC_CONVERTER = b"dav2-export-pytorch-metric-v1"

# src/encoder.cpp:40-70 and src/dpt.cpp:51-78
ARCH = {
    "vits": dict(dim=384, heads=6, depth=12, features=64, out_channels=(48, 96, 192, 384)),
    "vitb": dict(dim=768, heads=12, depth=12, features=128, out_channels=(96, 192, 384, 768)),
    "vitl": dict(dim=1024, heads=16, depth=24, features=256, out_channels=(256, 512, 1024, 1024)),
}


def _align(v: int) -> int:
    return (v + ALIGNMENT - 1) & ~(ALIGNMENT - 1)


def tensor_specs(encoder: str) -> dict[str, tuple[tuple[int, ...], str, float]]:
    """name -> (shape, init kind, parameter) for the full DepthAnythingV2 model."""
    a = ARCH[encoder]
    d, f, oc = a["dim"], a["features"], a["out_channels"]
    s: dict[str, tuple[tuple[int, ...], str, float]] = {}
    p = "pretrained."
    s[p + "cls_token"] = ((1, 1, d), "normal", 0.02)
    s[p + "pos_embed"] = ((1, 1370, d), "normal", 0.02)
    s[p + "mask_token"] = ((1, d), "const", 0.0)
    s[p + "patch_embed.proj.weight"] = ((d, 3, 14, 14), "normal", 0.02)
    s[p + "patch_embed.proj.bias"] = ((d,), "normal", 0.01)
    for i in range(a["depth"]):
        b = f"{p}blocks.{i}."
        s[b + "norm1.weight"] = ((d,), "const", 1.0)
        s[b + "norm1.bias"] = ((d,), "const", 0.0)
        s[b + "attn.qkv.weight"] = ((3 * d, d), "normal", 0.02)
        s[b + "attn.qkv.bias"] = ((3 * d,), "const", 0.0)
        s[b + "attn.proj.weight"] = ((d, d), "normal", 0.02)
        s[b + "attn.proj.bias"] = ((d,), "const", 0.0)
        s[b + "ls1.gamma"] = ((d,), "const", 1e-5)
        s[b + "norm2.weight"] = ((d,), "const", 1.0)
        s[b + "norm2.bias"] = ((d,), "const", 0.0)
        s[b + "mlp.fc1.weight"] = ((4 * d, d), "normal", 0.02)
        s[b + "mlp.fc1.bias"] = ((4 * d,), "const", 0.0)
        s[b + "mlp.fc2.weight"] = ((d, 4 * d), "normal", 0.02)
        s[b + "mlp.fc2.bias"] = ((d,), "const", 0.0)
        s[b + "ls2.gamma"] = ((d,), "const", 1e-5)
    s[p + "norm.weight"] = ((d,), "const", 1.0)
    s[p + "norm.bias"] = ((d,), "const", 0.0)

    h = "depth_head."

    def conv(name: str, cout: int, cin: int, k: int, bias: bool = True, fan_in: int | None = None) -> None:
        fi = fan_in if fan_in is not None else cin * k * k
        s[name + ".weight"] = ((cout, cin, k, k), "uniform", 1.0 / np.sqrt(fi))
        if bias:
            s[name + ".bias"] = ((cout,), "uniform", 1.0 / np.sqrt(fi))

    for i, c in enumerate(oc):
        conv(f"{h}projects.{i}", c, d, 1)
    # ConvTranspose2d weight is [in, out, k, k]; PyTorch's fan_in uses dim 1.
    s[h + "resize_layers.0.weight"] = ((oc[0], oc[0], 4, 4), "uniform", 1.0 / np.sqrt(oc[0] * 16))
    s[h + "resize_layers.0.bias"] = ((oc[0],), "uniform", 1.0 / np.sqrt(oc[0] * 16))
    s[h + "resize_layers.1.weight"] = ((oc[1], oc[1], 2, 2), "uniform", 1.0 / np.sqrt(oc[1] * 4))
    s[h + "resize_layers.1.bias"] = ((oc[1],), "uniform", 1.0 / np.sqrt(oc[1] * 4))
    conv(h + "resize_layers.3", oc[3], oc[3], 3)
    for i, c in enumerate(oc):
        conv(f"{h}scratch.layer{i + 1}_rn", f, c, 3, bias=False)
    for r in range(1, 5):
        base = f"{h}scratch.refinenet{r}"
        conv(base + ".out_conv", f, f, 1)
        for u in (1, 2):
            for cv in (1, 2):
                conv(f"{base}.resConfUnit{u}.conv{cv}", f, f, 3)
    conv(h + "scratch.output_conv1", f // 2, f, 3)
    conv(h + "scratch.output_conv2.0", 32, f // 2, 3)
    conv(h + "scratch.output_conv2.2", 1, 32, 1)
    return s


def synthetic_state(encoder: str, seed: int) -> dict[str, np.ndarray]:
    """Seeded float32 tensors for every name of `tensor_specs` (sorted order)."""
    rng = np.random.default_rng(seed)
    out: dict[str, np.ndarray] = {}
    for name, (shape, kind, param) in sorted(tensor_specs(encoder).items()):
        if kind == "normal":
            v = rng.standard_normal(shape, dtype=np.float32) * np.float32(param)
        elif kind == "uniform":
            v = rng.uniform(-param, param, size=shape).astype(np.float32)
        else:
            v = np.full(shape, param, dtype=np.float32)
        out[name] = np.ascontiguousarray(v, dtype=np.float32)
    return out


def write_model(path: str | Path, encoder: str, state: dict[str, np.ndarray], *, derivation: bool = True,
                metric_max_depth: float = 0.0, sha256: bytes = bytes(range(32))) -> None:
    """Writes `state` as a .dav2 file the way tools/export_model.py:116-201 lays it out."""
    names = sorted(state)
    records = []
    directory_offset = HEADER.size
    metadata_offset = directory_offset + len(names) * RECORD.size
    data_offset = _align(metadata_offset + (METADATA.size if derivation else 0))
    cursor = data_offset
    payloads = []
    for name in names:
        arr = np.ascontiguousarray(state[name], dtype=np.float32)
        if not 1 <= arr.ndim <= 4:
            raise ValueError(f"unsupported rank for {name}")
        encoded = name.encode("utf-8")
        if len(encoded) >= 112:
            raise ValueError(f"tensor name too long: {name}")
        payload = memoryview(arr.reshape(-1)).cast("B")
        cursor = _align(cursor)
        dims = list(arr.shape) + [0] * (4 - arr.ndim)
        records.append(RECORD.pack(encoded, DTYPE_FLOAT32, arr.ndim, *dims, cursor, payload.nbytes, arr.size,
                                   zlib.crc32(payload), 0, 0))
        payloads.append((cursor, payload))
        cursor += payload.nbytes
    file_bytes = cursor
    header = HEADER.pack(MAGIC, FORMAT_VERSION, ENDIAN_TAG, ENCODERS[encoder], len(names), directory_offset,
                         len(names) * RECORD.size, data_offset, file_bytes, metadata_offset if derivation else 0)
    with open(path, "wb") as f:
        f.write(header)
        for r in records:
            f.write(r)
        if derivation:
            metric = metric_max_depth > 0.0
            f.write(METADATA.pack(b"DAV2META", 1, METADATA.size, FORMAT_VERSION, ENCODERS[encoder],
                                  1 if metric else 0,
                                  struct.unpack("<I", struct.pack("<f", metric_max_depth))[0] if metric else 0,
                                  sha256, METRIC_CONVERTER if metric else RELATIVE_CONVERTER))
        for offset, payload in payloads:
            f.write(b"\0" * (offset - f.tell()))
            f.write(payload)
        assert f.tell() == file_bytes


def write_synthetic_model(path: str | Path, encoder: str, seed: int) -> dict[str, np.ndarray]:
    state = synthetic_state(encoder, seed)
    write_model(path, encoder, state)
    return state


@dataclass
class TensorRecord:
    name: str
    shape: tuple[int, ...]
    offset: int
    nbytes: int
    crc32: int


def read_records(path: str | Path) -> tuple[dict, list[TensorRecord]]:
    """Parses header and directory (no validation beyond the struct layout)."""
    with open(path, "rb") as f:
        head = HEADER.unpack(f.read(HEADER.size))
        keys = ("magic", "version", "endian", "encoder", "tensor_count", "directory_offset", "directory_bytes",
                "data_offset", "file_bytes", "metadata_offset")
        header = dict(zip(keys, head))
        f.seek(header["directory_offset"])
        recs = []
        for _ in range(header["tensor_count"]):
            r = RECORD.unpack(f.read(RECORD.size))
            name = r[0].split(b"\0", 1)[0].decode()
            rank = r[2]
            recs.append(TensorRecord(name, tuple(r[3:3 + rank]), r[7], r[8], r[10]))
    return header, recs


def imagenet_input(width: int, height: int, seed: int, batch: int = 1) -> np.ndarray:
    """Seeded U[0,1) RGB pixels, ImageNet-normalised, float32 [batch][3][H][W]."""
    rng = np.random.default_rng(seed)
    x = rng.random((batch, 3, height, width), dtype=np.float32)
    mean = np.array([0.485, 0.456, 0.406], dtype=np.float32).reshape(1, 3, 1, 1)
    std = np.array([0.229, 0.224, 0.225], dtype=np.float32).reshape(1, 3, 1, 1)
    return np.ascontiguousarray((x - mean) / std, dtype=np.float32)

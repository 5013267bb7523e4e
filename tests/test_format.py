""".dav2 format: the seeded writer, this build's loader and the reference's
own loader (src/model.cpp, built into oracle/_ref) on the fixtures of
tests/model_metadata.cpp:63-213 and on corrupted files. CPU only."""

import ctypes as C
import json
import shutil
import struct
import zlib
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
KATS = json.loads((GOLDEN / "reference_kats.json").read_text())
FORMAT_MESSAGES = ("invalid DAV2", "model file is truncated", "model encoder does not match", "duplicate DAV2")


def ref_verdict(ref_lib, path, encoder=0):
    n, present, depth = C.c_uint(), C.c_int(), C.c_float()
    err = C.create_string_buffer(256)
    rc = ref_lib.ref_model_open(str(path).encode(), encoder, C.byref(n), C.byref(present), C.byref(depth), err, 256)
    return rc, err.value.decode(), n.value, present.value, depth.value


def our_verdict(pkg, lib, path, encoder="vits"):
    """dav2_create validates the file before any device work; a file that
    passes fails afterwards for another reason (no GPU here, or a fixture that
    is not a full model)."""
    opts = pkg.create_options(encoder)
    ctx = C.c_void_p()
    st = lib.dav2_create(str(path).encode(), C.byref(opts), C.byref(ctx))
    if st == 0:
        lib.dav2_destroy(ctx)
        return "accept", ""
    msg = lib.dav2_last_error().decode()
    return ("reject" if any(m in msg for m in FORMAT_MESSAGES) else "accept"), msg


def test_crc32_kat(oracle):
    assert oracle.lib.orc_crc32(b"123456789", 9) == KATS["crc32_123456789"]
    data = np.random.default_rng(0).integers(0, 256, 100000, dtype=np.uint8).tobytes()
    assert oracle.lib.orc_crc32(data, len(data)) == zlib.crc32(data)


@pytest.mark.parametrize("name", sorted(KATS["metadata_verdicts"]))
def test_metadata_fixtures(pkg, lib, ref_lib, name):
    path = GOLDEN / name
    expected = KATS["metadata_verdicts"][name]
    rc, msg, n, present, depth = ref_verdict(ref_lib, path)
    assert ("accept" if rc == 0 else "reject") == expected, msg
    if rc == 0:
        assert n == 1 and depth == KATS["metadata_metric_max_depth"][name]
        assert present == (0 if "legacy" in name else 1)
    verdict, why = our_verdict(pkg, lib, path)
    assert verdict == expected, why
    if expected == "reject":
        assert why == msg  # same message as the reference loader


def _mutate(src: Path, dst: Path, offset: int, fmt_: str, value) -> Path:
    shutil.copy(src, dst)
    with open(dst, "r+b") as f:
        f.seek(offset)
        f.write(struct.pack(fmt_, value))
    return dst


CORRUPTIONS = [
    ("bad_magic", 0, "<8s", b"DAV2MOX\0"),
    ("bad_version", 8, "<I", 2),
    ("bad_endian", 12, "<I", 0x04030201),
    ("wrong_encoder", 16, "<I", 1),
    ("zero_tensors", 20, "<I", 0),
    ("file_bytes", 48, "<Q", 10**6),
    ("directory_bytes", 32, "<Q", 191),
    ("data_offset_misaligned", 40, "<Q", 390),
    ("metadata_offset", 56, "<Q", 200),
    ("record_dtype", 64 + 112, "<I", 2),
    ("record_rank0", 64 + 116, "<I", 0),
    ("record_rank5", 64 + 116, "<I", 5),
    ("record_unused_dim", 64 + 128, "<Q", 3),
    ("record_zero_dim", 64 + 120, "<Q", 0),
    ("record_count", 64 + 168, "<Q", 2),
    ("record_flags", 64 + 180, "<I", 1),
    ("record_offset_misaligned", 64 + 152, "<Q", 388),
    ("record_name_unterminated", 64, "<112s", b"x" * 112),
    ("record_name_empty", 64, "<B", 0),
    ("metadata_flags", 256 + 24, "<I", 2),
    ("metadata_converter", 256 + 64, "<8s", b"other\0\0\0"),
    ("metadata_version", 256 + 8, "<I", 9),
]


@pytest.mark.parametrize("name,offset,fmt_,value", CORRUPTIONS, ids=[c[0] for c in CORRUPTIONS])
def test_corrupted_files_rejected_like_reference(pkg, lib, ref_lib, tmp_path, name, offset, fmt_, value):
    path = _mutate(GOLDEN / "model_metadata_derived.dav2", tmp_path / f"{name}.dav2", offset, fmt_, value)
    rc, msg, *_ = ref_verdict(ref_lib, path)
    verdict, why = our_verdict(pkg, lib, path)
    assert rc != 0, f"reference accepted {name}"
    assert verdict == "reject", why
    assert why == msg


def test_truncated_file(pkg, lib, ref_lib, tmp_path):
    p = tmp_path / "t.dav2"
    p.write_bytes((GOLDEN / "model_metadata_derived.dav2").read_bytes()[:40])
    assert ref_verdict(ref_lib, p)[0] != 0
    assert our_verdict(pkg, lib, p)[0] == "reject"


def test_synthetic_model_round_trip(pkg, ref_lib, tmp_path):
    fmt = pkg.dav2_format
    path = tmp_path / "vits.dav2"
    state = fmt.write_synthetic_model(path, "vits", seed=1)
    rc, msg, n, present, depth = ref_verdict(ref_lib, path, 0)
    assert rc == 0, msg
    assert n == len(state) and present == 1 and depth == 0.0
    header, records = fmt.read_records(path)
    assert header["tensor_count"] == len(state) and [r.name for r in records] == sorted(state)
    for name in ("pretrained.pos_embed", "depth_head.resize_layers.0.weight", "pretrained.blocks.3.mlp.fc1.weight"):
        buf = np.empty(state[name].size, np.float32)
        assert ref_lib.ref_model_tensor(str(path).encode(), 0, name.encode(), buf.ctypes.data, buf.size) == buf.size
        assert np.array_equal(buf, state[name].reshape(-1))
    # official shapes (depth_anything_v2/dpt.py, dinov2.py)
    shapes = {r.name: r.shape for r in records}
    assert shapes["pretrained.pos_embed"] == (1, 1370, 384)
    assert shapes["depth_head.resize_layers.0.weight"] == (48, 48, 4, 4)
    assert shapes["depth_head.scratch.output_conv2.2.weight"] == (1, 32, 1, 1)
    assert sum(np.prod(s) for s in shapes.values()) == pytest.approx(24.8e6, rel=0.01)


def test_oracle_rejects_bad_crc(oracle, pkg, tmp_path):
    fmt = pkg.dav2_format
    path = tmp_path / "vits.dav2"
    fmt.write_synthetic_model(path, "vits", seed=2)
    _, records = fmt.read_records(path)
    data = bytearray(path.read_bytes())
    data[records[0].offset] ^= 0xFF
    path.write_bytes(bytes(data))
    with pytest.raises(RuntimeError, match="crc"):
        oracle.load_model(path, 0)


def test_mutated_files_match_reference_loader(pkg, lib, ref_lib, tmp_path):
    # Differential check of the header / index parser: 400 seeded mutations of
    # the metadata fixtures (bit flips, truncations, 32- and 64-bit boundary
    # values at aligned offsets, appended bytes); this build's verdict and
    # message equal the reference loader's (src/model.cpp) on every one.
    import random
    rng = random.Random(20261202)
    fixtures = sorted(GOLDEN.glob("*.dav2"))
    verdicts = {"accept": 0, "reject": 0}
    for it in range(400):
        b = bytearray(rng.choice(fixtures).read_bytes())
        kind = it % 5
        if kind == 0:
            for _ in range(rng.randint(1, 4)):
                i = rng.randrange(len(b))
                b[i] ^= 1 << rng.randrange(8)
        elif kind == 1:
            b = b[:rng.randrange(len(b))]
        elif kind == 2:
            i = rng.randrange(0, len(b) - 4) & ~3
            b[i:i + 4] = struct.pack("<I", rng.choice([0, 1, 0x7FFFFFFF, 0x80000000, 0xFFFFFFFF, len(b), 64, 4096]))
        elif kind == 3:
            i = rng.randrange(0, len(b) - 8) & ~7
            b[i:i + 8] = struct.pack("<Q", rng.choice([0, 1, 2**63, 2**64 - 1, len(b), 2**32, 2**40]))
        else:
            b += bytes(rng.randrange(256) for _ in range(rng.randint(1, 64)))
        path = tmp_path / f"mutated_{it % 4}.dav2"
        path.write_bytes(bytes(b))
        rc, msg, *_ = ref_verdict(ref_lib, path)
        want = "accept" if rc == 0 else "reject"
        got, why = our_verdict(pkg, lib, path)
        assert got == want, (it, kind, msg, why)
        if want == "reject":
            assert why == msg, (it, kind)
        verdicts[want] += 1
    assert verdicts["accept"] > 20 and verdicts["reject"] > 200

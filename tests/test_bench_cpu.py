"""bench.py's host-side contract, without a GPU: it measures one GPU and
refuses more, and its per-GEMM-shape table prices each shape against
max(2MNK / 5 POP/s, bytes / 8 TB/s)."""

import importlib.util
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_more_than_one_gpu_is_refused():
    run = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=300)
    assert run.returncode != 0
    assert "--gpus 2 is not supported" in run.stdout + run.stderr


def test_gemm_shape_table_prices_each_shape():
    bench = _bench()
    prof = {
        # fc2 at batch 8: 24 launches of 65.5 us, LayerScale (residual read back)
        "gemm_i8@10960x1024x4096:row_layerscale": {"ms": 24 * 0.0655, "launches": 24, "work": 0.0, "unit": "op"},
        # fc1 at batch 1: one launch of 18.3 us
        "gemm_i8@1370x4096x1024:row_gelu": {"ms": 0.0183, "launches": 1, "work": 0.0, "unit": "op"},
        "gemm_i8": {"ms": 1.0, "launches": 25, "work": 0.0, "unit": "op"},  # not a shape key
        "layer_norm": {"ms": 0.1, "launches": 4, "work": 0.0, "unit": "B"},
    }
    table = bench.gemm_shape_table(prof, steps=2)
    assert list(table) == ["10960x1024x4096:row_layerscale", "1370x4096x1024:row_gelu"]  # most time per step first

    fc2 = table["10960x1024x4096:row_layerscale"]
    m, n, k = 10960, 1024, 4096
    ops = 2.0 * m * n * k
    nbytes = m * k + n * k + 2 * 4.0 * m * n + 4.0 * m + 8.0 * n
    assert fc2["launches_per_step"] == 12
    assert fc2["avg_us"] == pytest.approx(65.5)
    assert fc2["attainable_us"] == pytest.approx(ops / 5e15 * 1e6)  # 18.4 us of MFMA > 17.4 us of HBM
    assert nbytes / 8e12 < ops / 5e15
    assert fc2["bound"] == "mfma"
    assert fc2["T/s"] == pytest.approx(ops / 65.5e-6 / 1e12)
    assert fc2["frac"] == pytest.approx(fc2["T/s"] / 5000.0)

    fc1 = table["1370x4096x1024:row_gelu"]
    m, n, k = 1370, 4096, 1024
    nbytes = m * k + n * k + 4.0 * m * n + 4.0 * m + 8.0 * n  # no residual
    assert fc1["bound"] == "hbm"
    assert fc1["attainable_us"] == pytest.approx(nbytes / 8e12 * 1e6)
    assert fc1["frac_of_attainable"] == pytest.approx(nbytes / 8e12 / 18.3e-6)

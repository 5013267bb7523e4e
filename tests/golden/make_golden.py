#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/ (run from the repo root).

* model_metadata_*.dav2 - the four .dav2 fixtures of the reference's
  tests/model_metadata.cpp:63-213: one float32 tensor "weight" = 42.0, ViT-S
  header, derivation record with sha256 bytes 0..31 and converter
  "dav2-export-pytorch-v1" (derived), metric 20 m and 40 m (invalid) with
  "dav2-export-pytorch-metric-v1", and a legacy file without the record.
* reference_kats.json - literal known answers from the reference's tests:
  CRC-32 of "123456789" (tests/vulkan_smoke.cpp:68-69), min/max + relative
  normalisation of {2,3,5,10} (:121-142), network shapes (tests/c_abi_smoke.c:16-21).
"""

import importlib.util
import json
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
OUT = Path(__file__).resolve().parent

spec = importlib.util.spec_from_file_location("dav2_format", ROOT / "depth-anything-v2_amd" / "dav2_format.py")
fmt = importlib.util.module_from_spec(spec)
import sys
sys.modules["dav2_format"] = fmt
spec.loader.exec_module(fmt)


def main():
    state = {"weight": np.array([42.0], np.float32)}
    fmt.write_model(OUT / "model_metadata_derived.dav2", "vits", state, derivation=True)
    fmt.write_model(OUT / "model_metadata_metric20.dav2", "vits", state, derivation=True, metric_max_depth=20.0)
    fmt.write_model(OUT / "model_metadata_metric40.dav2", "vits", state, derivation=True, metric_max_depth=40.0)
    fmt.write_model(OUT / "model_metadata_legacy.dav2", "vits", state, derivation=False)
    kats = {
        "crc32_123456789": 0xCBF43926,
        "minmax_input": [2.0, 3.0, 5.0, 10.0],
        "minmax_normalized": [0.0, 0.125, 0.375, 1.0],
        "minmax_tolerance": 1e-6,
        "network_shapes": [[640, 480, 518, 686, 518], [480, 640, 518, 518, 686]],
        "metadata_verdicts": {"model_metadata_derived.dav2": "accept", "model_metadata_metric20.dav2": "accept",
                              "model_metadata_metric40.dav2": "reject", "model_metadata_legacy.dav2": "accept"},
        "metadata_metric_max_depth": {"model_metadata_derived.dav2": 0.0, "model_metadata_metric20.dav2": 20.0,
                                      "model_metadata_legacy.dav2": 0.0},
    }
    (OUT / "reference_kats.json").write_text(json.dumps(kats, indent=1) + "\n")


if __name__ == "__main__":
    main()

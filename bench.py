#!/usr/bin/env python3
"""Throughput of the int8 Depth-Anything-V2 path on one MI355X.

Workload (default): ViT-L + DPT at 518x518, batch 1, int8 GEMMs and
convolutions with this build's integer-exact fused attention (in place of the
reference's binary16 attention of its int8 mode), seeded random weights in
a .dav2 file and a seeded ImageNet-normalised input. One step = one call of
the public entry dav2_infer_tensor_f32 on one image (host buffers: the input's
upload and the depth map's download are inside the step); `value` = 1 / the
median step time. With --batch B > 1 a step is one call of the batched device
entry dav2_infer_tensor_f32_device on B images already in HBM. Reported
beside it: the same graph with the input already resident in HBM
(dav2_infer_tensor_f32_device), and the int8 graph with the reference's own
binary16 attention arithmetic (DAV2_CREATE_REFERENCE_FP16_ATTENTION) through
the same host entry. Prints one JSON line.

Roofline: the dominant kernel is the int8 MFMA GEMM. Its algorithmic work is
2*M*N*K int8 ops per launch (unpadded K); achieved = total ops / total
launch time, measured with a start and a stop HIP event per GEMM launch that
its kernel dispatches record (hipExtLaunchKernelGGL) on the stream it runs on,
during a second timed pass of the same K steps.
"""

from __future__ import annotations

import argparse
import importlib.util
import json
import os
import sys
import tempfile
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
SEED = 0xDA20000
PEAK_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_HBM_GBS = 8000.0


def load_package():
    spec = importlib.util.spec_from_file_location("dav2_amd", ROOT / "depth-anything-v2_amd" / "__init__.py")
    mod = importlib.util.module_from_spec(spec)
    sys.modules.setdefault("dav2_amd", mod)
    spec.loader.exec_module(mod)
    return mod


def cpu_baseline(model_path: Path, encoder: str, size: int, budget_s: float) -> dict:
    """The CPU oracle (this build's restatement of the reference operators) on
    the host cores: one full image of the same workload, or - if one image
    exceeds the budget - the patch embedding plus as many encoder blocks as fit,
    extrapolated to the full image from the measured per-block time."""
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_py import Oracle

    fmt = load_package().dav2_format
    oracle = Oracle()
    # Every core this process may run on; OMP_NUM_THREADS, where the host
    # sets it (the GPU host caps a one-GPU job's CPU share this way), wins.
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or host_cpus()["usable"]
    oracle.lib.orc_set_threads(threads)
    enc_id = {"vits": 0, "vitb": 1, "vitl": 2}[encoder]
    h = oracle.load_model(model_path, enc_id)
    try:
        x = fmt.imagenet_input(size, size, SEED + 3)[0]
        t0 = time.perf_counter()
        oracle.infer(h, x, size, size, attention="exact")
        dt = time.perf_counter() - t0
        return {"value": 1.0 / dt, "unit": "images/s", "cores": oracle.lib.orc_get_threads(), "kind": "port",
                "sample": f"1 full {encoder} {size}x{size} image through the oracle's int8 graph ({dt:.2f} s)",
                **{f"host_{k}": v for k, v in host_cpus().items()}}
    finally:
        oracle.free_model(h)


def host_cpus() -> dict:
    """CPU facts of this host: logical CPUs (nproc of the machine), the CPUs
    this process may run on, and the CPU model name."""
    model = ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return {"nproc": os.cpu_count() or 1, "usable": usable, "cpu_model": model}


def cpu_preprocess_ms(width: int, height: int, input_size: int) -> float:
    """The oracle's restatement of the reference's CPU BGR8 preprocessing
    (src/image.cpp:163-270) on one frame, OpenMP over the host cores; the best
    of three runs."""
    import numpy as np
    sys.path.insert(0, str(ROOT / "tests"))
    from oracle_py import Oracle

    oracle = Oracle()
    dw, dh = oracle.network_shape(width, height, input_size)
    buf = np.random.default_rng(SEED + 5).integers(0, 256, size=width * height * 3, dtype=np.uint8)
    best = float("inf")
    for _ in range(3):
        t0 = time.perf_counter()
        oracle.preprocess_bgr8(buf, width, height, width * 3, dw, dh)
        best = min(best, time.perf_counter() - t0)
    return 1e3 * best


# gelu_quantize_rows_i8 (fc2's input quantization with fc1's GELU, from 4096
# rows) moves the bytes of quantize_rows_i8 but is bound by its GELU's VALU
# work; its HBM rate is reported all the same.
BANDWIDTH_KERNELS = ("layer_norm_quantize_i8", "layer_norm", "softmax_f32", "quantize_rows_i8", "gelu_quantize_rows_i8")


def gemm_shape_table(prof: dict, steps: int) -> dict:
    """Per GEMM shape (profiler keys "gemm_i8@MxNxK:epilogue"): average
    launch time, int8 rate, and the attainable bound of that shape,
    max(ops / 5 POP/s, bytes / 8 TB/s), with bytes = the int8 operands
    (M*K + N*K), the fp32 output (4*M*N, plus 4*M*N read back by the
    LayerScale-residual and residual epilogues) and the scales and bias."""
    table = {}
    for name, v in prof.items():
        if not name.startswith("gemm_i8@") or not v["ms"]:
            continue
        dims, tag = name.split("@", 1)[1].split(":")
        m, n, k = (int(t) for t in dims.split("x"))
        ops = 2.0 * m * n * k
        out_bytes = 4.0 * m * n * (2 if tag in ("row_layerscale", "transposed_residual") else 1)
        nbytes = m * k + n * k + out_bytes + 4.0 * m + 8.0 * n
        avg_s = v["ms"] * 1e-3 / v["launches"]
        bound_s = max(ops / (PEAK_INT8_TOPS * 1e12), nbytes / (PEAK_HBM_GBS * 1e9))
        table[f"{dims}:{tag}"] = {"launches_per_step": v["launches"] / steps, "avg_us": 1e6 * avg_s,
                                  "T/s": ops / avg_s / 1e12, "frac": ops / avg_s / 1e12 / PEAK_INT8_TOPS,
                                  "attainable_us": 1e6 * bound_s, "frac_of_attainable": bound_s / avg_s,
                                  "bound": "mfma" if ops / (PEAK_INT8_TOPS * 1e12) >= nbytes / (PEAK_HBM_GBS * 1e9)
                                  else "hbm"}
    return dict(sorted(table.items(), key=lambda kv: -kv[1]["avg_us"] * kv[1]["launches_per_step"]))


def profile_config(pkg, fmt, torch, model: Path, size: int, batch: int, fp32_attention: bool, steps: int) -> dict:
    """A few profiled steps of one configuration: per-launch HIP events give
    each kernel's time; reported are the GEMM's int8 rate and the HBM rate of
    the bandwidth-bound kernels, with the images/s of the profiled pass."""
    flags = pkg.FORCE_INT8 | (pkg.FORCE_FP32_ATTENTION if fp32_attention else 0)
    x = torch.from_numpy(fmt.imagenet_input(size, size, SEED + 3, batch)).cuda()
    n_out = batch * size * size
    out = torch.empty(n_out, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    with pkg.Context(str(model), "vitl", flags) as ctx:
        ctx.infer_device(x.data_ptr(), batch, size, size, out.data_ptr(), n_out, stream)
        torch.cuda.synchronize()
        ctx.profile(True)
        t0 = time.perf_counter()
        for _ in range(steps):
            ctx.infer_device(x.data_ptr(), batch, size, size, out.data_ptr(), n_out, stream)
        torch.cuda.synchronize()
        dt = time.perf_counter() - t0
        prof = ctx.profile_report()
        ctx.profile(False)
    res = {"profiled_images_per_s": batch * steps / dt}
    g = prof.get("gemm_i8")
    if g and g["ms"]:
        rate = g["work"] / (g["ms"] * 1e-3) / 1e12
        res["gemm_i8"] = {"T/s": rate, "frac": rate / PEAK_INT8_TOPS, "avg_us": 1e3 * g["ms"] / g["launches"]}
        # the encoder's GEMM shapes (the most time per step)
        res["gemm_shapes"] = dict(list(gemm_shape_table(prof, steps).items())[:6])
    for name in BANDWIDTH_KERNELS:
        v = prof.get(name)
        if v and v["ms"]:
            rate = v["work"] / (v["ms"] * 1e-3) / 1e9
            res[name] = {"GB/s": rate, "frac_hbm": rate / PEAK_HBM_GBS, "avg_us": 1e3 * v["ms"] / v["launches"]}
    del x, out
    torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--encoder", default="vitl", choices=["vits", "vitb", "vitl"])
    ap.add_argument("--size", type=int, default=518)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--fp32-attention", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=30.0)
    ap.add_argument("--profile-json", default="")
    ap.add_argument("--no-fp32-mode", action="store_true", help="skip the FORCE_FP32 / FORCE_FP16 / REFERENCE_FP16_ATTENTION comparison runs")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the batch-8 / 1036x1036 kernel measurements")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run one device-to-device copy of MIB MiB (HBM counter calibration) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported "
              "(images are independent, so several GPUs would each run their own share of the batch)",
              file=sys.stderr)
        return 2
    if args.size % 14:
        print("--size must be a multiple of 14", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    if args.copy_calibration:
        # A plain copy kernel of known size: reads and writes exactly
        # MIB MiB, so FETCH_SIZE / WRITE_SIZE of its dispatch give the
        # factor between those counters and HBM bytes.
        n = args.copy_calibration * 2**20 // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": n * 4}))
        return 0

    pkg = load_package()
    fmt = pkg.dav2_format
    flags = pkg.FORCE_INT8 | (pkg.FORCE_FP32_ATTENTION if args.fp32_attention else 0)
    with tempfile.TemporaryDirectory(prefix="dav2_bench_") as tmp:
        model = Path(tmp) / f"{args.encoder}.dav2"
        fmt.write_synthetic_model(model, args.encoder, seed=SEED + 3)
        print(f"bench: wrote {model.stat().st_size / 2**20:.0f} MiB synthetic {args.encoder} model", file=sys.stderr,
              flush=True)
        ctx = pkg.Context(str(model), args.encoder, flags)
        x = torch.from_numpy(fmt.imagenet_input(args.size, args.size, SEED + 3, args.batch)).cuda()
        n_out = args.batch * args.size * args.size
        out = torch.empty(n_out, dtype=torch.float32, device="cuda")
        stream = torch.cuda.current_stream().cuda_stream

        def device_step():
            ctx.infer_device(x.data_ptr(), args.batch, args.size, args.size, out.data_ptr(), n_out, stream)

        x_host = fmt.imagenet_input(args.size, args.size, SEED + 3)[0]

        def host_step():
            ctx.infer(x_host, args.size, args.size)  # synchronous: returns with the depth map on the host

        step = host_step if args.batch == 1 else device_step
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        # The timed region: exactly K steps, each timed on its own (every step
        # ends synchronised); value = batch / median step time.
        calls = []
        t0 = time.perf_counter()
        for _ in range(args.steps):
            h0 = time.perf_counter()
            step()
            if args.batch > 1:
                torch.cuda.synchronize()
            calls.append(time.perf_counter() - h0)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        median_s = float(np.median(calls))
        print(f"bench: {args.steps} steps in {elapsed:.3f} s (median {1e3 * median_s:.3f} ms)", file=sys.stderr,
              flush=True)
        host_entry = {"entry": ("dav2_infer_tensor_f32 (host buffers, PCIe copies included)" if args.batch == 1
                                else "dav2_infer_tensor_f32_device (batched device entry)"),
                      "calls": len(calls), "median_ms": 1e3 * median_s, "mean_ms": 1e3 * float(np.mean(calls)),
                      "min_ms": 1e3 * float(np.min(calls)), "images_per_s_median": args.batch / median_s}

        # The same graph on an input already resident in HBM
        # (dav2_infer_tensor_f32_device): K back-to-back steps, and the median
        # of per-step synchronised times.
        for _ in range(2):
            device_step()
        torch.cuda.synchronize()
        d0 = time.perf_counter()
        for _ in range(args.steps):
            device_step()
        torch.cuda.synchronize()
        device_rate = args.batch * args.steps / (time.perf_counter() - d0)
        step_s = []
        for _ in range(max(20, args.steps)):
            s0 = time.perf_counter()
            device_step()
            torch.cuda.synchronize()
            step_s.append(time.perf_counter() - s0)
        device_median = args.batch / float(np.median(step_s))
        host_steps = min(args.steps, 10)

        # Host-image entries (dav2_infer_bgr8): a 518x518 BGR8 frame through
        # the GPU preprocessing and the same inference, PCIe copies included;
        # then the cubic preprocessing kernel alone on a 1920x1080 frame
        # (resized to the 518 network shape, 924x518), timed with HIP events
        # on the stream it runs on.
        image_paths = None
        if args.batch == 1:
            import ctypes as C
            lib = pkg.load()
            rng = np.random.default_rng(SEED + 5)
            bgr = rng.integers(0, 256, size=(args.size, args.size, 3), dtype=np.uint8)
            ctx.infer_bgr8(bgr, args.size)
            b0 = time.perf_counter()
            for _ in range(host_steps):
                ctx.infer_bgr8(bgr, args.size)
            bgr_rate = host_steps / (time.perf_counter() - b0)
            fw, fh = 1920, 1080
            shape = pkg.ImageShape()
            pkg.check(lib.dav2_get_network_shape(fw, fh, 518, C.byref(shape)), lib)
            frame = torch.from_numpy(rng.integers(0, 256, size=fh * fw * 3, dtype=np.uint8)).cuda()
            pre = torch.empty(3 * shape.width * shape.height, dtype=torch.float32, device="cuda")

            def preprocess():
                pkg.check(lib.dav2_hip_preprocess_bgr8(frame.data_ptr(), fw, fh, fw * 3, shape.width, shape.height,
                                                       pre.data_ptr(), stream), lib)

            for _ in range(3):
                preprocess()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            reps = 50
            e0.record()
            for _ in range(reps):
                preprocess()
            e1.record()
            torch.cuda.synchronize()
            pre_us = 1e3 * e0.elapsed_time(e1) / reps
            pre_bytes = fw * fh * 3 + 3 * shape.width * shape.height * 4
            image_paths = {
                "bgr8_entry_images_per_s": bgr_rate,
                "bgr8_entry": f"dav2_infer_bgr8, {args.size}x{args.size} BGR8 host frame, input_size {args.size}",
                "preprocess_bgr8": {"frame": f"{fw}x{fh} BGR8 -> {shape.width}x{shape.height} RGB CHW",
                                    "avg_us": pre_us, "bytes": pre_bytes,
                                    "GB/s": pre_bytes / (pre_us * 1e-6) / 1e9,
                                    "frac_hbm": pre_bytes / (pre_us * 1e-6) / 1e9 / PEAK_HBM_GBS}}

        # Second pass with per-launch HIP events for the kernel rooflines.
        ctx.profile(True)
        torch.cuda.synchronize()
        p0 = time.perf_counter()
        for _ in range(args.steps):
            device_step()
        torch.cuda.synchronize()
        profiled_elapsed = time.perf_counter() - p0
        prof = ctx.profile_report()
        ctx.profile(False)
        depth = out.cpu().numpy()
        ctx.close()

        # The other precision / attention modes on the same model and input:
        # short runs, reported beside the int8 headline (FORCE_FP32, FORCE_FP16,
        # and the int8 graph with the reference's materialised binary16
        # attention, REFERENCE_FP16_ATTENTION).
        def mode_rate(flags, steps):
            with pkg.Context(str(model), args.encoder, flags) as cm:
                def stepm():
                    cm.infer_device(x.data_ptr(), 1, args.size, args.size, out.data_ptr(), n_out, stream)

                for _ in range(2):
                    stepm()
                torch.cuda.synchronize()
                f0 = time.perf_counter()
                for _ in range(steps):
                    stepm()
                torch.cuda.synchronize()
                return steps / (time.perf_counter() - f0)

        def host_entry_median(flags, calls_n):
            with pkg.Context(str(model), args.encoder, flags) as cm:
                cm.infer(x_host, args.size, args.size)
                ts = []
                for _ in range(calls_n):
                    h0 = time.perf_counter()
                    cm.infer(x_host, args.size, args.size)
                    ts.append(time.perf_counter() - h0)
            return {"calls": calls_n, "median_ms": 1e3 * float(np.median(ts)),
                    "images_per_s_median": 1.0 / float(np.median(ts))}

        fp32_rate = fp16_rate = ref16_rate = coop_rate = None
        ref16_host = coop_host = None
        if args.batch == 1 and not args.no_fp32_mode:
            fp32_rate = mode_rate(pkg.FORCE_FP32, 5)
            fp16_rate = mode_rate(pkg.FORCE_FP16, 5)
            ref16_rate = mode_rate(pkg.REFERENCE_FP16_ATTENTION, 10)
            ref16_host = host_entry_median(pkg.REFERENCE_FP16_ATTENTION, 20)
            ref16_host["entry"] = ("dav2_infer_tensor_f32, int8 graph with the reference's binary16 attention "
                                   "arithmetic (DAV2_CREATE_REFERENCE_FP16_ATTENTION)")
            print("bench: reference-arithmetic attention " + json.dumps(ref16_host), file=sys.stderr, flush=True)
            coop_rate = mode_rate(pkg.REFERENCE_FP16_COOP_ATTENTION, 10)
            coop_host = host_entry_median(pkg.REFERENCE_FP16_COOP_ATTENTION, 20)
            coop_host["entry"] = ("dav2_infer_tensor_f32, int8 graph with the reference's binary16 attention as on "
                                  "cooperative-matrix devices: bmm_score_coop_fp16 scores on the f16 MFMA "
                                  "(DAV2_CREATE_REFERENCE_FP16_COOP_ATTENTION)")
            print("bench: cooperative-matrix reference attention " + json.dumps(coop_host), file=sys.stderr,
                  flush=True)

        gemm = prof.get("gemm_i8", {})
        g_ms = gemm.get("ms", 0.0)
        g_launches = max(1, gemm.get("launches", 1))
        achieved = gemm.get("work", 0.0) / (g_ms * 1e-3) / 1e12 if g_ms else 0.0
        traffic = None
        tfile = ROOT / "profiles" / "gemm_i8_traffic.json"
        if tfile.exists():
            try:
                t = json.loads(tfile.read_text())
                key = f"{args.encoder}_{args.size}_b{args.batch}"
                traffic = t.get(key, {}).get("bytes_per_launch")
            except (ValueError, OSError):
                traffic = None
        kernels = {}
        gemm_shapes = gemm_shape_table(prof, args.steps)
        for name, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"]):
            if "@" in name:
                continue
            rate = v["work"] / (v["ms"] * 1e-3) if v["ms"] else 0.0
            if v["unit"] == "B":
                kernels[name] = {"ms_per_step": v["ms"] / args.steps, "avg_us": 1e3 * v["ms"] / v["launches"],
                                 "GB/s": rate / 1e9, "frac_hbm": rate / 1e9 / PEAK_HBM_GBS}
            else:
                kernels[name] = {"ms_per_step": v["ms"] / args.steps, "avg_us": 1e3 * v["ms"] / v["launches"],
                                 "T/s": rate / 1e12}
        if args.profile_json:
            Path(args.profile_json).write_text(json.dumps({"raw": prof, "kernels": kernels}, indent=1))
        print("bench: per-kernel " + json.dumps(kernels), file=sys.stderr, flush=True)

        # Further configurations of the same model family, a few profiled
        # steps each: the bandwidth-bound kernels (LayerNorm + quantize,
        # materialised softmax of the fp32-attention path) and the GEMM at
        # batch 8 and at 1036x1036 batch 4.
        extra = None
        if not args.no_extra and args.encoder == "vitl" and args.size == 518 and args.batch == 1:
            extra = {}
            for size, batch, fp32_att in ((518, 8, False), (1036, 4, False), (518, 8, True), (1036, 4, True)):
                key = f"vitl_{size}_b{batch}" + ("_fp32_attention" if fp32_att else "")
                extra[key] = profile_config(pkg, fmt, torch, model, size, batch, fp32_att, steps=3)
                print(f"bench: extra {key} " + json.dumps(extra[key]), file=sys.stderr, flush=True)

        cpu = None
        if not args.no_cpu_baseline:
            cpu = cpu_baseline(model, args.encoder, args.size, args.cpu_budget)
            if image_paths is not None:
                cpu["preprocess_bgr8_1080p_ms"] = cpu_preprocess_ms(1920, 1080, 518)

    ms = 1e3 * median_s
    result = {
        "metric": "images/sec ViT-L 518² bs1 on 1 MI355X; int8 GEMM % MFMA peak; LN/softmax % HBM",
        "value": args.batch / median_s,
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded random-init weights in a .dav2 file, seeded ImageNet-normalised input)",
        "config": {"workload": f"{args.encoder} + DPT {args.size}x{args.size} batch {args.batch}, int8 GEMMs and "
                               f"convolutions, {'fp32' if args.fp32_attention else 'integer-exact'} attention, "
                               + ("dav2_infer_tensor_f32 (host buffers)" if args.batch == 1
                                  else "dav2_infer_tensor_f32_device (batched)"),
                   "size": args.size, "global_batch": args.batch,
                   "parallelism": "single GPU"},
        "roofline": {"kernel": "gemm_i8", "bound": "mfma", "achieved": achieved, "peak": PEAK_INT8_TOPS,
                     "unit": "TFLOP/s", "work": "int8 ops, 2*M*N*K per GEMM",
                     "frac": achieved / PEAK_INT8_TOPS,
                     "avg_launch_us": 1e3 * g_ms / g_launches, "launches_per_step": g_launches / args.steps,
                     "traffic": traffic},
        "kernels": {k: kernels[k] for k in list(kernels)[:8]},
        "gemm_shapes": gemm_shapes,
        "profiled_ms_per_step": 1e3 * profiled_elapsed / args.steps,
        "host_entry": host_entry,
        "device_resident_images_per_s": device_rate,
        "device_median_images_per_s": device_median,
        "reference_arithmetic_host_entry": ref16_host,
        "reference_arithmetic_coop_host_entry": coop_host,
        "extra_configs": extra,
        "image_paths": image_paths,
        "fp32_mode_images_per_s": fp32_rate,
        "fp16_mode_images_per_s": fp16_rate,
        "reference_fp16_attention_images_per_s": ref16_rate,
        "reference_fp16_coop_attention_images_per_s": coop_rate,
        "depth_finite": bool(np.isfinite(depth).all()),
        "cpu_baseline": cpu,
    }
    print(json.dumps(result))
    return 0


if __name__ == "__main__":
    sys.exit(main())

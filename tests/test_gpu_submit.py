"""dav2_submit_hip, the HIP counterpart of the reference's zero-copy GPU
submission (src/vulkan_executor.cpp:656-800, job API src/dav2.cpp:429-473):
the float32 RGBA/BGRA preprocessing kernel (preprocess_rgba.glsl) bit for bit
against the oracle, and whole submissions against the oracle's pipeline
(preprocess, int8 graph, min/max normalisation, bilinear resize to the image).
The cross-process (IPC handle) form is tests/ipc_submit_check.py, which
starts its producer process before touching the GPU; the last test here runs
it as a child process."""

import ctypes as C
import subprocess
import sys
import time
from pathlib import Path

import numpy as np
import pytest

from gpu_util import dev, empty, host, ok, ptr, stream

pytestmark = pytest.mark.gpu

SEED = 0xDA20000


def _announce(*args):
    print("case:", *args, flush=True)


@pytest.mark.parametrize("width,height,input_size,pad,rgba", [(37, 23, 70, 0, True), (100, 61, 140, 5, False),
                                                              (640, 480, 518, 0, False), (333, 17, 56, 3, True),
                                                              (1920, 1080, 518, 16, False), (1, 9, 28, 0, True)])
def test_preprocess_rgba8_bit_exact(gpu, lib, oracle, width, height, input_size, pad, rgba):
    torch = gpu
    stride = width + pad  # pixels
    dw, dh = oracle.network_shape(width, height, input_size)
    _announce("preprocess_rgba8", width, height, stride, dw, dh, rgba)
    words = np.random.default_rng(width + height).integers(0, 2**32, size=height * stride, dtype=np.uint32)
    ref = oracle.preprocess_rgba8(words, width, height, stride, dw, dh, rgba)
    wd = dev(torch, words.view(np.int32))
    out = empty(torch, (3, dh, dw), torch.float32)
    ok(lib, lib.dav2_hip_preprocess_rgba8(ptr(wd), width, height, 4 * stride, dw, dh, int(rgba), ptr(out),
                                          stream(torch)))
    assert np.array_equal(host(torch, out).view(np.uint32), ref.view(np.uint32))


@pytest.fixture(scope="module")
def vits_model(pkg, tmp_path_factory):
    p = tmp_path_factory.mktemp("submit_models") / "vits.dav2"
    pkg.dav2_format.write_synthetic_model(p, "vits", seed=SEED + 1)
    return p


@pytest.fixture(scope="module")
def hip():
    h = C.CDLL("libamdhip64.so", mode=C.RTLD_GLOBAL)
    h.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    h.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
    h.hipEventDestroy.argtypes = [C.c_void_p]
    return h


def oracle_submit(oracle, model, words, width, height, stride, input_size, rgba):
    """vulkan_executor.cpp:694-787 on the CPU: preprocess, int8 graph,
    normalize_relative at the network size, bilinear to the image size."""
    nw, nh = oracle.network_shape(width, height, input_size)
    chw = oracle.preprocess_rgba8(words, width, height, stride, nw, nh, rgba)
    h = oracle.load_model(model, 0)
    try:
        depth, _, _ = oracle.infer(h, chw, nw, nh, attention="exact")
    finally:
        oracle.free_model(h)
    norm = oracle.normalize_relative(depth, oracle.reduce_minmax(depth))
    return oracle.bilinear(norm.reshape(1, nh, nw), width, height)[0]


def _request(pkg, width, height, stride_pixels, input_size, rgba, frame):
    r = pkg.HipSubmitRequest()
    r.struct_size, r.abi_version = C.sizeof(r), pkg.DAV2_ABI_VERSION
    r.width, r.height, r.row_stride_bytes = width, height, 4 * stride_pixels
    r.pixel_format = pkg.GPU_PIXEL_RGBA8 if rgba else pkg.GPU_PIXEL_BGRA8
    r.input_size, r.source_frame_id = input_size, frame
    return r


def _wait(pkg, lib, job, limit_s=60.0):
    st = pkg.GpuJobStatus()
    st.struct_size = C.sizeof(st)
    t0 = time.time()
    while True:
        assert lib.dav2_gpu_job_poll(job, C.byref(st)) == 0
        if st.state not in (pkg.GPU_JOB_QUEUED, pkg.GPU_JOB_RUNNING) or time.time() - t0 > limit_s:
            return st
        time.sleep(0.002)


@pytest.mark.parametrize("width,height,input_size,pad,rgba", [(300, 200, 140, 0, False), (97, 131, 112, 3, True)])
def test_submit_hip_matches_oracle(gpu, pkg, lib, oracle, hip, vits_model, width, height, input_size, pad, rgba):
    torch = gpu
    _announce("submit_hip", width, height, input_size, pad, rgba)
    stride = width + pad
    words = np.random.default_rng(width * 3 + height).integers(0, 2**32, size=height * stride, dtype=np.uint32)
    want = oracle_submit(oracle, vits_model, words, width, height, stride, input_size, rgba)
    with pkg.Context(str(vits_model), "vits") as ctx:
        src = torch.from_numpy(words.view(np.int32)).to("cuda")  # on torch's stream; the job waits for its event
        ev = C.c_void_p()
        assert hip.hipEventCreate(C.byref(ev)) == 0
        assert hip.hipEventRecord(ev, C.c_void_p(stream(torch))) == 0
        out = torch.full((height, width), float("nan"), device="cuda")
        torch.cuda.synchronize()
        r = _request(pkg, width, height, stride, input_size, rgba, frame=77)
        r.input, r.input_byte_size = ptr(src), 4 * words.size
        r.output, r.output_byte_size, r.wait_event = ptr(out), 4 * out.numel(), ev
        job = C.c_void_p()
        assert lib.dav2_submit_hip(ctx.handle, C.byref(r), C.byref(job)) == 0, lib.dav2_last_error()
        st = _wait(pkg, lib, job)
        assert st.state == pkg.GPU_JOB_COMPLETE and st.output_count == 1 and st.source_frame_id == 77
        assert lib.dav2_gpu_job_cancel(job) == 10  # INVALID_STATE: already complete
        lib.dav2_gpu_job_release(job)
        hip.hipEventDestroy(ev)
        got = host(torch, out)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_submit_hip_in_flight_polls_running(gpu, pkg, lib, hip, vits_model):
    """vulkan_executor.cpp:450-457: a job whose GPU work has not finished
    polls as RUNNING. The job waits for an event recorded behind a bounded
    spin kernel (torch.cuda._sleep) on torch's stream."""
    torch = gpu
    width, height = 64, 48
    _announce("submit_hip running", width, height)
    src = torch.zeros(width * height, dtype=torch.int32, device="cuda")
    out = torch.zeros(width * height, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    with pkg.Context(str(vits_model), "vits") as ctx:
        r = _request(pkg, width, height, width, 56, False, frame=9)
        r.input, r.input_byte_size, r.output, r.output_byte_size = ptr(src), 4 * src.numel(), ptr(out), \
            4 * out.numel()
        job = C.c_void_p()
        # a first submission sizes the context's workspaces
        assert lib.dav2_submit_hip(ctx.handle, C.byref(r), C.byref(job)) == 0, lib.dav2_last_error()
        assert _wait(pkg, lib, job).state == pkg.GPU_JOB_COMPLETE
        lib.dav2_gpu_job_release(job)
        ev = C.c_void_p()
        assert hip.hipEventCreate(C.byref(ev)) == 0
        torch.cuda._sleep(200_000_000)  # bounded spin: 0.1-2 s depending on the counter's clock
        assert hip.hipEventRecord(ev, C.c_void_p(stream(torch))) == 0
        r.wait_event = ev
        assert lib.dav2_submit_hip(ctx.handle, C.byref(r), C.byref(job)) == 0, lib.dav2_last_error()
        st = pkg.GpuJobStatus()
        st.struct_size = C.sizeof(st)
        assert lib.dav2_gpu_job_poll(job, C.byref(st)) == 0
        assert st.state == pkg.GPU_JOB_RUNNING
        done = _wait(pkg, lib, job)
        assert done.state == pkg.GPU_JOB_COMPLETE
        lib.dav2_gpu_job_release(job)
        hip.hipEventDestroy(ev)
        torch.cuda.synchronize()


def test_submit_hip_cancel_and_checks(gpu, pkg, lib, vits_model):
    torch = gpu
    width, height = 64, 48
    src = torch.zeros(width * height, dtype=torch.int32, device="cuda")
    out = torch.zeros(width * height, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    with pkg.Context(str(vits_model), "vits") as ctx:
        def submit(**fields):
            r = _request(pkg, width, height, width, 56, False, frame=5)
            r.input, r.input_byte_size, r.output, r.output_byte_size = ptr(src), 4 * src.numel(), ptr(out), \
                4 * out.numel()
            for k, v in fields.items():
                setattr(r, k, v)
            job = C.c_void_p()
            return lib.dav2_submit_hip(ctx.handle, C.byref(r), C.byref(job)), job
        st, job = submit()
        assert st == 0
        rc = lib.dav2_gpu_job_cancel(job)
        status = _wait(pkg, lib, job)
        if rc == 0:
            assert status.state == pkg.GPU_JOB_CANCELLED and status.output_count == 0
        else:
            assert rc == 10 and status.state == pkg.GPU_JOB_COMPLETE
        lib.dav2_gpu_job_release(job)
        assert submit(row_stride_bytes=4 * width - 4)[0] == 1       # stride shorter than a row
        assert submit(row_stride_bytes=4 * width + 2)[0] == 1       # not a multiple of 4
        assert submit(pixel_format=3)[0] == 1                       # DEPTH_FLOAT32 is no input format
        assert submit(input_byte_size=4 * src.numel() - 4)[0] == 1  # rows exceed the buffer
        assert submit(output_byte_size=4 * out.numel() - 4)[0] == 7  # BUFFER_TOO_SMALL
        assert submit(input_size=0)[0] == 1
        assert submit(flags=2)[0] == 1
        assert submit(struct_size=8)[0] == 1
        assert lib.dav2_submit_hip(None, None, None) == 1
        assert lib.dav2_gpu_job_poll(None, None) == 1


def test_ipc_submit_cross_process():
    # Producer and consumer in processes of their own (memory handles over
    # IPC, the wait event over IPC where the runtime records interprocess
    # events); the submission's output must equal the oracle's pipeline.
    script = Path(__file__).resolve().parent / "ipc_submit_check.py"
    r = subprocess.run([sys.executable, "-u", str(script)], capture_output=True, text=True, timeout=100)
    print(r.stdout[-2000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0
    assert "ipc submit bit-exact vs oracle: True" in r.stdout

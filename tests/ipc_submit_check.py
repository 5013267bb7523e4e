"""Cross-process check of dav2_submit_hip (run directly, not collected by
pytest): a producer process allocates the BGRA input and the depth output
with hipMalloc, records an interprocess event and passes the IPC handles to
this process, which submits through them (input = output = NULL) and
releases the job; the producer then reads the output back. The result must
equal the oracle's pipeline bit for bit. The producer synchronises its
uploads before publishing the memory handles; a submission that asks to wait
on an interprocess event (DAV2_HIP_SUBMIT_WAIT_EVENT_IPC) must be refused
with DAV2_STATUS_UNSUPPORTED (the runtime refused hipEventRecord of an
interprocess event on the MI355X it was tried on, so that form is not
offered).

The producer is started before this process makes any HIP call, so no
process that has initialised the GPU starts another program.

    python3 tests/ipc_submit_check.py          # exit status 0 on success
"""

import ctypes as C
import json
import os
import subprocess
import sys
import tempfile

import numpy as np

W, H, STRIDE, INPUT_SIZE, SEED = 180, 120, 184, 112, 0xDA20000


def producer(out_path: str) -> int:
    hip = C.CDLL("libamdhip64.so")
    words = np.random.default_rng(SEED).integers(0, 2**32, size=H * STRIDE, dtype=np.uint32)
    pin, pout = C.c_void_p(), C.c_void_p()
    out_bytes = 4 * W * H
    assert hip.hipMalloc(C.byref(pin), C.c_size_t(words.nbytes)) == 0
    assert hip.hipMalloc(C.byref(pout), C.c_size_t(out_bytes)) == 0
    assert hip.hipMemcpy(pin, C.c_void_p(words.ctypes.data), C.c_size_t(words.nbytes), 1) == 0
    assert hip.hipMemset(pout, 0, C.c_size_t(out_bytes)) == 0
    h_in, h_out = (C.c_uint8 * 64)(), (C.c_uint8 * 64)()
    assert hip.hipIpcGetMemHandle(h_in, pin) == 0
    assert hip.hipIpcGetMemHandle(h_out, pout) == 0
    # The uploads are complete (synchronised) before the handles are published.
    assert hip.hipDeviceSynchronize() == 0
    print(json.dumps({"in": bytes(h_in).hex(), "out": bytes(h_out).hex(), "bytes": words.nbytes}), flush=True)
    line = sys.stdin.readline()  # the consumer has released its job (or gave up)
    rc = 1
    if line.strip() == "done":
        host = np.empty(W * H, np.float32)
        assert hip.hipMemcpy(C.c_void_p(host.ctypes.data), pout, C.c_size_t(out_bytes), 2) == 0
        np.save(out_path, host)
        rc = 0
    print("saved" if rc == 0 else "skipped", flush=True)
    hip.hipFree(pin)
    hip.hipFree(pout)
    return rc


def consumer() -> int:
    here = os.path.dirname(os.path.abspath(__file__))
    tmp = tempfile.mkdtemp(prefix="dav2_ipc_")
    out_path = os.path.join(tmp, "depth.npy")
    child = subprocess.Popen([sys.executable, "-u", os.path.abspath(__file__), "producer", out_path],
                             stdin=subprocess.PIPE, stdout=subprocess.PIPE, text=True)
    try:
        handles = json.loads(child.stdout.readline())
        sys.path.insert(0, here)
        from conftest import load_package
        from oracle_py import Oracle
        from test_gpu_submit import oracle_submit

        pkg = load_package()
        lib = pkg.load()
        model = os.path.join(tmp, "vits.dav2")
        pkg.dav2_format.write_synthetic_model(model, "vits", seed=SEED + 1)
        with pkg.Context(model, "vits") as ctx:
            r = pkg.HipSubmitRequest()
            r.struct_size, r.abi_version = C.sizeof(r), pkg.DAV2_ABI_VERSION
            r.width, r.height, r.row_stride_bytes, r.pixel_format = W, H, 4 * STRIDE, pkg.GPU_PIXEL_BGRA8
            r.input_size = INPUT_SIZE
            r.input_byte_size, r.output_byte_size = handles["bytes"], 4 * W * H
            for field, key in (("input_ipc", "in"), ("output_ipc", "out")):
                C.memmove(getattr(r, field), bytes.fromhex(handles[key]), 64)
            job = C.c_void_p()
            # A wait on another process's event is refused before anything runs.
            r.flags = pkg.HIP_SUBMIT_WAIT_EVENT_IPC
            st = lib.dav2_submit_hip(ctx.handle, C.byref(r), C.byref(job))
            print("interprocess wait event status", st, (lib.dav2_last_error() or b"").decode(), flush=True)
            if st != 8 or job.value is not None:  # DAV2_STATUS_UNSUPPORTED
                return 1
            r.flags = 0
            st = lib.dav2_submit_hip(ctx.handle, C.byref(r), C.byref(job))
            print("submit status", st, (lib.dav2_last_error() or b"").decode(), flush=True)
            if st != 0:
                return 1
            lib.dav2_gpu_job_release(job)  # waits for the GPU work, closes the mappings
        child.stdin.write("done\n")
        child.stdin.flush()
        if child.stdout.readline().strip() != "saved":
            return 1
        got = np.load(out_path).reshape(H, W)
        words = np.random.default_rng(SEED).integers(0, 2**32, size=H * STRIDE, dtype=np.uint32)
        want = oracle_submit(Oracle(), model, words, W, H, STRIDE, INPUT_SIZE, False)
        same = bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
        print("ipc submit bit-exact vs oracle:", same, flush=True)
        return 0 if same else 1
    finally:
        if child.stdin and not child.stdin.closed:
            child.stdin.close()
        try:
            child.wait(timeout=60)
        except subprocess.TimeoutExpired:
            child.kill()


if __name__ == "__main__":
    sys.exit(producer(sys.argv[2]) if len(sys.argv) > 1 and sys.argv[1] == "producer" else consumer())

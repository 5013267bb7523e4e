"""Device-memory plumbing for the GPU tests: torch tensors hold the buffers,
the C ABI does the work."""

from __future__ import annotations

import numpy as np


def dev(torch, a: np.ndarray):
    # complete before any other stream (a context's or operator set's own)
    # reads it
    t = torch.from_numpy(np.ascontiguousarray(a)).to("cuda")
    torch.cuda.current_stream().synchronize()
    return t


def empty(torch, shape, dtype):
    return torch.empty(shape, dtype=dtype, device="cuda")


def ptr(t) -> int:
    return t.data_ptr()


def stream(torch) -> int:
    return torch.cuda.current_stream().cuda_stream


def host(torch, t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def ok(lib, rc: int) -> None:
    if rc != 0:
        raise AssertionError(f"HIP launcher returned {rc}: {lib.dav2_hip_error_string(rc).decode()}")


def db(pkg, t, nbytes: int | None = None):
    """dav2_device_buffer view of a torch tensor."""
    if t is None:
        return pkg.DeviceBuffer(None, 0)
    return pkg.DeviceBuffer(t.data_ptr(), nbytes if nbytes is not None else t.numel() * t.element_size())

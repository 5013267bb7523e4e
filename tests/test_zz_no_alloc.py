"""dav2_ops_linear_int8_noalloc, the allocation-free variant of
dav2_ops_linear_int8 (no reference counterpart): through the C ABI, bit for
bit against dav2_ops_linear_int8 on the same inputs, on calls in a row that
shrink (so the second call reuses the scratch the first one filled), with and
without the padded-weight part, with the transposed weight layout, through
two instances whose calls are queued back to back on their own streams, and
the size limit's error."""

import ctypes as C

import numpy as np
import pytest

from gpu_util import db, dev, empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(gpu, lib):
    h = lib.dav2_ops_create(0)
    assert h, lib.dav2_ops_last_error()
    yield h
    lib.dav2_ops_destroy(h)


def _case(torch, oracle, rows, ic, oc, seed, transposed=False):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, ic)) * rng.uniform(0.1, 4, (rows, 1))).astype(np.float32)
    w = (rng.standard_normal((oc, ic)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(oc) * 0.01).astype(np.float32)
    q, s = oracle.quantize_weight_rows(w)  # reference layout: [oc][ic] bytes
    return [dev(torch, a) for a in (x, np.ascontiguousarray(q.T if transposed else q), s, b)]


def _launch(pkg, lib, ops, fn, torch, held, rows, ic, oc, gelu, transposed=False):
    out = empty(torch, (rows, oc), torch.float32)
    out.fill_(float("nan"))
    torch.cuda.current_stream().synchronize()  # the fill lands before the instance's stream writes
    rc = fn(ops, db(pkg, out), *[db(pkg, t) for t in held], rows, ic, oc, int(gelu), int(transposed))
    assert rc == 0, lib.dav2_ops_last_error().decode()
    return out


def _run(pkg, lib, ops, fn, torch, held, rows, ic, oc, gelu, transposed=False):
    out = _launch(pkg, lib, ops, fn, torch, held, rows, ic, oc, gelu, transposed)
    assert lib.dav2_ops_synchronize(ops) == 0
    return host(torch, out)


@pytest.mark.parametrize("first,second", [((1370, 1024, 3072, False), (300, 588, 384, True)),
                                          ((2048, 4096, 1024, True), (77, 4096, 1024, False)),
                                          ((5000, 432, 96, False), (1369, 1024, 256, True))])
def test_noalloc_matches_linear_int8_twice(gpu, pkg, lib, oracle, ops, first, second):
    torch = gpu
    for i, (rows, ic, oc, gelu) in enumerate((first, second)):
        print("case: linear_int8_noalloc", i, rows, ic, oc, gelu, flush=True)
        held = _case(torch, oracle, rows, ic, oc, seed=rows + ic + oc)
        want = _run(pkg, lib, ops, lib.dav2_ops_linear_int8, torch, held, rows, ic, oc, gelu)
        got = _run(pkg, lib, ops, lib.dav2_ops_linear_int8_noalloc, torch, held, rows, ic, oc, gelu)
        assert np.isfinite(want).all()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_transposed_weight_matches_linear_int8(gpu, pkg, lib, oracle, ops):
    # the reference's [K][N] int8_transposed_buffer, transposed into the scratch
    torch = gpu
    for rows, ic, oc, gelu in ((1370, 1024, 3072, True), (200, 588, 96, False)):
        print("case: linear_int8_noalloc transposed", rows, ic, oc, gelu, flush=True)
        held = _case(torch, oracle, rows, ic, oc, seed=rows + 3 * oc, transposed=True)
        want = _run(pkg, lib, ops, lib.dav2_ops_linear_int8, torch, held, rows, ic, oc, gelu, True)
        got = _run(pkg, lib, ops, lib.dav2_ops_linear_int8_noalloc, torch, held, rows, ic, oc, gelu, True)
        assert np.isfinite(want).all()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_two_instances_back_to_back(gpu, pkg, lib, oracle, ops):
    # Two instances (two streams) share the GPU's scratch; their calls are
    # queued without a synchronisation in between, so each must wait for the
    # previous one. Every output equals its own dav2_ops_linear_int8 result.
    torch = gpu
    other = lib.dav2_ops_create(0)
    assert other, lib.dav2_ops_last_error()
    try:
        shapes = [(2000, 1024, 1024, False), (1500, 1024, 3072, True), (2000, 4096, 512, False),
                  (900, 588, 384, True)]
        cases = [_case(torch, oracle, r, i, o, seed=11 + n) for n, (r, i, o, _) in enumerate(shapes)]
        torch.cuda.synchronize()
        outs = []
        for n, ((rows, ic, oc, gelu), held) in enumerate(zip(shapes, cases)):
            inst = ops if n % 2 == 0 else other
            outs.append(_launch(pkg, lib, inst, lib.dav2_ops_linear_int8_noalloc, torch, held, rows, ic, oc, gelu))
        assert lib.dav2_ops_synchronize(ops) == 0 and lib.dav2_ops_synchronize(other) == 0
        for (rows, ic, oc, gelu), held, out in zip(shapes, cases, outs):
            print("case: two instances", rows, ic, oc, gelu, flush=True)
            want = _run(pkg, lib, ops, lib.dav2_ops_linear_int8, torch, held, rows, ic, oc, gelu)
            assert np.array_equal(host(torch, out).view(np.uint32), want.view(np.uint32))
    finally:
        lib.dav2_ops_destroy(other)


def test_noalloc_allocates_nothing(gpu, pkg, lib, oracle, ops):
    # free device memory is unchanged across calls of a size the growing
    # workspace of a fresh instance would have had to allocate for
    torch = gpu
    hip = C.CDLL("libamdhip64.so")
    free, total = C.c_size_t(), C.c_size_t()
    rows, ic, oc = 4000, 1000, 512  # ic % 64 != 0: the padded weight too
    held = _case(torch, oracle, rows, ic, oc, seed=5)
    torch.cuda.synchronize()
    fresh = lib.dav2_ops_create(0)
    try:
        assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
        before = free.value
        for _ in range(3):
            _run(pkg, lib, fresh, lib.dav2_ops_linear_int8_noalloc, torch, held, rows, ic, oc, False)
        assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
        assert free.value == before
    finally:
        lib.dav2_ops_destroy(fresh)


def test_noalloc_rejects_sizes_beyond_the_scratch(gpu, pkg, lib, oracle, ops):
    torch = gpu
    rows, ic, oc = 40000, 1024, 64  # 40000 x 1024 bytes > 32 MiB
    x = empty(torch, (rows, ic), torch.float32)
    w = empty(torch, (oc, ic), torch.int8)
    s = empty(torch, (oc,), torch.float32)
    out = empty(torch, (rows, oc), torch.float32)
    rc = lib.dav2_ops_linear_int8_noalloc(ops, db(pkg, out), db(pkg, x), db(pkg, w), db(pkg, s), db(pkg, s), rows, ic,
                                          oc, 0, 0)
    assert rc == 1
    assert "32 MiB" in lib.dav2_ops_last_error().decode()

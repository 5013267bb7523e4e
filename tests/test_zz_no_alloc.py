"""dav2_ops_linear_int8_noalloc, the allocation-free variant of
dav2_ops_linear_int8 (no reference counterpart): through the C ABI, bit for
bit against dav2_ops_linear_int8 on the same inputs, on calls in a row that
shrink (so the second call reuses the scratch the first one filled), with and
without the padded-weight part, and the size limit's error."""

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


def _case(torch, oracle, rows, ic, oc, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, ic)) * rng.uniform(0.1, 4, (rows, 1))).astype(np.float32)
    w = (rng.standard_normal((oc, ic)) * 0.02).astype(np.float32)
    b = (rng.standard_normal(oc) * 0.01).astype(np.float32)
    q, s = oracle.quantize_weight_rows(w)  # reference layout: [oc][ic] bytes
    return [dev(torch, a) for a in (x, np.ascontiguousarray(q), s, b)]


def _run(pkg, lib, ops, fn, torch, held, rows, ic, oc, gelu):
    out = empty(torch, (rows, oc), torch.float32)
    out.fill_(float("nan"))
    rc = fn(ops, db(pkg, out), *[db(pkg, t) for t in held], rows, ic, oc, int(gelu))
    assert rc == 0, lib.dav2_ops_last_error().decode()
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
                                          oc, 0)
    assert rc == 1
    assert "32 MiB" in lib.dav2_ops_last_error().decode()

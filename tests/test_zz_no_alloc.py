"""kd_reduce_noalloc (the allocation-free variant of kd_reduce) against kd_reduce itself.

The variant runs the same kernels; only the split path's segment partials live in a static
device buffer instead of the growable workspace. So every result must equal kd_reduce's bit for
bit. Each case makes two calls in a row through the C ABI, the second with a smaller input (the
buffer keeps the first call's partials: the second must not read them), on the split path (few
long rows) and on the paths that use no scratch.
"""
import numpy as np
import pytest

import kd

pytestmark = pytest.mark.gpu

# (rows, chunk) pairs: the first call, then the smaller second call.
SPLIT = [((1, 1 << 24), (1, 1 << 20)), ((3, 200000), (2, 70000)), ((500, 16384), (7, 30000))]
NO_SCRATCH = [((4096, 4096), (64, 300))]


def values(rng, dtype, n):
    if dtype == kd.BOOL:
        return (rng.random(n) < 0.999).astype(np.uint8)
    if dtype == kd.I64:
        return rng.integers(-(2**40), 2**40, n).astype(np.int64)
    x = rng.uniform(-1, 1, n).astype(kd.NUMPY_DTYPE[dtype])
    x[rng.integers(0, n)] = 3.5  # a unique maximum somewhere inside
    return x


def out_dtype(op, dtype):
    if op in (kd.REDUCE_SUM, kd.REDUCE_PROD) and dtype in (kd.I64, kd.BOOL):
        return np.int64
    if op in (kd.REDUCE_ALL, kd.REDUCE_ANY):
        return np.uint8
    return kd.NUMPY_DTYPE[dtype]


def run(kdb, fn, op, dtype, dx, rows, chunk):
    out = kdb.empty((rows,), out_dtype(op, dtype))
    kdb.check(getattr(kdb.lib, fn)(op, 0, dtype, out.ptr, dx.ptr, chunk, rows), fn)
    return out.numpy()


CASES = [(kd.REDUCE_SUM, kd.F32), (kd.REDUCE_MAX, kd.F32), (kd.REDUCE_MIN, kd.F64), (kd.REDUCE_SUM, kd.I64),
         (kd.REDUCE_PROD, kd.F64), (kd.REDUCE_ALL, kd.BOOL), (kd.REDUCE_ANY, kd.BOOL), (kd.REDUCE_SUM, kd.BOOL)]


@pytest.mark.parametrize("op,dtype", CASES, ids=[f"op{o}-dt{d}" for o, d in CASES])
@pytest.mark.parametrize("shapes", SPLIT + NO_SCRATCH, ids=lambda s: f"{s[0][0]}x{s[0][1]}-then-{s[1][0]}x{s[1][1]}")
def test_noalloc_equals_kd_reduce(kdb, op, dtype, shapes):
    rng = np.random.default_rng(hash((op, dtype, shapes)) % (1 << 32))
    for rows, chunk in shapes:
        x = values(rng, dtype, rows * chunk)
        if op == kd.REDUCE_PROD:
            x = (1.0 + x * 1e-6).astype(x.dtype)  # products of long rows stay finite
        dx = kdb.to_device(x)
        got = run(kdb, "kd_reduce_noalloc", op, dtype, dx, rows, chunk)
        want = run(kdb, "kd_reduce", op, dtype, dx, rows, chunk)
        np.testing.assert_array_equal(got, want)


def test_noalloc_edge_cases(kdb):
    dx = kdb.to_device(np.ones(8, np.float32))
    out = kdb.empty((1,), np.float32)
    assert kdb.lib.kd_reduce_noalloc(kd.REDUCE_SUM, 0, kd.F32, out.ptr, dx.ptr, 8, 0) == 0  # no output: no-op
    assert kdb.lib.kd_reduce_noalloc(kd.REDUCE_MAX, 0, kd.F32, out.ptr, dx.ptr, 0, 1) != 0  # max of nothing
    assert "empty chunk" in kdb.error()
    assert kdb.lib.kd_reduce_noalloc(kd.REDUCE_SUM, 0, kd.F32, out.ptr, dx.ptr, -1, 1) != 0
    assert kdb.lib.kd_reduce_noalloc(kd.REDUCE_SUM, 0, 9, out.ptr, dx.ptr, 8, 1) != 0
    # a sum of an empty chunk is zero, as kd_reduce gives it
    kdb.check(kdb.lib.kd_reduce_noalloc(kd.REDUCE_SUM, 0, kd.F32, out.ptr, dx.ptr, 0, 1), "noalloc")
    assert out.numpy()[0] == 0.0

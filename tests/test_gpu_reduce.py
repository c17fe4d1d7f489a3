"""kd_reduce against the C oracle (which restates reference src/cuda/kernels.inl:59-134, 278-307).

Covers each kernel path (grouped short rows, one workgroup per row, split long rows), every
dtype, NaN/inf rows (tests/test_cuda.cpp:287-300), long deterministic sums (:302-311), empty
inputs (:313-320) and the C2 config at full size (sum over dim 1 and global max of a[4096,4096]).
f32 sums accumulate in double on both sides, so they are expected bit-exact; f64 sums may differ
in the last bits from the different summation order (tolerance 1e-12 relative to sum |x|).
"""
import numpy as np
import pytest

import kd
import support

pytestmark = pytest.mark.gpu

SHAPES = [(1, 1), (3, 7), (600, 64), (5, 300), (2, 512), (700, 513), (4, 4096), (3, 5000), (2, 100000),
          (1, 1 << 20), (4096, 4096)]


def oracle_reduce(oracle, op, dtype, x, rows, chunk):
    out_np = np.int64 if (op == kd.REDUCE_SUM and dtype in (kd.I64, kd.BOOL)) else kd.NUMPY_DTYPE[dtype]
    out = np.zeros(rows, out_np)
    assert oracle.oracle_reduce(op, 0, dtype, support.ptr(out), support.ptr(x), chunk, rows) == 0
    return out


def values(rng, dtype, n):
    npd = kd.NUMPY_DTYPE[dtype]
    if dtype == kd.BOOL:
        return rng.integers(0, 2, n).astype(np.uint8)
    if dtype == kd.I64:
        return rng.integers(-(2**62), 2**62, n).astype(np.int64)
    return rng.uniform(-1, 1, n).astype(npd)


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
@pytest.mark.parametrize("op", [kd.REDUCE_SUM, kd.REDUCE_MAX, kd.REDUCE_MIN], ids=["sum", "max", "min"])
@pytest.mark.parametrize("rows,chunk", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_reduce_matches_oracle(kdb, oracle, op, dtype, rows, chunk):
    if rows * chunk > (1 << 22) and dtype != kd.F32:
        pytest.skip("full-size shapes run for f32 only")
    rng = np.random.default_rng(rows * 31 + chunk + op * 7 + dtype)
    x = values(rng, dtype, rows * chunk)
    want = oracle_reduce(oracle, op, dtype, x, rows, chunk)
    dx = kdb.to_device(x)
    out = kdb.empty((rows,), want.dtype)
    kdb.call("reduce", op, 0, dtype, out.ptr, dx.ptr, chunk, rows)
    got = out.numpy()
    if dtype == kd.F64 and op == kd.REDUCE_SUM:
        scale = np.abs(x.reshape(rows, chunk)).sum(axis=1) + 1e-300
        assert np.all(np.abs(got - want) <= 1e-12 * scale)
    else:
        np.testing.assert_array_equal(got, want)


def test_non_finite_rows(kdb, oracle):
    x = np.array([1, np.inf, 2, -np.inf, 1, 2, np.nan, 1, 2, 0.0, -0.0, 0.0], np.float32)
    for op in (kd.REDUCE_SUM, kd.REDUCE_MAX, kd.REDUCE_MIN):
        want = oracle_reduce(oracle, op, kd.F32, x, 4, 3)
        dx = kdb.to_device(x)
        out = kdb.empty((4,), np.float32)
        kdb.call("reduce", op, 0, kd.F32, out.ptr, dx.ptr, 3, 4)
        got = out.numpy()
        assert np.array_equal(np.isnan(got), np.isnan(want))
        np.testing.assert_array_equal(got[~np.isnan(got)], want[~np.isnan(want)])


def test_long_sum_is_deterministic(kdb):
    rng = np.random.default_rng(5)
    x = rng.normal(size=200000).astype(np.float64)
    dx = kdb.to_device(x)
    outs = []
    for _ in range(3):
        out = kdb.empty((1,), np.float64)
        kdb.call("reduce", kd.REDUCE_SUM, 0, kd.F64, out.ptr, dx.ptr, x.size, 1)
        outs.append(out.numpy()[0])
    assert outs[0] == outs[1] == outs[2]
    assert abs(outs[0] - np.sum(x)) <= 1e-10 * np.abs(x).sum()


def test_integer_sum_wraps(kdb):
    x = np.array([2**63 - 1, 1], np.int64)
    dx = kdb.to_device(x)
    out = kdb.empty((1,), np.int64)
    kdb.call("reduce", kd.REDUCE_SUM, 0, kd.I64, out.ptr, dx.ptr, 2, 1)
    assert out.numpy()[0] == -(2**63)


def test_empty_chunks(kdb):
    out = kdb.to_device(np.full(3, 5.0, np.float32))
    kdb.call("reduce", kd.REDUCE_SUM, 0, kd.F32, out.ptr, out.ptr, 0, 3)
    np.testing.assert_array_equal(out.numpy(), [0, 0, 0])
    with pytest.raises(kd.KdError):
        kdb.call("reduce", kd.REDUCE_MAX, 0, kd.F32, out.ptr, out.ptr, 0, 3)


COLUMN_SHAPES = [(1, 1), (13, 7), (64, 3), (700, 513), (4096, 256), (4096, 768), (100000, 3), (3, 100000), (4097, 1)]


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
@pytest.mark.parametrize("op", [kd.REDUCE_SUM, kd.REDUCE_MAX, kd.REDUCE_MIN], ids=["sum", "max", "min"])
@pytest.mark.parametrize("outer,inner", COLUMN_SHAPES, ids=[f"{o}x{i}" for o, i in COLUMN_SHAPES])
def test_reduce_columns_matches_oracle(kdb, oracle, op, dtype, outer, inner):
    """kd_reduce_columns (leading dim of a contiguous [outer, inner] tensor, read in place) against
    oracle_reduce_columns, which the CPU suite pins bit for bit to the reference's reduce tasks over
    the transposed copy kael makes today. Same tolerance rule as kd_reduce."""
    rng = np.random.default_rng(outer * 17 + inner + op * 5 + dtype)
    x = values(rng, dtype, outer * inner)
    out_np = np.int64 if (op == kd.REDUCE_SUM and dtype in (kd.I64, kd.BOOL)) else kd.NUMPY_DTYPE[dtype]
    want = np.zeros(inner, out_np)
    assert oracle.oracle_reduce_columns(op, 0, dtype, support.ptr(want), support.ptr(x), outer, inner) == 0
    dx = kdb.to_device(x)
    out = kdb.empty((inner,), out_np)
    kdb.call("reduce_columns", op, 0, dtype, out.ptr, dx.ptr, outer, inner)
    got = out.numpy()
    if dtype == kd.F64 and op == kd.REDUCE_SUM:
        scale = np.abs(x.reshape(outer, inner)).sum(axis=0) + 1e-300
        assert np.all(np.abs(got - want) <= 1e-12 * scale)
    else:
        np.testing.assert_array_equal(got, want)


def test_reduce_columns_non_finite_and_empty(kdb, oracle):
    x = np.array([[1, np.inf, np.nan], [2, -np.inf, 0.0], [-0.0, 1, 3]], np.float32).ravel()
    for op in (kd.REDUCE_SUM, kd.REDUCE_MAX, kd.REDUCE_MIN):
        want = np.zeros(3, np.float32)
        assert oracle.oracle_reduce_columns(op, 0, kd.F32, support.ptr(want), support.ptr(x), 3, 3) == 0
        dx = kdb.to_device(x)
        out = kdb.empty((3,), np.float32)
        kdb.call("reduce_columns", op, 0, kd.F32, out.ptr, dx.ptr, 3, 3)
        got = out.numpy()
        assert np.array_equal(np.isnan(got), np.isnan(want)) and np.array_equal(got[~np.isnan(want)], want[~np.isnan(want)])
    out = kdb.empty((4,), np.float32)
    kdb.call("reduce_columns", kd.REDUCE_SUM, 0, kd.F32, out.ptr, None, 0, 4)  # no rows: sum identity
    np.testing.assert_array_equal(out.numpy(), np.zeros(4, np.float32))
    kdb.call("reduce_columns", kd.REDUCE_SUM, 0, kd.F32, None, None, 5, 0)  # no columns: nothing to write

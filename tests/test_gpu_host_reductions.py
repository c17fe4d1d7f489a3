"""kd_reduce PROD / ALL / ANY, kd_arg_reduce and kd_cumsum against the C oracle (itself pinned
to kael's CPU path in test_oracle_host_reductions.py).

Bit-exact: argmax / argmin (the first-extreme rule is order independent), all / any, integer
and bool prod and cumsum (wrapping int64 arithmetic is associative). Floating prod and cumsum
accumulate in double on the device in a different order than kael's host code: f32 results
within rtol 1e-6 (prod) and, for cumsum, within 1e-6 of the running sum of |x| plus one f32
ulp; f64 within 1e-12 of the same scales.
Shapes reach every launch path: groups of lanes per short row, a workgroup per row, rows split
across workgroups (reductions), one workgroup per row and segmented scans with 8 or 16 elements
per lane (cumsum).
"""
import numpy as np
import pytest

import kd
from support import ptr

pytestmark = pytest.mark.gpu

NP = {kd.F32: np.float32, kd.F64: np.float64, kd.I64: np.int64, kd.BOOL: np.bool_}
DTYPES = [kd.F32, kd.F64, kd.I64, kd.BOOL]
IDS = ["f32", "f64", "i64", "bool"]
REDUCE_SHAPES = [(1, 1), (3, 7), (1000, 100), (600, 3000), (3, 100000), (1, 2000003)]
# Includes many short rows ((513, 4), (520, 1000), (600, 2048)) and C2's (4096, 4096).
SCAN_SHAPES = [(1, 1), (3, 7), (700, 130), (2, 30000), (1, 70001), (2, 1000003), (3, 333333), (64, 4096),
               (3, 262144), (513, 4), (520, 1000), (600, 2048), (4096, 4096)]


def sample(dtype, shape, rng, kind):
    rows, cols = shape
    if dtype == kd.BOOL:
        return rng.random(shape) < (0.999 if kind == "all" else 0.001)
    if dtype == kd.I64:
        if kind in ("prod", "cumsum"):
            return rng.integers(-(2 ** 62), 2 ** 62, shape, dtype=np.int64)
        return rng.integers(-5, 6, shape, dtype=np.int64)
    x = rng.uniform(0.999, 1.001, shape) if kind == "prod" else rng.uniform(-1, 1, shape)
    x = x.astype(NP[dtype])
    if kind in ("argmax", "argmin") and cols > 10:
        x[0, cols - 3] = np.nan          # a NaN late in the row (another segment than the extreme)
        x[0, cols // 2] = np.nan
        ext = x[-1].max() if kind == "argmax" else x[-1].min()
        x[-1, cols - 1] = ext            # a tie at the end must lose to the earlier extreme
    if kind in ("all", "any") and cols > 2:
        x[:, cols // 2] = 0.0
        x[0, :] = 0.0
        if rows > 1:
            x[1, :] = -0.0
            x[1, cols - 1] = np.nan
    return x


def run(kdb, oracle, kind, dtype, x):
    rows, cols = x.shape
    xs = np.ascontiguousarray(x)
    dx = kdb.to_device(xs)
    if kind in ("argmax", "argmin"):
        out = kdb.empty((rows,), np.int64)
        kdb.call("arg_reduce", 1 if kind == "argmax" else 0, dtype, out.ptr, dx.ptr, cols, rows)
        want = np.zeros(rows, np.int64)
        assert oracle.oracle_arg_reduce(1 if kind == "argmax" else 0, dtype, ptr(want), ptr(xs), cols, rows) == 0
    elif kind == "cumsum":
        odt = NP[dtype] if dtype in (kd.F32, kd.F64) else np.int64
        out = kdb.empty((rows, cols), odt)
        kdb.call("cumsum", dtype, out.ptr, dx.ptr, cols, rows)
        want = np.zeros((rows, cols), odt)
        assert oracle.oracle_cumsum(dtype, ptr(want), ptr(xs), cols, rows) == 0
    else:
        op = {"prod": kd.REDUCE_PROD, "all": kd.REDUCE_ALL, "any": kd.REDUCE_ANY}[kind]
        odt = np.uint8 if kind != "prod" else (NP[dtype] if dtype in (kd.F32, kd.F64) else np.int64)
        out = kdb.empty((rows,), odt)
        kdb.call("reduce", op, 0, dtype, out.ptr, dx.ptr, cols, rows)
        want = np.zeros(rows, odt)
        assert oracle.oracle_reduce(op, 0, dtype, ptr(want), ptr(xs), cols, rows) == 0
    return out.numpy(), want


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("kind", ["argmax", "argmin", "all", "any"])
def test_order_free_reductions_are_bit_exact(kdb, oracle, kind, dtype):
    rng = np.random.default_rng(31 * dtype + len(kind))
    for shape in REDUCE_SHAPES:
        got, want = run(kdb, oracle, kind, dtype, sample(dtype, shape, rng, kind))
        np.testing.assert_array_equal(got, want, err_msg=f"{kind} {shape}")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_prod(kdb, oracle, dtype):
    rng = np.random.default_rng(5 + dtype)
    for shape in REDUCE_SHAPES:
        got, want = run(kdb, oracle, "prod", dtype, sample(dtype, shape, rng, "prod"))
        if dtype in (kd.I64, kd.BOOL):
            np.testing.assert_array_equal(got, want, err_msg=f"prod {shape}")
        else:
            np.testing.assert_allclose(got, want, rtol=1e-6 if dtype == kd.F32 else 1e-12, err_msg=f"prod {shape}")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_cumsum(kdb, oracle, dtype):
    rng = np.random.default_rng(11 + dtype)
    for shape in SCAN_SHAPES:
        x = sample(dtype, shape, rng, "cumsum")
        got, want = run(kdb, oracle, "cumsum", dtype, x)
        if dtype in (kd.I64, kd.BOOL):
            np.testing.assert_array_equal(got, want, err_msg=f"cumsum {shape}")
        else:
            # Both sides round a sum of the same terms; kael's sequential f32 (or f64) running sum
            # carries at most ~i ulps of the running |x| sum, the device's double sum less.
            scale = np.cumsum(np.abs(x.astype(np.float64)), axis=1)
            eps = np.finfo(NP[dtype]).eps
            bound = (1e-6 if dtype == kd.F32 else 1e-12) * scale + eps * np.abs(want.astype(np.float64))
            err = np.abs(got.astype(np.float64) - want.astype(np.float64))
            assert np.all(err <= bound), f"cumsum {shape}: worst excess {(err - bound).max()}"


def test_cumsum_float_matches_exact_prefix(kdb):
    """Small integers in f32: every prefix is exact in binary, so the device must be exact."""
    x = np.arange(1, 4097, dtype=np.float32).reshape(2, 2048) % 97
    dx = kdb.to_device(x)
    out = kdb.empty(x.shape, np.float32)
    kdb.call("cumsum", kd.F32, out.ptr, dx.ptr, 2048, 2)
    np.testing.assert_array_equal(out.numpy(), np.cumsum(x, axis=1))


def test_empty_and_errors(kdb):
    out = kdb.empty((2,), np.float32)
    x = kdb.empty((2, 1), np.float32)
    kdb.call("reduce", kd.REDUCE_PROD, 0, kd.F32, out.ptr, x.ptr, 0, 2)
    np.testing.assert_array_equal(out.numpy(), [1, 1])
    idx = kdb.empty((2,), np.int64)
    with pytest.raises(kd.KdError):
        kdb.call("arg_reduce", 1, kd.F32, idx.ptr, x.ptr, 0, 2)
    kdb.call("cumsum", kd.F32, out.ptr, x.ptr, 0, 2)  # nothing to do

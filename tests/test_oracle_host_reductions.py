"""Pins the oracle's prod / all / any / argmax / argmin / cumsum against kael's own CPU path.

kael computes these on the host (reference src/ops/reduce.cpp:202-219,236-268,285-295,
362-369,399-469; src/ops/sequence.cpp:95-117). The oracle restates those algorithms (the
8-lane, 16384-element-block, pairwise-merge order of prod included), so it must agree with
kael compiled from the reference sources bit for bit, floats included. numpy pins what does
not depend on rounding order: argmax / argmin (numpy also returns the first extreme and the
first NaN), all / any (NaN is truthy), integer prod and cumsum (both wrap modulo 2^64).
"""
import numpy as np
import pytest

import kd
from support import ptr, ref_error

WHAT = {"prod": 0, "all": 1, "any": 2, "argmax": 3, "argmin": 4, "cumsum": 5}
NP = {kd.F32: np.float32, kd.F64: np.float64, kd.I64: np.int64, kd.BOOL: np.bool_}
SHAPES = [(1, 1), (3, 7), (5, 8), (4, 9), (2, 16384 + 37), (1, 3 * 16384 + 5)]


def sample(dtype, shape, rng, kind):
    rows, cols = shape
    if dtype == kd.BOOL:
        return rng.random(shape) < (0.95 if kind == "all" else 0.05)
    if dtype == kd.I64:
        if kind in ("prod", "cumsum"):
            return rng.integers(-(2 ** 62), 2 ** 62, shape, dtype=np.int64)  # products and sums wrap
        return rng.integers(-5, 6, shape, dtype=np.int64)  # ties for argmax / argmin
    x = rng.uniform(0.95, 1.05, shape) if kind == "prod" else rng.uniform(-1, 1, shape)
    x = x.astype(NP[dtype])
    if kind in ("argmax", "argmin") and cols > 3:
        x[0, cols // 3] = np.nan
        x[0, 2 * cols // 3] = np.nan
        x[-1, 1] = x[-1, 2] = x[-1].max() if kind == "argmax" else x[-1].min()  # a tie
    if kind in ("all", "any") and cols > 2:
        x[:, 1] = 0.0
        x[0, :] = -0.0
        if rows > 1:
            x[1, :] = 0.0
            x[1, cols - 1] = np.nan
    if kind == "prod" and rows > 1 and cols > 4:
        x[1, cols // 2] = 0.0
    return x


def out_buffer(kind, dtype, rows, cols):
    if kind in ("argmax", "argmin"):
        return np.zeros(rows, np.int64)
    if kind in ("all", "any"):
        return np.zeros(rows, np.uint8)
    odt = NP[dtype] if dtype in (kd.F32, kd.F64) else np.int64
    return np.zeros((rows, cols) if kind == "cumsum" else rows, odt)


def run_oracle(oracle, kind, dtype, x):
    rows, cols = x.shape
    out = out_buffer(kind, dtype, rows, cols)
    xs = np.ascontiguousarray(x)
    if kind in ("argmax", "argmin"):
        rc = oracle.oracle_arg_reduce(1 if kind == "argmax" else 0, dtype, ptr(out), ptr(xs), cols, rows)
    elif kind == "cumsum":
        rc = oracle.oracle_cumsum(dtype, ptr(out), ptr(xs), cols, rows)
    else:
        op = {"prod": kd.REDUCE_PROD, "all": kd.REDUCE_ALL, "any": kd.REDUCE_ANY}[kind]
        rc = oracle.oracle_reduce(op, 0, dtype, ptr(out), ptr(xs), cols, rows)
    assert rc == 0, oracle.oracle_last_error()
    return out


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
@pytest.mark.parametrize("kind", list(WHAT))
def test_oracle_matches_kael_cpu(oracle, refdev, kind, dtype):
    rng = np.random.default_rng(100 * WHAT[kind] + dtype)
    for shape in SHAPES:
        x = sample(dtype, shape, rng, kind)
        want = out_buffer(kind, dtype, *shape)
        assert refdev.ref_host_reduce(WHAT[kind], dtype, ptr(want), ptr(np.ascontiguousarray(x)), *shape) == 0, \
            ref_error(refdev)
        got = run_oracle(oracle, kind, dtype, x)
        np.testing.assert_array_equal(got.view(np.uint8), want.view(np.uint8), err_msg=f"{kind} {shape}")


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
@pytest.mark.parametrize("kind", ["argmax", "argmin", "all", "any"])
def test_oracle_order_free_results_match_numpy(oracle, kind, dtype):
    rng = np.random.default_rng(7 * WHAT[kind] + dtype)
    for shape in SHAPES:
        x = sample(dtype, shape, rng, kind)
        got = run_oracle(oracle, kind, dtype, x)
        if kind == "argmax":
            want = np.argmax(x, axis=1)
        elif kind == "argmin":
            want = np.argmin(x, axis=1)
        elif kind == "all":
            want = np.all(x, axis=1)
        else:
            want = np.any(x, axis=1)
        np.testing.assert_array_equal(got, want.astype(got.dtype), err_msg=f"{kind} {shape}")


def test_oracle_integer_prod_and_cumsum_wrap_like_numpy(oracle):
    rng = np.random.default_rng(3)
    x = rng.integers(-(2 ** 62), 2 ** 62, (3, 20000), dtype=np.int64)
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(run_oracle(oracle, "prod", kd.I64, x), np.prod(x, axis=1))
        np.testing.assert_array_equal(run_oracle(oracle, "cumsum", kd.I64, x), np.cumsum(x, axis=1))
    b = rng.random((4, 999)) < 0.5
    np.testing.assert_array_equal(run_oracle(oracle, "cumsum", kd.BOOL, b), np.cumsum(b, axis=1))
    np.testing.assert_array_equal(run_oracle(oracle, "prod", kd.BOOL, b), np.prod(b, axis=1))


def test_oracle_float_cumsum_is_the_sequential_sum(oracle):
    """f32 cumsum accumulates in f32, one element after another: a prefix that is exact in
    binary (small integers) must come out exact, and the sequential f32 rounding is visible."""
    x = np.array([[2.0 ** 24, 1.0, 1.0, 1.0, 1.0]], np.float32)
    got = run_oracle(oracle, "cumsum", kd.F32, x)
    np.testing.assert_array_equal(got, [[2.0 ** 24] * 5])  # 2^24 + 1 rounds back to 2^24 each step
    y = np.arange(1, 2001, dtype=np.float32).reshape(1, -1)
    np.testing.assert_array_equal(run_oracle(oracle, "cumsum", kd.F32, y), np.cumsum(y, axis=1))


def test_oracle_empty_and_errors(oracle):
    out = np.zeros(2, np.float32)
    x = np.zeros((2, 0), np.float32)
    assert oracle.oracle_reduce(kd.REDUCE_PROD, 0, kd.F32, ptr(out), ptr(x), 0, 2) == 0
    np.testing.assert_array_equal(out, [1, 1])
    flags = np.full(2, 7, np.uint8)
    assert oracle.oracle_reduce(kd.REDUCE_ALL, 0, kd.F32, ptr(flags), ptr(x), 0, 2) == 0
    np.testing.assert_array_equal(flags, [1, 1])
    assert oracle.oracle_reduce(kd.REDUCE_ANY, 0, kd.F32, ptr(flags), ptr(x), 0, 2) == 0
    np.testing.assert_array_equal(flags, [0, 0])
    idx = np.zeros(2, np.int64)
    assert oracle.oracle_arg_reduce(1, kd.F32, ptr(idx), ptr(x), 0, 2) != 0

"""Randomised index layouts for kd_gather / kd_scatter_add against the C oracle (seeded).

Each case draws an iteration shape of rank 1-4 and an axis; the data tensor has that shape with
its own extent along the axis; data, index and scatter source tensors each get a random layout
(row-major, permuted, stepped), and the index tensor may broadcast (stride 0) along dims, as
index_select's does (reference src/ops/indexing.cpp:109-118). A gather's output is contiguous
in iteration order (reference src/cuda/kernels.inl:185-210). Gather is bit-exact in
every dtype; scatter_add is bit-exact for i64 (wrapping sums commute) and within 1e-5 for
floating types (colliding indices are added by atomics in another order than the oracle's).
"""
import numpy as np
import pytest

import kd
import support
from test_gpu_index import index_layout

pytestmark = pytest.mark.gpu

SIZES = [1, 2, 3, 5, 8, 13, 40]


def random_strides(shape, rng):
    """Element strides of a random non-overlapping layout of `shape`, and the storage length."""
    rank = len(shape)
    kind = rng.integers(0, 3)
    order = rng.permutation(rank) if kind == 1 else np.arange(rank)
    steps = [int(rng.integers(1, 3)) if kind == 2 else 1 for _ in range(rank)]
    strides = [0] * rank
    acc = 1
    for d in reversed(order):
        strides[d] = acc * steps[d]
        acc *= max(shape[d], 1) * steps[d]
    length = 1 + sum((n - 1) * s for n, s in zip(shape, strides)) if all(shape) else 1
    return strides, length


def make_case(seed):
    rng = np.random.default_rng(seed)
    rank = int(rng.integers(1, 5))
    shape = [SIZES[int(rng.integers(0, len(SIZES)))] for _ in range(rank)]
    axis = int(rng.integers(0, rank))
    extent = SIZES[int(rng.integers(0, len(SIZES)))]
    data_shape = list(shape)
    data_shape[axis] = extent
    data_strides, data_len = random_strides(data_shape, rng)
    index_strides, index_len = random_strides(shape, rng)
    for d in range(rank):  # broadcast indices along some dims
        if d != axis and rng.random() < 0.2:
            index_strides[d] = 0
    other_strides, other_len = random_strides(shape, rng)
    return rng, shape, axis, extent, (data_strides, data_len), (index_strides, index_len), (other_strides, other_len)


CASES = list(range(240))
NP = {kd.F32: np.float32, kd.F64: np.float64, kd.I64: np.int64, kd.BOOL: np.uint8}


def values(rng, dtype, n):
    if dtype == kd.I64:
        return rng.integers(-(2 ** 62), 2 ** 62, n, dtype=np.int64)
    if dtype == kd.BOOL:
        return rng.integers(0, 2, n).astype(np.uint8)
    return (rng.normal(size=n) * 3).astype(NP[dtype])


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
def test_random_gathers(kdb, oracle, dtype):
    for seed in CASES:
        rng, shape, axis, extent, (ds, dl), (is_, il), (os_, ol) = make_case(seed)
        data = values(rng, dtype, dl)
        idx = rng.integers(0, extent, il).astype(np.int64)
        lay = index_layout(tuple(shape), axis, ds, is_, os_)
        want = np.zeros(ol, NP[dtype])
        assert oracle.oracle_gather(dtype, support.ptr(want), support.ptr(data), support.ptr(idx), lay) == 0
        dd, di, do = kdb.to_device(data), kdb.to_device(idx), kdb.to_device(np.zeros(ol, NP[dtype]))
        kdb.call("gather", dtype, do.ptr, dd.ptr, di.ptr, lay)
        got = do.numpy()
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), f"seed {seed}: shape {shape} axis {axis}"


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64], ids=["f32", "f64", "i64"])
def test_random_scatter_adds(kdb, oracle, dtype):
    for seed in CASES:
        rng, shape, axis, extent, (ds, dl), (is_, il), (ss, sl) = make_case(seed)
        target = values(rng, dtype, dl)
        idx = rng.integers(0, extent, il).astype(np.int64)
        src = values(rng, dtype, sl)
        lay = index_layout(tuple(shape), axis, ds, is_, ss)
        want = target.copy()
        assert oracle.oracle_scatter_add(dtype, support.ptr(want), support.ptr(idx), support.ptr(src), lay) == 0
        dt, di, dsrc = kdb.to_device(target), kdb.to_device(idx), kdb.to_device(src)
        kdb.call("scatter_add", dtype, dt.ptr, di.ptr, dsrc.ptr, lay)
        got = dt.numpy()
        if dtype == kd.I64:
            assert np.array_equal(got, want), f"seed {seed}: shape {shape} axis {axis}"
        else:
            np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5, err_msg=f"seed {seed}: shape {shape} axis {axis}")

"""kd_gather / kd_scatter_add against the C oracle (reference src/cuda/kernels.inl:179-221).

Covers the embedding lookup of GPT-2 decode ([1]/[64] token ids into [50257,768] and [1024,768]),
gather along an inner axis with a transposed index tensor (tests/test_cuda.cpp:365-384) and
i64 scatter_add wrapping (:482-490). Gather is bit-exact; f32 scatter_add with colliding indices
adds in a different order than the oracle (atomics), so it is checked to 1e-5.
"""
import ctypes

import numpy as np
import pytest

import kd
import support

pytestmark = pytest.mark.gpu


index_layout = kd.index_layout


@pytest.mark.parametrize("tokens", [1, 64])
def test_embedding_gather(kdb, oracle, tokens):
    rng = np.random.default_rng(tokens)
    vocab, dim = 50257, 768
    table = rng.normal(0, 0.02, (vocab, dim)).astype(np.float32)
    ids = rng.integers(0, vocab, tokens).astype(np.int64)
    # index_select(weight, 0, ids) -> gather over shape [tokens, dim], axis 0 (indexing.cpp:109-118)
    lay = index_layout((tokens, dim), 0, (dim, 1), (1, 0), (dim, 1))
    want = np.empty((tokens, dim), np.float32)
    assert oracle.oracle_gather(kd.F32, support.ptr(want), support.ptr(table), support.ptr(ids), lay) == 0
    dt, di, do = kdb.to_device(table), kdb.to_device(ids), kdb.empty((tokens, dim), np.float32)
    kdb.call("gather", kd.F32, do.ptr, dt.ptr, di.ptr, lay)
    np.testing.assert_array_equal(do.numpy(), want)


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
def test_gather_inner_axis_transposed_indices(kdb, oracle, dtype):
    rng = np.random.default_rng(dtype)
    npd = kd.NUMPY_DTYPE[dtype]
    data = (rng.normal(size=(6, 5)) * 10).astype(npd)
    idx = rng.integers(0, 5, (3, 6)).astype(np.int64)  # used transposed: shape [6, 3], strides (1, 6)
    lay = index_layout((6, 3), 1, (5, 1), (1, 6), (3, 1))
    want = np.empty((6, 3), npd)
    assert oracle.oracle_gather(dtype, support.ptr(want), support.ptr(data), support.ptr(idx), lay) == 0
    dd, di, do = kdb.to_device(data), kdb.to_device(idx), kdb.empty((6, 3), npd)
    kdb.call("gather", dtype, do.ptr, dd.ptr, di.ptr, lay)
    np.testing.assert_array_equal(do.numpy(), want)


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64], ids=["f32", "f64", "i64"])
def test_scatter_add(kdb, oracle, dtype):
    rng = np.random.default_rng(10 + dtype)
    npd = kd.NUMPY_DTYPE[dtype]
    rows, dim, n = 96, 256, 4096  # char-GPT embedding gradient: index_add_ of [4096,256] into [96,256]
    target = np.zeros((rows, dim), npd)
    ids = rng.integers(0, rows, n).astype(np.int64)
    src = (rng.normal(size=(n, dim)) * 4).astype(npd) if dtype != kd.I64 else rng.integers(-9, 9, (n, dim)).astype(np.int64)
    lay = index_layout((n, dim), 0, (dim, 1), (1, 0), (dim, 1))
    want = target.copy()
    assert oracle.oracle_scatter_add(dtype, support.ptr(want), support.ptr(ids), support.ptr(src), lay) == 0
    dtgt, di, ds = kdb.to_device(target), kdb.to_device(ids), kdb.to_device(src)
    kdb.call("scatter_add", dtype, dtgt.ptr, di.ptr, ds.ptr, lay)
    got = dtgt.numpy()
    if dtype == kd.I64:
        np.testing.assert_array_equal(got, want)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-4)


def test_int64_scatter_add_wraps(kdb):
    target = kdb.to_device(np.array([2**63 - 1], np.int64))
    ids = kdb.to_device(np.array([0], np.int64))
    src = kdb.to_device(np.array([1], np.int64))
    kdb.call("scatter_add", kd.I64, target.ptr, ids.ptr, src.ptr, index_layout((1,), 0, (1,), (1,), (1,)))
    assert target.numpy()[0] == -(2**63)


# Row mode (one wave per row, the index loaded once per row): embedding-shaped layouts whose
# innermost dim is contiguous and not indexed, with 16-byte vectors where every row start allows
# them, single elements otherwise (odd row lengths, a data pointer one element off alignment),
# an indexed middle axis, and the element path for rows shorter than a wave.
ROW_LAYOUTS = [
    # (data shape, index count, axis, row length, data offset in elements)
    ((300, 256), 1000, 0, 256, 0),
    ((300, 67), 1000, 0, 67, 0),
    ((300, 256), 517, 0, 256, 1),
    ((5, 40, 96), 33, 1, 96, 0),
    ((300, 40), 1000, 0, 40, 0),
]


def _row_case(dtype, data_shape, n_idx, axis, offset, seed):
    rng = np.random.default_rng(seed)
    npd = kd.NUMPY_DTYPE[dtype]
    flat = (rng.normal(size=int(np.prod(data_shape)) + offset) * 8).astype(npd)
    data = flat[offset:].reshape(data_shape)
    ids = rng.integers(0, data_shape[axis], n_idx).astype(np.int64)
    shape = list(data_shape)
    shape[axis] = n_idx
    dstr = [int(np.prod(data_shape[d + 1:])) for d in range(len(data_shape))]
    istr = [0] * len(shape)
    istr[axis] = 1
    sstr = [int(np.prod(shape[d + 1:])) for d in range(len(shape))]
    return flat, data, ids, shape, kd.index_layout(tuple(shape), axis, dstr, istr, sstr)


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
@pytest.mark.parametrize("case", range(len(ROW_LAYOUTS)))
def test_gather_rows(kdb, oracle, dtype, case):
    data_shape, n_idx, axis, _, offset = ROW_LAYOUTS[case]
    flat, data, ids, shape, lay = _row_case(dtype, data_shape, n_idx, axis, offset, case)
    npd = kd.NUMPY_DTYPE[dtype]
    want = np.empty(shape, npd)
    assert oracle.oracle_gather(dtype, support.ptr(want), support.ptr(np.ascontiguousarray(data)), support.ptr(ids),
                                lay) == 0
    np.testing.assert_array_equal(want, np.take(data, ids, axis=axis))
    dflat, di, do = kdb.to_device(flat), kdb.to_device(ids), kdb.empty(tuple(shape), npd)
    size = np.dtype(npd).itemsize
    kdb.call("gather", dtype, do.ptr, dflat.ptr + offset * size, di.ptr, lay)
    np.testing.assert_array_equal(do.numpy(), want)


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64], ids=["f32", "f64", "i64"])
@pytest.mark.parametrize("case", range(len(ROW_LAYOUTS)))
def test_scatter_add_rows(kdb, oracle, dtype, case):
    data_shape, n_idx, axis, _, offset = ROW_LAYOUTS[case]
    flat, data, ids, shape, lay = _row_case(dtype, data_shape, n_idx, axis, offset, 50 + case)
    npd = kd.NUMPY_DTYPE[dtype]
    rng = np.random.default_rng(case)
    src = (rng.normal(size=shape) * 4).astype(npd) if dtype != kd.I64 else rng.integers(-9, 9, shape).astype(np.int64)
    want = np.ascontiguousarray(data).copy()
    assert oracle.oracle_scatter_add(dtype, support.ptr(want), support.ptr(ids), support.ptr(src), lay) == 0
    dflat, di, ds = kdb.to_device(flat), kdb.to_device(ids), kdb.to_device(src)
    size = np.dtype(npd).itemsize
    kdb.call("scatter_add", dtype, dflat.ptr + offset * size, di.ptr, ds.ptr, lay)
    got = dflat.numpy()[offset:].reshape(data_shape)
    if dtype == kd.I64:
        np.testing.assert_array_equal(got, want)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-4)


BOUNDS_CASES = [  # count, stride
    (1, 1), (7, 1), (4096, 1), (16384, 1), (16385, 1), (1 << 20, 1), (9_000_001, 1), (1000, 3), (5000, 0), (3000, -2),
]


@pytest.mark.parametrize("count, stride", BOUNDS_CASES, ids=[f"{c}x{s}" for c, s in BOUNDS_CASES])
def test_index_bounds(kdb, oracle, count, stride):
    """kd_index_bounds (the min and max kael reads back before a device gather / scatter_add, one
    call) against numpy's min / max of the same strided run and the oracle: exact, with the
    int64 extremes planted at random positions for the larger runs; one workgroup up to 16384
    elements, partial pairs and a combine launch above."""
    rng = np.random.default_rng(count + stride)
    span = (count - 1) * abs(stride) + 1
    store = rng.integers(-(1 << 40), 1 << 40, span).astype(np.int64)
    if count > 2 and stride != 0:
        run = np.arange(count) * abs(stride)
        lo, hi = rng.choice(count, 2, replace=False)
        store[run[lo]], store[run[hi]] = np.iinfo(np.int64).min, np.iinfo(np.int64).max
    first = 0 if stride >= 0 else (count - 1) * abs(stride)
    values = store[first + np.arange(count) * stride]
    want = np.array([values.min(), values.max()], np.int64)
    dev = kdb.to_device(store)
    got = np.zeros(2, np.int64)
    kdb.call("index_bounds", dev.ptr + first * 8, count, stride, support.ptr(got))
    np.testing.assert_array_equal(got, want)
    orc = np.zeros(2, np.int64)
    assert oracle.oracle_index_bounds(ctypes.c_void_p(store.ctypes.data + first * 8), count, stride,
                                      support.ptr(orc)) == 0
    np.testing.assert_array_equal(orc, want)


def test_index_bounds_rejects_an_empty_run(kdb):
    dev = kdb.to_device(np.zeros(4, np.int64))
    got = np.zeros(2, np.int64)
    with pytest.raises(kd.KdError):
        kdb.call("index_bounds", dev.ptr, 0, 1, support.ptr(got))

"""Pins the C oracle against the reference's own device tasks at the exact device boundary.

Both sides take identical kd_element_layout / kd_index_layout arguments over host memory:
  oracle_*     oracle/kd_oracle.c (the restatement)
  ref_dev_*    reference src/cuda/kernels.inl executed by the reference's host emulation
               backend (src/cuda/backend_fake.cpp), compiled unmodified.
Integer, bool, copy and non-transcendental float results must be bit-exact. Transcendental
ops call the same glibc functions on both sides, but the reference build may contract a*b+c
into FMA, so they are compared to 2e-6 relative. The emulation backend visits elements in
reverse order (backend_fake.cpp:13-18), so f32 scatter_add with collisions differs in order.
"""
import ctypes

import numpy as np
import pytest

import kd
import support
from views import View, contiguous, layout_of, random_values, stepped, transposed

EXACT_OPS = set(range(36)) - {kd.OP[n] for n in ("POWER", "EXP", "LOG", "LOG1P", "EXPM1", "RSQRT", "SIN", "COS",
                                                  "TANH", "SIGMOID", "GELU_EXACT", "GELU_TANH")}


def layouts(n_in):
    shape = (5, 12)
    return {
        "contiguous": [contiguous(shape)] * (n_in + 1),
        "transposed": [contiguous(shape)] + [transposed(shape)] * n_in,
        "strided": [contiguous(shape)] + [stepped(shape)] * n_in,
        "broadcast": [contiguous(shape)] + [contiguous((12,))] * n_in,
        "column": [contiguous(shape)] + [contiguous((5, 1))] * n_in,
        "batched": [contiguous((2, 3, 4))] + [View((2, 3, 4), (1, 8, 2))] * n_in,
    }


def run_pair(oracle, refdev, views, in_dtype, out_dtype, call_o, call_r, rng, op=None):
    in_np, out_np = kd.NUMPY_DTYPE[in_dtype], kd.NUMPY_DTYPE[out_dtype]
    stores = [np.zeros(views[0].storage_len, out_np)] + [random_values(rng, in_np, v.storage_len, op) for v in views[1:]]
    a = [s.copy() for s in stores]
    b = [s.copy() for s in stores]
    sizes = [np.dtype(out_np).itemsize] + [np.dtype(in_np).itemsize] * (len(views) - 1)
    la = layout_of(oracle.oracle_layout_build, views, sizes, [x.ctypes.data + v.offset * s for x, v, s in zip(a, views, sizes)])
    lb = layout_of(oracle.oracle_layout_build, views, sizes, [x.ctypes.data + v.offset * s for x, v, s in zip(b, views, sizes)])
    assert call_o(la) == 0
    assert call_r(lb) == 0, support.ref_error(refdev)
    return a[0], b[0]


def same(x, y, exact, what):
    if x.dtype.kind == "f":
        if exact:
            ok = (x == y) | (np.isnan(x) & np.isnan(y))
            assert ok.all(), f"{what}: {x[~ok][:4]} vs {y[~ok][:4]}"
        else:
            ok, msg = support.golden_close(x, y, 2e-6, 1e-7 if x.dtype == np.float32 else 1e-15)
            assert ok, f"{what}: {msg}"
    else:
        assert np.array_equal(x, y), what


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
@pytest.mark.parametrize("op", range(36), ids=lambda o: kd.OPS[o])
def test_elementwise_matches_reference_tasks(oracle, refdev, op, dtype):
    if op in kd.FLOATING_OPS and dtype not in (kd.F32, kd.F64):
        pytest.skip("the reference host never sends floating ops on integer dtypes")
    if op == kd.OP["DIVIDES"] and dtype in (kd.I64, kd.BOOL):
        pytest.skip("integer division by zero is undefined in the reference (traps)")
    rng = np.random.default_rng(op * 5 + dtype)
    p = kd.params(reals=(-0.5, 0.75), integers=(-3, 20)) if op == kd.OP["CLAMP"] else kd.params(reals=(7.0, 0), integers=(7, 0))
    out_dtype = kd.BOOL if op in kd.COMPARE_OPS else dtype
    for name, views in layouts(kd.op_inputs(op)).items():
        a, b = run_pair(oracle, refdev, views, dtype, out_dtype,
                        lambda lay: oracle.oracle_elementwise(op, out_dtype, dtype, lay, p),
                        lambda lay: refdev.ref_dev_elementwise(op, out_dtype, dtype, lay, p), rng, op)
        same(a, b, op in EXACT_OPS, f"{kd.OPS[op]}/{name}")


@pytest.mark.parametrize("out_dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL])
@pytest.mark.parametrize("in_dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL])
def test_convert_matches_reference_tasks(oracle, refdev, in_dtype, out_dtype):
    rng = np.random.default_rng(in_dtype * 4 + out_dtype)
    for name, views in layouts(1).items():
        a, b = run_pair(oracle, refdev, views, in_dtype, out_dtype,
                        lambda lay: oracle.oracle_convert(out_dtype, in_dtype, lay),
                        lambda lay: refdev.ref_dev_convert(out_dtype, in_dtype, lay), rng)
        same(a, b, True, f"convert/{name}")


def test_saturating_casts_match(oracle, refdev):
    x = np.array([np.nan, np.inf, -np.inf, 1e300, -1e300, 9.3e18, -9.3e18, 2.9, -2.9, 0.5], np.float64)
    views = [contiguous((10,)), contiguous((10,))]
    for out_dtype in (kd.I64, kd.BOOL, kd.F32):
        outs = []
        for fn in (lambda l: oracle.oracle_convert(out_dtype, kd.F64, l), lambda l: refdev.ref_dev_convert(out_dtype, kd.F64, l)):
            o = np.zeros(10, kd.NUMPY_DTYPE[out_dtype])
            lay = layout_of(oracle.oracle_layout_build, views, [o.itemsize, 8], [o.ctypes.data, x.ctypes.data])
            assert fn(lay) == 0
            outs.append(o)
        same(outs[0], outs[1], True, f"cast to {out_dtype}")


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL])
@pytest.mark.parametrize("op", [kd.REDUCE_SUM, kd.REDUCE_MAX, kd.REDUCE_MIN])
@pytest.mark.parametrize("rows,chunk", [(1, 1), (7, 13), (3, 4096), (2, 4097), (2, 50000), (1, 300001)])
def test_reduce_matches_reference_tasks_bit_exact(oracle, refdev, op, dtype, rows, chunk):
    rng = np.random.default_rng(rows + chunk + op + dtype)
    x = random_values(rng, kd.NUMPY_DTYPE[dtype], rows * chunk)
    out_np = np.int64 if (op == kd.REDUCE_SUM and dtype in (kd.I64, kd.BOOL)) else kd.NUMPY_DTYPE[dtype]
    a, b = np.zeros(rows, out_np), np.zeros(rows, out_np)
    assert oracle.oracle_reduce(op, 0, dtype, support.ptr(a), support.ptr(x), chunk, rows) == 0
    assert refdev.ref_dev_reduce(op, 0, dtype, support.ptr(b), support.ptr(x), chunk, rows) == 0
    same(a, b, True, "reduce")


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL])
@pytest.mark.parametrize("op", [kd.REDUCE_SUM, kd.REDUCE_MAX, kd.REDUCE_MIN])
@pytest.mark.parametrize("outer,inner", [(1, 1), (13, 7), (4096, 5), (4097, 3), (9000, 2), (2, 300)])
def test_reduce_columns_match_reference_tasks_over_the_transposed_copy(oracle, refdev, op, dtype, outer, inner):
    """oracle_reduce_columns (kd_reduce_columns' restatement) against what kael does today for a
    contiguous [outer, inner] tensor reduced over its leading dim: plan_reduction's copy with that
    dim moved last, then the reference's device reduce tasks with chunk = outer, rows = inner."""
    rng = np.random.default_rng(outer * 31 + inner + op + dtype)
    x = random_values(rng, kd.NUMPY_DTYPE[dtype], outer * inner)
    out_np = np.int64 if (op == kd.REDUCE_SUM and dtype in (kd.I64, kd.BOOL)) else kd.NUMPY_DTYPE[dtype]
    a, b = np.zeros(inner, out_np), np.zeros(inner, out_np)
    assert oracle.oracle_reduce_columns(op, 0, dtype, support.ptr(a), support.ptr(x), outer, inner) == 0
    xt = np.ascontiguousarray(x.reshape(outer, inner).T)
    assert refdev.ref_dev_reduce(op, 0, dtype, support.ptr(b), support.ptr(xt), outer, inner) == 0
    same(a, b, True, "reduce_columns")


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64])
@pytest.mark.parametrize("b,m,k,n", [(1, 1, 1, 1), (1, 5, 3, 9), (2, 33, 20, 65), (3, 4, 0, 2), (1, 64, 128, 7)])
def test_matmul_matches_reference_tasks(oracle, refdev, dtype, b, m, k, n):
    rng = np.random.default_rng(m * n + k)
    npd = kd.NUMPY_DTYPE[dtype]
    A = random_values(rng, npd, b * m * k) if dtype == kd.I64 else rng.uniform(-1, 1, b * m * k).astype(npd)
    B = random_values(rng, npd, b * k * n) if dtype == kd.I64 else rng.uniform(-1, 1, b * k * n).astype(npd)
    o1, o2 = np.full(b * m * n, 3, npd), np.full(b * m * n, 3, npd)
    s = kd.MatmulSizes(b, m, k, n)
    assert oracle.oracle_matmul(dtype, support.ptr(A), support.ptr(B), support.ptr(o1), s, 0) == 0
    assert refdev.ref_dev_matmul(dtype, support.ptr(A), support.ptr(B), support.ptr(o2), s) == 0
    if dtype == kd.I64:
        same(o1, o2, True, "matmul")
        return
    # The reference build may contract acc + a*b into one FMA; bound the difference by the
    # accumulated magnitude sum_k |a_ik||b_kj| (a few ulps of it).
    scale = np.matmul(np.abs(A.reshape(b, m, k)).astype(np.float64), np.abs(B.reshape(b, k, n)).astype(np.float64)).ravel()
    eps = np.finfo(npd).eps
    assert np.all(np.abs(o1.astype(np.float64) - o2) <= 4 * eps * (scale + 1e-30)), "matmul"


def index_layout(shape, axis, ds, ix, ss):
    lay = kd.IndexLayout()
    lay.dims, lay.axis, lay.count = len(shape), axis, int(np.prod(shape))
    for d in range(len(shape)):
        lay.shape[d], lay.data_strides[d], lay.index_strides[d], lay.source_strides[d] = shape[d], ds[d], ix[d], ss[d]
    return lay


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL])
def test_gather_and_scatter_match_reference_tasks(oracle, refdev, dtype):
    rng = np.random.default_rng(dtype)
    npd = kd.NUMPY_DTYPE[dtype]
    data = random_values(rng, npd, 6 * 5)
    idx = rng.integers(0, 5, 18).astype(np.int64)
    lay = index_layout((6, 3), 1, (5, 1), (1, 6), (3, 1))
    a, b = np.zeros(18, npd), np.zeros(18, npd)
    assert oracle.oracle_gather(dtype, support.ptr(a), support.ptr(data), support.ptr(idx), lay) == 0
    assert refdev.ref_dev_gather(dtype, support.ptr(b), support.ptr(data), support.ptr(idx), lay) == 0
    same(a, b, True, "gather")
    if dtype == kd.BOOL:
        return
    src = random_values(rng, npd, 18)
    t1, t2 = data.copy(), data.copy()
    assert oracle.oracle_scatter_add(dtype, support.ptr(t1), support.ptr(idx), support.ptr(src), lay) == 0
    assert refdev.ref_dev_scatter_add(dtype, support.ptr(t2), support.ptr(idx), support.ptr(src), lay) == 0
    same(t1, t2, dtype == kd.I64, "scatter_add")


def test_fill_matches(oracle, refdev):
    for dtype, v in ((kd.F32, -1.5), (kd.F64, 2.25), (kd.I64, 2**53 + 1), (kd.BOOL, 1)):
        val = np.array([v], kd.NUMPY_DTYPE[dtype])
        a, b = np.zeros(37, val.dtype), np.zeros(37, val.dtype)
        assert oracle.oracle_fill(dtype, support.ptr(a), 37, support.ptr(val)) == 0
        assert refdev.ref_dev_fill(dtype, support.ptr(b), 37, support.ptr(val)) == 0
        same(a, b, True, "fill")

"""Fused row kernels against the C oracle (which restates reference src/ops/nn.cpp:52-129,
214-240) and, for the GELU slope, kael's own autograd (GeluBackward) through the reference build.

Shapes: GPT-2 attention rows (P <= 1024), char-GPT CE rows (96 classes), LayerNorm rows (256,
768), rows longer than one wave's register tile (1025, 50257), plus +-inf / all -inf rows as in
the reference's softmax golden cases. Tolerance: rtol 1e-5 / atol 1e-6 for f32 (the device exp
and log come from ROCm's device library, the CPU's from glibc), 1e-12 for f64.
"""
import numpy as np
import pytest

import kd
import support

pytestmark = pytest.mark.gpu

COLS = [1, 10, 64, 96, 300, 768, 1024, 1025, 50257]


def tol(dtype):
    return (1e-5, 1e-6) if dtype == kd.F32 else (1e-12, 1e-14)


def check(got, want, dtype, what):
    ok, msg = support.golden_close(got, want, *tol(dtype))
    assert ok, f"{what}: {msg}"


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64], ids=["f32", "f64"])
@pytest.mark.parametrize("cols", COLS)
@pytest.mark.parametrize("log", [0, 1], ids=["softmax", "log_softmax"])
def test_softmax_rows(kdb, oracle, dtype, cols, log):
    rng = np.random.default_rng(cols + log)
    rows = 9 if cols < 50257 else 4
    npd = kd.NUMPY_DTYPE[dtype]
    x = rng.normal(0, 4, (rows, cols)).astype(npd)
    if cols >= 10:
        x[1, 3] = np.inf
        x[2, :] = -np.inf
        x[3, 5] = -np.inf
    want = np.empty_like(x)
    assert oracle.oracle_softmax_rows(dtype, support.ptr(want), support.ptr(x), rows, cols, log) == 0
    dx, dy = kdb.to_device(x), kdb.empty(x.shape, npd)
    kdb.call("softmax_rows", dtype, dy.ptr, dx.ptr, rows, cols, log)
    check(dy.numpy(), want, dtype, "softmax")


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64], ids=["f32", "f64"])
@pytest.mark.parametrize("cols", [1, 4, 256, 768, 1024, 3000])
@pytest.mark.parametrize("affine", [False, True])
def test_standardize_rows(kdb, oracle, dtype, cols, affine):
    rng = np.random.default_rng(cols * 2 + affine)
    rows = 33
    npd = kd.NUMPY_DTYPE[dtype]
    x = rng.normal(0.3, 2, (rows, cols)).astype(npd)
    w = rng.normal(1, 0.1, cols).astype(npd) if affine else None
    b = rng.normal(0, 0.1, cols).astype(npd) if affine else None
    want = np.empty_like(x)
    assert oracle.oracle_standardize_rows(dtype, support.ptr(want), support.ptr(x), rows, cols, 1e-5,
                                          support.ptr(w) if affine else None, support.ptr(b) if affine else None) == 0
    dx, dy = kdb.to_device(x), kdb.empty(x.shape, npd)
    dw = kdb.to_device(w) if affine else None
    db = kdb.to_device(b) if affine else None
    kdb.call("standardize_rows", dtype, dy.ptr, dx.ptr, rows, cols, 1e-5, dw.ptr if affine else None,
             db.ptr if affine else None)
    check(dy.numpy(), want, dtype, "standardize")
    if not affine and cols > 1:
        y = dy.numpy().astype(np.float64)
        assert np.allclose(y.mean(axis=1), 0, atol=1e-5)
        assert np.allclose(y.var(axis=1), 1, atol=1e-3)


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64], ids=["f32", "f64"])
@pytest.mark.parametrize("rows,cols", [(64, 10), (4096, 96), (7, 2000)])
def test_cross_entropy(kdb, oracle, dtype, rows, cols):
    rng = np.random.default_rng(rows + cols)
    npd = kd.NUMPY_DTYPE[dtype]
    x = rng.normal(0, 3, (rows, cols)).astype(npd)
    t = rng.integers(0, cols, rows).astype(np.int64)
    w = np.full(rows, 1.0 / rows, npd)
    want = np.empty(rows, npd)
    assert oracle.oracle_cross_entropy_rows(dtype, support.ptr(want), support.ptr(x), support.ptr(t), rows, cols) == 0
    dx, dt, dl = kdb.to_device(x), kdb.to_device(t), kdb.empty((rows,), npd)
    kdb.call("cross_entropy_rows", dtype, dl.ptr, dx.ptr, dt.ptr, rows, cols)
    check(dl.numpy(), want, dtype, "cross_entropy")
    gwant = np.empty_like(x)
    assert oracle.oracle_cross_entropy_grad(dtype, support.ptr(gwant), support.ptr(x), support.ptr(t), support.ptr(w),
                                            rows, cols) == 0
    dw, dg = kdb.to_device(w), kdb.empty(x.shape, npd)
    kdb.call("cross_entropy_grad", dtype, dg.ptr, dx.ptr, dt.ptr, dw.ptr, rows, cols)
    check(dg.numpy(), gwant, dtype, "cross_entropy_grad")
    # Each gradient row sums to zero (softmax sums to one).
    assert np.allclose(dg.numpy().astype(np.float64).sum(axis=1), 0, atol=1e-6)

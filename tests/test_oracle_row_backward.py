"""Pins of the oracle's row backward passes (oracle_softmax_rows_backward,
oracle_standardize_rows_backward), which restate kael's composed SoftmaxBackward,
LogSoftmaxBackward and StandardizeBackward (reference src/autograd/functions_reduce.cpp:150-192).

  1. The reference's own device path: kael's autograd with the reference's host emulation of its
     device tasks (src/cuda/backend_fake.cpp running src/cuda/kernels.inl) composes the same
     backward from element ops and device reductions: equal bit for bit.
  2. kael's CPU autograd (its own CPU reductions): equal within f32 rounding.
  3. Mathematics, independent of kael: the gradient of sum(g * op(x)) by central differences in
     float64, and the invariants a mistake would break (softmax: a constant g gives zero;
     log_softmax: each row of the gradient sums to sum(g) - sum(g) * sum(exp(y)) = 0; standardize:
     a constant g and g = y give zero).
  4. kael with the optional device branches (oracle/kael_fused.py) over the oracle: the branch calls
     the fused entry point and keeps the bits of kael's composed path.
"""
import ctypes

import numpy as np
import pytest

import kd
import support

P = support.ptr
KIND = {"softmax": 0, "log_softmax": 1, "standardize": 2}
SHAPES = [(5, 7), (64, 10), (33, 128), (16, 256), (4, 768), (2, 4097), (3, 10000)]
EPS = 1e-5


def forward(oracle, kind, dtype, x):
    rows, cols = x.shape
    y = np.empty_like(x)
    if kind == "standardize":
        assert oracle.oracle_standardize_rows(dtype, P(y), P(x), rows, cols, EPS, None, None) == 0
    else:
        assert oracle.oracle_softmax_rows(dtype, P(y), P(x), rows, cols, int(kind == "log_softmax")) == 0
    return y


def oracle_backward(oracle, kind, dtype, x, y, g):
    rows, cols = x.shape
    out = np.empty_like(x)
    if kind == "standardize":
        assert oracle.oracle_standardize_rows_backward(dtype, P(out), P(x), P(y), P(g), rows, cols, EPS) == 0
    else:
        assert oracle.oracle_softmax_rows_backward(dtype, P(out), P(y), P(g), rows, cols,
                                                   int(kind == "log_softmax")) == 0
    return out


def kael_grad(lib, kind, device, x, g, with_y=False):
    """x.grad of sum(g * op(x)) through kael's autograd; with_y: also kael's forward output."""
    rows, cols = x.shape
    out, y = np.empty_like(x), np.empty_like(x)
    dt = 0 if x.dtype == np.float32 else 1
    assert lib.ref_row_grad(KIND[kind], device, dt, P(x), P(g), rows, cols, EPS, P(out), P(y)) == 0, \
        support.ref_error(lib)
    return (out, y) if with_y else out


def inputs(kind, shape, npdtype, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0, 2, shape).astype(npdtype)
    g = rng.uniform(-1, 1, shape).astype(npdtype)
    return x, g


@pytest.mark.parametrize("npdtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("kind", list(KIND))
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_oracle_equals_reference_device_composition(oracle, refdev, kind, npdtype, shape):
    x, g = inputs(kind, shape, npdtype, shape[0] * 7 + shape[1])
    dtype = kd.F32 if npdtype == np.float32 else kd.F64
    # kael on the reference's emulated device: its forward output y (composed on the device for
    # standardize, nn.cpp:253-258) and the composed backward from that y.
    want, y = kael_grad(refdev, kind, 1, x, g, with_y=True)
    got = oracle_backward(oracle, kind, dtype, x, y, g)
    np.testing.assert_array_equal(got, want)
    cpu = kael_grad(refdev, kind, 0, x, g)
    scale = np.abs(cpu).max()
    tol = 1e-5 if npdtype == np.float32 else 1e-12
    assert np.abs(got.astype(np.float64) - cpu).max() <= tol * scale


def numeric_gradient(f, x, h=1e-6):
    """Central differences of the scalar f at x (float64), one coordinate at a time."""
    grad = np.empty_like(x)
    flat, gflat = x.reshape(-1), grad.reshape(-1)
    for i in range(flat.size):
        keep = flat[i]
        flat[i] = keep + h
        up = f(x)
        flat[i] = keep - h
        down = f(x)
        flat[i] = keep
        gflat[i] = (up - down) / (2 * h)
    return grad


@pytest.mark.parametrize("kind", list(KIND))
def test_oracle_matches_finite_differences(oracle, kind):
    """The gradient of sum(g * op(x)) in float64 by central differences, where op is numpy's own
    softmax, log_softmax or standardization (no oracle code in the objective)."""
    rng = np.random.default_rng(11)
    x = rng.normal(0, 1.5, (3, 9))
    g = rng.uniform(-1, 1, (3, 9))

    def op(v):
        if kind == "standardize":
            return (v - v.mean(axis=1, keepdims=True)) / np.sqrt(v.var(axis=1, keepdims=True) + EPS)
        s = v - v.max(axis=1, keepdims=True)
        if kind == "softmax":
            e = np.exp(s)
            return e / e.sum(axis=1, keepdims=True)
        return s - np.log(np.exp(s).sum(axis=1, keepdims=True))

    want = numeric_gradient(lambda v: float((g * op(v)).sum()), x.copy())
    y = forward(oracle, kind, kd.F64, x)
    got = oracle_backward(oracle, kind, kd.F64, x, y, g)
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-8)


def test_invariants(oracle):
    rng = np.random.default_rng(12)
    x = rng.normal(0, 1, (6, 50))
    c = np.full_like(x, 0.75)
    # softmax is invariant to adding a constant: a constant gradient has no component left
    y = forward(oracle, "softmax", kd.F64, x)
    assert np.abs(oracle_backward(oracle, "softmax", kd.F64, x, y, c)).max() < 1e-15
    # log_softmax: the gradient of each row sums to zero (shift invariance again)
    g = rng.uniform(-1, 1, x.shape)
    ly = forward(oracle, "log_softmax", kd.F64, x)
    np.testing.assert_allclose(oracle_backward(oracle, "log_softmax", kd.F64, x, ly, g).sum(axis=1), 0, atol=1e-13)
    # standardize is invariant to shifts and (nearly, eps aside) to scalings of each row: constant
    # g and g = y give a zero gradient
    sy = forward(oracle, "standardize", kd.F64, x)
    assert np.abs(oracle_backward(oracle, "standardize", kd.F64, x, sy, c)).max() < 1e-13
    assert np.abs(oracle_backward(oracle, "standardize", kd.F64, x, sy, sy)).max() < 1e-4


def test_planted_mistake_is_caught(refdev):
    """A restatement that forgot y in the softmax row sum (sum(g) instead of sum(g * y)) differs
    from kael's composed backward: the comparison above would fail."""
    x, g = inputs("softmax", (4, 64), np.float32, 3)
    want = kael_grad(refdev, "softmax", 1, x, g)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    y = (e / e.sum(axis=1, keepdims=True)).astype(np.float32)
    wrong = y * (g - g.sum(axis=1, keepdims=True, dtype=np.float64).astype(np.float32))
    assert not np.allclose(wrong, want, rtol=1e-3)


@pytest.mark.parametrize("kind", list(KIND))
def test_fused_branch_calls_the_entry_point_and_keeps_the_bits(oracle, kael_oracle_fused, kind):
    counters = {"softmax": 11, "log_softmax": 11, "standardize": 12}
    fn = kael_oracle_fused.ref_extension_calls
    fn.restype, fn.argtypes = ctypes.c_longlong, [ctypes.c_int]
    x, g = inputs(kind, (16, 256), np.float32, 5)
    before = fn(counters[kind])
    got, y = kael_grad(kael_oracle_fused, kind, 1, x, g, with_y=True)
    assert fn(counters[kind]) == before + 1
    np.testing.assert_array_equal(got, oracle_backward(oracle, kind, kd.F32, x, y, g))

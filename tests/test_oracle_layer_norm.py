"""Pins of the oracle's LayerNorm (oracle_layer_norm_rows, oracle_layer_norm_rows_backward), which
restate kael's LayerNorm::forward, standardize(x) * weight + bias (reference src/nn/layers.cpp:60-68),
and its backward as kael composes it from AddBackward, MulBackward and StandardizeBackward
(src/autograd/functions_math.cpp:54-72, functions_reduce.cpp:176-192).

  1. The reference's own device path: kael's LayerNorm module and autograd over the reference's
     host emulation of its device tasks; given that path's standardized rows, the oracle's
     gradients (input, weight, bias) are equal bit for bit.
  2. kael's CPU path: the forward (standardize in double, then the product and the sum each
     rounded) equal bit for bit; the gradients within f32 rounding.
  3. Mathematics: a constant incoming gradient and a unit weight give a zero input gradient; the
     bias gradient is the column sum of g and the weight gradient the column sum of g * y.
  4. kael with the optional device branches over the oracle: the LayerNorm branch runs
     layer_norm_rows and its backward, and its gradients are the oracle's for its own standardized
     rows, bit for bit.
"""
import ctypes

import numpy as np
import pytest

import kd
import support

P = support.ptr
EPS = 1e-5
SHAPES = [(5, 7), (16, 256), (33, 768), (4, 1030)]


def inputs(rows, cols, npd, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.2, 1.5, (rows, cols)).astype(npd)
    w = rng.normal(1, 0.2, cols).astype(npd)
    b = rng.normal(0, 0.2, cols).astype(npd)
    g = rng.uniform(-1, 1, (rows, cols)).astype(npd)
    return x, w, b, g


def kael_layer_norm(lib, device, x, w, b, g):
    rows, cols = x.shape
    out, y, gx = np.empty_like(x), np.empty_like(x), np.empty_like(x)
    gw, gb = np.empty_like(w), np.empty_like(w)
    dt = 0 if x.dtype == np.float32 else 1
    assert lib.ref_layer_norm_grads(device, dt, P(x), P(w), P(b), P(g), rows, cols, EPS, P(out), P(y), P(gx), P(gw),
                                    P(gb)) == 0, support.ref_error(lib)
    return out, y, gx, gw, gb


def oracle_backward(oracle, dtype, x, y, g, w):
    rows, cols = x.shape
    gx, gw, gb = np.empty_like(x), np.empty_like(w), np.empty_like(w)
    assert oracle.oracle_layer_norm_rows_backward(dtype, P(gx), P(gw), P(gb), P(x), P(y), P(g), P(w), rows, cols,
                                                  EPS) == 0
    return gx, gw, gb


@pytest.mark.parametrize("npd", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_backward_equals_the_reference_device_composition(oracle, refdev, npd, shape):
    x, w, b, g = inputs(*shape, npd, shape[0] * 7 + shape[1])
    dtype = kd.F32 if npd == np.float32 else kd.F64
    _, y, gx, gw, gb = kael_layer_norm(refdev, 1, x, w, b, g)
    ox, ow, ob = oracle_backward(oracle, dtype, x, y, g, w)
    np.testing.assert_array_equal(ox, gx)
    np.testing.assert_array_equal(ow, gw)
    np.testing.assert_array_equal(ob, gb)


@pytest.mark.parametrize("npd", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_forward_equals_kael_cpu_and_gradients_are_close(oracle, refdev, npd, shape):
    x, w, b, g = inputs(*shape, npd, shape[0] * 5 + shape[1])
    dtype = kd.F32 if npd == np.float32 else kd.F64
    rows, cols = shape
    out, y, gx, gw, gb = kael_layer_norm(refdev, 0, x, w, b, g)
    o_out, o_y = np.empty_like(x), np.empty_like(x)
    assert oracle.oracle_layer_norm_rows(dtype, P(o_out), P(o_y), P(x), rows, cols, EPS, P(w), P(b)) == 0
    np.testing.assert_array_equal(o_y, y)
    np.testing.assert_array_equal(o_out, out)
    ox, ow, ob = oracle_backward(oracle, dtype, x, y, g, w)
    tol = 1e-5 if npd == np.float32 else 1e-12
    for got, want in ((ox, gx), (ow, gw), (ob, gb)):
        np.testing.assert_allclose(got, want, rtol=tol, atol=tol * np.abs(want).max())


def test_mathematical_invariants(oracle):
    x, _, _, g = inputs(9, 64, np.float64, 3)
    y = np.empty_like(x)
    assert oracle.oracle_standardize_rows(kd.F64, P(y), P(x), 9, 64, EPS, None, None) == 0
    ones = np.ones(64)
    gx, gw, gb = oracle_backward(oracle, kd.F64, x, y, np.full_like(x, 0.5), ones)
    assert np.abs(gx).max() < 1e-12
    gx, gw, gb = oracle_backward(oracle, kd.F64, x, y, g, ones * 2.0)
    np.testing.assert_allclose(gb, g.sum(axis=0), rtol=1e-13)
    np.testing.assert_allclose(gw, (g * y).sum(axis=0), rtol=1e-12, atol=1e-13)
    # the input gradient for weight w is the standardize backward of g * w
    sx = np.empty_like(x)
    assert oracle.oracle_standardize_rows_backward(kd.F64, P(sx), P(x), P(y), P(g * 2.0), 9, 64, EPS) == 0
    np.testing.assert_array_equal(gx, sx)


@pytest.mark.parametrize("shape", [(16, 256), (5, 7)], ids=["16x256", "5x7"])
def test_fused_branch_takes_the_entry_points_and_keeps_the_bits(oracle, kael_oracle_fused, shape):
    lib = kael_oracle_fused
    fn = lib.ref_extension_calls
    fn.restype, fn.argtypes = ctypes.c_longlong, [ctypes.c_int]
    x, w, b, g = inputs(*shape, np.float32, 11)
    before = fn(16), fn(17)
    out, y, gx, gw, gb = kael_layer_norm(lib, 1, x, w, b, g)
    assert fn(16) - before[0] >= 1 and fn(17) - before[1] == 1
    ox, ow, ob = oracle_backward(oracle, kd.F32, x, y, g, w)
    np.testing.assert_array_equal(ox, gx)
    np.testing.assert_array_equal(ow, gw)
    np.testing.assert_array_equal(ob, gb)

"""Pins of the C oracle that do not depend on the reference's implementation: closed forms,
invariants and brute force, chosen so that a dropped term, a wrong index or a transposed operand
fails. Also the row kernels and GELU slope against kael's CPU path (fused CPU row kernels of
reference src/ops/nn.cpp:52-129, GeluBackward of src/autograd/functions_math.cpp:221-231).
"""
import ctypes

import numpy as np
import pytest

import kd
import support
from views import contiguous, layout_of

P = support.ptr


def test_softmax_rows_sum_to_one_and_shift_invariant(oracle):
    rng = np.random.default_rng(0)
    x = rng.normal(0, 5, (17, 301))
    y = np.empty_like(x)
    z = np.empty_like(x)
    assert oracle.oracle_softmax_rows(kd.F64, P(y), P(x), 17, 301, 0) == 0
    np.testing.assert_allclose(y.sum(axis=1), 1, rtol=1e-14)
    xs = x + 123.0
    assert oracle.oracle_softmax_rows(kd.F64, P(z), P(xs), 17, 301, 0) == 0
    np.testing.assert_allclose(z, y, rtol=1e-11)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    np.testing.assert_allclose(y, e / e.sum(axis=1, keepdims=True), rtol=1e-13)
    assert oracle.oracle_softmax_rows(kd.F64, P(z), P(x), 17, 301, 1) == 0
    np.testing.assert_allclose(np.exp(z), y, rtol=1e-12)


def test_standardize_moments_and_affine(oracle):
    rng = np.random.default_rng(1)
    x = rng.normal(3, 7, (9, 257))
    y = np.empty_like(x)
    assert oracle.oracle_standardize_rows(kd.F64, P(y), P(x), 9, 257, 0.0, None, None) == 0
    np.testing.assert_allclose(y.mean(axis=1), 0, atol=1e-13)
    np.testing.assert_allclose(y.var(axis=1), 1, rtol=1e-12)
    w, b = rng.normal(size=257), rng.normal(size=257)
    z = np.empty_like(x)
    assert oracle.oracle_standardize_rows(kd.F64, P(z), P(x), 9, 257, 1e-5, P(w), P(b)) == 0
    ref = (x - x.mean(axis=1, keepdims=True)) / np.sqrt(x.var(axis=1, keepdims=True) + 1e-5) * w + b
    np.testing.assert_allclose(z, ref, rtol=1e-10, atol=1e-12)


def test_cross_entropy_closed_forms(oracle):
    rng = np.random.default_rng(2)
    x = rng.normal(0, 2, (33, 96))
    t = rng.integers(0, 96, 33).astype(np.int64)
    loss = np.empty(33)
    assert oracle.oracle_cross_entropy_rows(kd.F64, P(loss), P(x), P(t), 33, 96) == 0
    lse = np.log(np.exp(x).sum(axis=1))
    np.testing.assert_allclose(loss, lse - x[np.arange(33), t], rtol=1e-12)
    w = np.full(33, 1.0)
    g = np.empty_like(x)
    assert oracle.oracle_cross_entropy_grad(kd.F64, P(g), P(x), P(t), P(w), 33, 96) == 0
    onehot = np.zeros_like(x)
    onehot[np.arange(33), t] = 1
    np.testing.assert_allclose(g, np.exp(x - lse[:, None]) - onehot, atol=1e-14)


def test_matmul_brute_force_and_identity(oracle):
    rng = np.random.default_rng(3)
    a = rng.normal(size=(2, 5, 7))
    b = rng.normal(size=(2, 7, 3))
    out = np.empty((2, 5, 3))
    assert oracle.oracle_matmul(kd.F64, P(a), P(b), P(out), kd.MatmulSizes(2, 5, 7, 3), 0) == 0
    brute = np.array([[[sum(a[z, i, k] * b[z, k, j] for k in range(7)) for j in range(3)] for i in range(5)] for z in range(2)])
    np.testing.assert_allclose(out, brute, rtol=1e-13)
    eye = np.eye(6, dtype=np.float32)
    m = rng.normal(size=(6, 4)).astype(np.float32)
    o = np.empty((6, 4), np.float32)
    assert oracle.oracle_matmul(kd.F32, P(eye), P(m), P(o), kd.MatmulSizes(1, 6, 6, 4), 0) == 0
    np.testing.assert_array_equal(o, m)
    # transposed-operand strides give the transposed product
    st = kd.MatmulStrides()
    st.a[:] = [0, 1, 7]
    st.b[:] = [0, 3, 1]
    st.out[:] = [0, 3, 1]
    a2 = a[0].copy()  # [5,7] used as A^T: rows of length 5
    o2 = np.empty((7, 3))
    b2 = rng.normal(size=(5, 3))
    assert oracle.oracle_matmul_strided(kd.F64, P(a2), P(b2), P(o2), kd.MatmulSizes(1, 7, 5, 3), st) == 0
    np.testing.assert_allclose(o2, a2.T @ b2, rtol=1e-13)


def test_integer_wrapping(oracle):
    big = np.array([2**63 - 1, 2**62, -(2**63)], np.int64)
    one = np.array([1, 2, -1], np.int64)
    out = np.zeros(3, np.int64)
    views = [contiguous((3,))] * 3
    for op, want in (("PLUS", [-(2**63), 2**62 + 2, 2**63 - 1]), ("TIMES", [2**63 - 1, -(2**63), -(2**63)]),
                     ("MINUS", [2**63 - 2, 2**62 - 2, -(2**63) + 1])):
        lay = layout_of(oracle.oracle_layout_build, views, [8, 8, 8], [out.ctypes.data, big.ctypes.data, one.ctypes.data])
        assert oracle.oracle_elementwise(kd.OP[op], kd.I64, kd.I64, lay, kd.params()) == 0
        np.testing.assert_array_equal(out, np.array(want, np.int64))
    s = np.zeros(1, np.int64)
    assert oracle.oracle_reduce(kd.REDUCE_SUM, kd.I64, kd.I64, P(s), P(np.array([2**63 - 1, 1], np.int64)), 2, 1) == 0
    assert s[0] == -(2**63)


def test_gelu_slope_against_numerical_derivative_and_kael_autograd(oracle, refdev):
    x = np.linspace(-6, 6, 1001)
    g = np.ones_like(x)
    for op, tanh_form in ((kd.OP["GELU_EXACT_BACKWARD"], 0), (kd.OP["GELU_TANH_BACKWARD"], 1)):
        out = np.empty_like(x)
        views = [contiguous(x.shape)] * 3
        lay = layout_of(oracle.oracle_layout_build, views, [8, 8, 8], [out.ctypes.data, x.ctypes.data, g.ctypes.data])
        assert oracle.oracle_elementwise(op, kd.F64, kd.F64, lay, kd.params()) == 0
        fwd = kd.OP["GELU_TANH" if tanh_form else "GELU_EXACT"]
        h = 1e-5
        vals = []
        for shift in (h, -h):
            xs = x + shift
            y = np.empty_like(x)
            lay2 = layout_of(oracle.oracle_layout_build, [contiguous(x.shape)] * 2, [8, 8], [y.ctypes.data, xs.ctypes.data])
            assert oracle.oracle_elementwise(fwd, kd.F64, kd.F64, lay2, kd.params()) == 0
            vals.append(y)
        np.testing.assert_allclose(out, (vals[0] - vals[1]) / (2 * h), atol=1e-8)
        # kael autograd on the CPU path
        x32 = np.linspace(-4, 4, 257).astype(np.float32)
        g32 = np.random.default_rng(4).normal(size=257).astype(np.float32)
        want = np.empty_like(x32)
        assert refdev.ref_gelu_backward(kd.F32, P(want), P(x32), P(g32), 257, tanh_form) == 0
        got = np.empty_like(x32)
        lay3 = layout_of(oracle.oracle_layout_build, [contiguous((257,))] * 3, [4, 4, 4], [got.ctypes.data, x32.ctypes.data, g32.ctypes.data])
        assert oracle.oracle_elementwise(op, kd.F32, kd.F32, lay3, kd.params()) == 0
        # The slope is a difference of O(0.5) terms that cancels near x = -0.75; contraction into
        # FMA on the reference build moves it by a few float ulps of those terms.
        np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-6 * np.abs(g32).max())


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64])
def test_row_kernels_match_kael_cpu(oracle, refdev, dtype):
    rng = np.random.default_rng(5)
    npd = kd.NUMPY_DTYPE[dtype]
    x = rng.normal(0, 3, (40, 96)).astype(npd)
    for log in (0, 1):
        a, b = np.empty_like(x), np.empty_like(x)
        assert oracle.oracle_softmax_rows(dtype, P(a), P(x), 40, 96, log) == 0
        assert refdev.ref_softmax(dtype, P(b), P(x), 40, 96, log) == 0
        ok, msg = support.golden_close(a, b, 2e-6, 1e-7)
        assert ok, msg
    w, bias = rng.normal(size=96).astype(npd), rng.normal(size=96).astype(npd)
    a, b = np.empty_like(x), np.empty_like(x)
    assert oracle.oracle_standardize_rows(dtype, P(a), P(x), 40, 96, 1e-5, P(w), P(bias)) == 0
    assert refdev.ref_layer_norm(dtype, P(b), P(x), 40, 96, 1e-5, P(w), P(bias)) == 0
    np.testing.assert_array_equal(a, b)
    t = rng.integers(0, 96, 40).astype(np.int64)
    la, lb = np.empty(40, npd), np.empty(40, npd)
    assert oracle.oracle_cross_entropy_rows(dtype, P(la), P(x), P(t), 40, 96) == 0
    assert refdev.ref_cross_entropy(dtype, P(lb), P(x), P(t), 40, 96) == 0
    ok, msg = support.golden_close(la, lb, 2e-6, 1e-7)
    assert ok, msg
    rw = rng.uniform(0.5, 1.5, 40).astype(npd)
    ga, gb = np.empty_like(x), np.empty_like(x)
    assert oracle.oracle_cross_entropy_grad(dtype, P(ga), P(x), P(t), P(rw), 40, 96) == 0
    assert refdev.ref_cross_entropy_grad(dtype, P(gb), P(x), P(t), P(rw), 40, 96) == 0
    ok, msg = support.golden_close(ga, gb, 2e-6, 1e-7)
    assert ok, msg


def test_matmul_two_level_batches_against_numpy_views(oracle):
    """oracle_matmul_strided_heads on attention-shaped views (q[b, h] and k[b, h]^T of a
    [B, T, 3, H, D] store, the output [B, H, T, T]) against numpy's product of the same views:
    exact in wrapping int64 with small values, and a mistaken head / outer stride or batch order
    changes the result."""
    B, T, H, D = 2, 5, 3, 4
    C = H * D
    rng = np.random.default_rng(8)
    qkv = rng.integers(-9, 10, (B, T, 3, H, D)).astype(np.int64)
    q = qkv[:, :, 0].transpose(0, 2, 1, 3)            # [B, H, T, D]
    k = qkv[:, :, 1].transpose(0, 2, 1, 3)
    want = q @ k.transpose(0, 1, 3, 2)                # [B, H, T, T]
    st = kd.MatmulStrides()
    st.a[:] = [T * 3 * C, 3 * C, 1]
    st.b[:] = [T * 3 * C, 1, 3 * C]
    st.out[:] = [H * T * T, T, 1]
    heads = kd.MatmulHeads(H, D, D, T * T)
    # zero padding after the store keeps the mistaken-stride call below inside its buffer
    flat = np.concatenate([qkv.ravel(), np.zeros(2 * T * 3 * C, np.int64)])
    out = np.zeros(B * H * T * T, np.int64)
    assert oracle.oracle_matmul_strided_heads(kd.I64, P(flat), P(flat[C:].copy()), P(out), kd.MatmulSizes(B * H, T, D, T),
                                              st, heads) == 0
    np.testing.assert_array_equal(out.reshape(B, H, T, T), want)
    swapped = kd.MatmulHeads(H, D, D, T * T)
    swapped.a = 3 * C  # the head stride mistaken for the row stride
    assert oracle.oracle_matmul_strided_heads(kd.I64, P(flat), P(flat[C:].copy()), P(out), kd.MatmulSizes(B * H, T, D, T),
                                              st, swapped) == 0
    assert not np.array_equal(out.reshape(B, H, T, T), want)
    assert oracle.oracle_matmul_strided_heads(kd.I64, P(flat), P(flat), P(out), kd.MatmulSizes(5, T, D, T), st, heads) != 0


@pytest.mark.parametrize("count, stride", [(1, 1), (9, 1), (50, 3), (40, 0), (30, -2)])
def test_index_bounds_is_min_and_max(oracle, count, stride):
    """oracle_index_bounds (kael's range check: max and min of the indices) against numpy's
    min / max of the same strided run, with int64's extremes in the run."""
    rng = np.random.default_rng(count)
    span = (count - 1) * abs(stride) + 1
    store = rng.integers(-1000, 1000, span).astype(np.int64)
    if count > 2 and stride != 0:
        store[abs(stride)] = np.iinfo(np.int64).min
        store[2 * abs(stride)] = np.iinfo(np.int64).max
    first = 0 if stride >= 0 else (count - 1) * abs(stride)
    values = store[first + np.arange(count) * stride]
    got = np.zeros(2, np.int64)
    assert oracle.oracle_index_bounds(ctypes.c_void_p(store.ctypes.data + first * 8), count, stride,
                                      support.ptr(got)) == 0
    assert got.tolist() == [values.min(), values.max()]
    assert oracle.oracle_index_bounds(ctypes.c_void_p(store.ctypes.data), 0, 1, support.ptr(got)) != 0

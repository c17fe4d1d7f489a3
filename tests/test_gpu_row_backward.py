"""kd_softmax_rows_backward and kd_standardize_rows_backward against the C oracle (which restates
kael's composed SoftmaxBackward / LogSoftmaxBackward / StandardizeBackward, reference
src/autograd/functions_reduce.cpp:150-192, and is pinned bit for bit to the reference's device
composition in test_oracle_row_backward.py), then through kael's autograd with the optional device
branches against kael's CPU path.

Both sides round every element op to the element type and accumulate the row sums in double; only
the order of those double sums differs, so results agree to within one rounding of a row sum:
|got - want| <= 1e-5 |want| + 1e-6 max|g| max(1, max|y|) for f32 (the reference's f32 tolerance,
tests/support/allclose.h:24, with the absolute term scaled to the operands), 1e-12 for f64.
Shapes: the wave-per-row path (cols % 4 == 0 up to 1024: C4's attention rows of 128 and LayerNorm
rows of 256, GPT-2's 768), the workgroup path (odd widths, rows past 1024, 50257-wide logits rows),
masked (-inf) log-softmax entries, and empty inputs.
"""
import ctypes

import numpy as np
import pytest

import kd
import support

pytestmark = pytest.mark.gpu

P = support.ptr
EPS = 1e-5
SHAPES = [(1, 1), (7, 10), (4096, 128), (4096, 256), (64, 768), (33, 1000), (8, 1024), (5, 1025), (3, 4097),
          (2, 50257), (16384, 128)]


def device_backward(kdb, kind, dtype, x, y, g):
    rows, cols = x.shape
    dx, dy, dg = kdb.to_device(x), kdb.to_device(y), kdb.to_device(g)
    out = kdb.empty(x.shape, x.dtype)
    if kind == "standardize":
        kdb.call("standardize_rows_backward", dtype, out.ptr, dx.ptr, dy.ptr, dg.ptr, rows, cols, EPS)
    else:
        kdb.call("softmax_rows_backward", dtype, out.ptr, dy.ptr, dg.ptr, rows, cols, int(kind == "log_softmax"))
    return out.numpy()


def oracle_forward_backward(oracle, kind, dtype, x, g):
    rows, cols = x.shape
    y = np.empty_like(x)
    out = np.empty_like(x)
    if kind == "standardize":
        assert oracle.oracle_standardize_rows(dtype, P(y), P(x), rows, cols, EPS, None, None) == 0
        assert oracle.oracle_standardize_rows_backward(dtype, P(out), P(x), P(y), P(g), rows, cols, EPS) == 0
    else:
        log = int(kind == "log_softmax")
        assert oracle.oracle_softmax_rows(dtype, P(y), P(x), rows, cols, log) == 0
        assert oracle.oracle_softmax_rows_backward(dtype, P(out), P(y), P(g), rows, cols, log) == 0
    return y, out


def check_close(got, want, g, y, npdtype):
    if npdtype == np.float64:
        scale = np.abs(want).max() + 1e-300
        assert np.abs(got - want).max() <= 1e-12 * scale
        return
    finite_y = np.abs(y[np.isfinite(y)]).max() if np.isfinite(y).any() else 1.0
    atol = 1e-6 * np.abs(g).max() * max(1.0, float(finite_y))
    bad = np.abs(got.astype(np.float64) - want) > 1e-5 * np.abs(want) + atol
    assert not bad.any(), f"{bad.sum()} of {bad.size} beyond tolerance; first {np.argwhere(bad)[0]}"


@pytest.mark.parametrize("npdtype", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("kind", ["softmax", "log_softmax", "standardize"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
def test_row_backward_matches_oracle(kdb, oracle, kind, npdtype, shape):
    if npdtype == np.float64 and shape[0] * shape[1] > (1 << 21):
        pytest.skip("full-size shapes run for f32 only")
    rng = np.random.default_rng(shape[0] * 131 + shape[1])
    x = rng.normal(0, 2, shape).astype(npdtype)
    g = rng.uniform(-1, 1, shape).astype(npdtype)
    dtype = kd.F32 if npdtype == np.float32 else kd.F64
    y, want = oracle_forward_backward(oracle, kind, dtype, x, g)
    got = device_backward(kdb, kind, dtype, x, y, g)
    check_close(got, want, g, y, npdtype)


def test_masked_log_softmax_rows(kdb, oracle):
    """Attention-style masked rows: -inf scores give y = -inf and exp(y) = 0, so those entries
    pass g through unchanged."""
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (64, 128)).astype(np.float32)
    x[:, 65:] = -np.inf
    g = rng.uniform(-1, 1, x.shape).astype(np.float32)
    y, want = oracle_forward_backward(oracle, "log_softmax", kd.F32, x, g)
    got = device_backward(kdb, "log_softmax", kd.F32, x, y, g)
    np.testing.assert_array_equal(got[:, 65:], g[:, 65:])
    check_close(got, want, g, y, np.float32)


def test_empty_and_bad_arguments(kdb):
    z = kdb.empty((1,), np.float32)
    kdb.call("softmax_rows_backward", kd.F32, z.ptr, z.ptr, z.ptr, 0, 5, 0)
    kdb.call("standardize_rows_backward", kd.F32, z.ptr, z.ptr, z.ptr, z.ptr, 3, 0, EPS)
    assert kdb.lib.kd_softmax_rows_backward(kd.I64, z.ptr, z.ptr, z.ptr, 1, 1, 0) != 0
    assert kdb.lib.kd_standardize_rows_backward(kd.F32, z.ptr, z.ptr, z.ptr, z.ptr, -1, 1, EPS) != 0


@pytest.mark.parametrize("kind,index", [("softmax", 0), ("log_softmax", 1), ("standardize", 2)])
def test_through_kael_autograd_matches_cpu(kael_hip_fused, oracle, kind, index):
    """kael's autograd on the MI355X with the optional branches (the backward runs the fused
    kernel) against kael's CPU autograd, and against the oracle fed kael's own forward output."""
    lib = kael_hip_fused
    rng = np.random.default_rng(index)
    x = rng.normal(0, 2, (512, 256)).astype(np.float32)
    g = rng.uniform(-1, 1, x.shape).astype(np.float32)
    dev, y = np.empty_like(x), np.empty_like(x)
    cpu = np.empty_like(x)
    assert lib.ref_row_grad(index, 1, 0, P(x), P(g), 512, 256, EPS, P(dev), P(y)) == 0, support.ref_error(lib)
    assert lib.ref_row_grad(index, 0, 0, P(x), P(g), 512, 256, EPS, P(cpu), None) == 0, support.ref_error(lib)
    assert np.abs(dev.astype(np.float64) - cpu).max() <= 1e-5 * np.abs(cpu).max()
    want = np.empty_like(x)
    if kind == "standardize":
        assert oracle.oracle_standardize_rows_backward(kd.F32, P(want), P(x), P(y), P(g), 512, 256, EPS) == 0
    else:
        assert oracle.oracle_softmax_rows_backward(kd.F32, P(want), P(y), P(g), 512, 256, index) == 0
    check_close(dev, want, g, y, np.float32)

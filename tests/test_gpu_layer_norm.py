"""kd_layer_norm_rows and kd_layer_norm_rows_backward (kael's LayerNorm::forward and its composed
backward in 1 + 2 launches) against the C oracle, which test_oracle_layer_norm.py pins bit for bit to
the reference's device composition; then kael's LayerNorm module with the optional device branch
against kael's CPU path.

Tolerances: the forward as kd_standardize_rows (rtol 1e-5 / atol 1e-6 f32, 1e-12 f64: the device
multiplies by the reciprocal of the scale in double, the oracle divides); the input gradient as
kd_standardize_rows_backward (the row sums in another order); the weight and bias gradients are
column sums in double of the same f32 terms, compared within 1e-6 of the sum of their magnitudes.
Shapes: C4's LayerNorm rows (4096 x 256), GPT-2's (64 x 768), the wave path's limit (8 x 1024), the
workgroup path (odd widths, rows past 1024, rows off 16-byte alignment), one row, no rows.
"""
import numpy as np
import pytest

import kd
import support
from test_gpu_row_backward import check_close

pytestmark = pytest.mark.gpu

P = support.ptr
EPS = 1e-5
# The backward's row groups (a wave loads 4 rows of <= 256 columns, 2 of <= 512, 1 of <= 1024
# before it processes them): 4096 x 256 and 300 x 512 fill them, 200 x 256 and 20000 x 256 leave a
# partial last group, 1 x 256 a group of one row.
SHAPES = [(4096, 256), (64, 768), (8, 1024), (33, 1000), (5, 7), (3, 1030), (1, 256), (300, 512), (200, 256),
          (20000, 256)]


def inputs(rows, cols, npd, seed):
    rng = np.random.default_rng(seed)
    x = rng.normal(0.2, 1.5, (rows, cols)).astype(npd)
    w = rng.normal(1, 0.2, cols).astype(npd)
    b = rng.normal(0, 0.2, cols).astype(npd)
    g = rng.uniform(-1, 1, (rows, cols)).astype(npd)
    return x, w, b, g


def tol(npd):
    return (1e-5, 1e-6) if npd == np.float32 else (1e-12, 1e-14)


def device_forward(kdb, dtype, x, w, b, offset=0):
    rows, cols = x.shape
    npd = x.dtype

    def place(a):
        padded = np.zeros(a.size + offset, npd)
        padded[offset:] = a.ravel()
        return kdb.to_device(padded)

    dx, dw, db = place(x), place(w), place(b)
    out, y = kdb.empty((x.size + offset,), npd), kdb.empty((x.size + offset,), npd)
    s = np.dtype(npd).itemsize * offset
    kdb.call("layer_norm_rows", dtype, out.ptr + s, y.ptr + s, dx.ptr + s, rows, cols, EPS, dw.ptr + s, db.ptr + s)
    return out.numpy()[offset:].reshape(x.shape), y.numpy()[offset:].reshape(x.shape)


def device_backward(kdb, dtype, x, y, g, w, offset=0, columns=True):
    rows, cols = x.shape
    npd = x.dtype

    def place(a):
        padded = np.zeros(a.size + offset, npd)
        padded[offset:] = a.ravel()
        return kdb.to_device(padded)

    dx, dy, dg, dw = place(x), place(y), place(g), place(w)
    gx = kdb.empty((x.size + offset,), npd)
    gw, gb = kdb.empty((cols + offset,), npd), kdb.empty((cols + offset,), npd)
    s = np.dtype(npd).itemsize * offset
    kdb.call("layer_norm_rows_backward", dtype, gx.ptr + s, gw.ptr + s if columns else None,
             gb.ptr + s if columns else None, dx.ptr + s, dy.ptr + s, dg.ptr + s, dw.ptr + s, rows, cols, EPS)
    return gx.numpy()[offset:].reshape(x.shape), gw.numpy()[offset:], gb.numpy()[offset:]


def column_close(got, want, terms):
    bound = 1e-6 * np.abs(terms).sum(axis=0) + 1e-30
    assert np.all(np.abs(got.astype(np.float64) - want.astype(np.float64)) <= bound)


@pytest.mark.parametrize("npd", [np.float32, np.float64], ids=["f32", "f64"])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{r}x{c}" for r, c in SHAPES])
@pytest.mark.parametrize("offset", [0, 1], ids=["aligned", "unaligned"])
def test_layer_norm_matches_oracle(kdb, oracle, npd, shape, offset):
    if npd == np.float64 and shape[0] * shape[1] > (1 << 20):
        pytest.skip("full-size shapes run for f32 only")
    rows, cols = shape
    dtype = kd.F32 if npd == np.float32 else kd.F64
    x, w, b, g = inputs(rows, cols, npd, rows * 3 + cols + offset)
    want_out, want_y = np.empty_like(x), np.empty_like(x)
    assert oracle.oracle_layer_norm_rows(dtype, P(want_out), P(want_y), P(x), rows, cols, EPS, P(w), P(b)) == 0
    out, y = device_forward(kdb, dtype, x, w, b, offset)
    for got, want in ((out, want_out), (y, want_y)):
        ok, msg = support.golden_close(got, want, *tol(npd))
        assert ok, msg
    # the same kernels as kd_standardize_rows: bit for bit
    plain, affine = kdb.empty(x.shape, npd), kdb.empty(x.shape, npd)
    dx, dw, db = kdb.to_device(x), kdb.to_device(w), kdb.to_device(b)
    kdb.call("standardize_rows", dtype, plain.ptr, dx.ptr, rows, cols, EPS, None, None)
    kdb.call("standardize_rows", dtype, affine.ptr, dx.ptr, rows, cols, EPS, dw.ptr, db.ptr)
    if offset == 0:
        np.testing.assert_array_equal(y, plain.numpy())
        np.testing.assert_array_equal(out, affine.numpy())
    # backward from the device's own standardized rows
    gx, gw, gb = device_backward(kdb, dtype, x, y, g, w, offset)
    wx, ww, wb = np.empty_like(x), np.empty_like(w), np.empty_like(w)
    assert oracle.oracle_layer_norm_rows_backward(dtype, P(wx), P(ww), P(wb), P(x), P(y), P(g), P(w), rows, cols,
                                                  EPS) == 0
    check_close(gx, wx, g * w, y, npd)
    column_close(gw, ww, (g * y).astype(np.float64))
    column_close(gb, wb, g.astype(np.float64))


def test_without_column_gradients_and_without_rows(kdb, oracle):
    x, w, b, g = inputs(64, 256, np.float32, 5)
    _, y = device_forward(kdb, kd.F32, x, w, b)
    full, _, _ = device_backward(kdb, kd.F32, x, y, g, w)
    only, _, _ = device_backward(kdb, kd.F32, x, y, g, w, columns=False)
    np.testing.assert_array_equal(full, only)
    gw, gb = kdb.to_device(np.ones(256, np.float32)), kdb.to_device(np.ones(256, np.float32))
    kdb.call("layer_norm_rows_backward", kd.F32, None, gw.ptr, gb.ptr, None, None, None, None, 0, 256, EPS)
    np.testing.assert_array_equal(gw.numpy(), 0)
    np.testing.assert_array_equal(gb.numpy(), 0)
    with pytest.raises(kd.KdError):
        kdb.call("layer_norm_rows", kd.I64, gw.ptr, gw.ptr, gw.ptr, 1, 256, EPS, gw.ptr, gw.ptr)


@pytest.mark.parametrize("shape", [(256, 256), (32, 768), (7, 1030)], ids=["256x256", "32x768", "7x1030"])
def test_kael_layer_norm_module_matches_cpu(kael_hip_fused, shape):
    """kael's nn::LayerNorm through its autograd, on this device with the optional branch (one
    forward launch, one backward node) against kael's CPU path."""
    from test_oracle_layer_norm import kael_layer_norm

    x, w, b, g = inputs(*shape, np.float32, 17)
    cpu = kael_layer_norm(kael_hip_fused, 0, x, w, b, g)
    dev = kael_layer_norm(kael_hip_fused, 1, x, w, b, g)
    for name, got, want in zip(("out", "standardized", "grad_x", "grad_w", "grad_b"), dev, cpu):
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5 * max(1.0, float(np.abs(want).max())), err_msg=name)

"""kd_elementwise / kd_convert / kd_fill against the C oracle, through the C ABI.

Layout cases mirror the reference's device tests (tests/test_cuda.cpp:224-265: contiguous,
transposed, strided, row/column/0-d broadcast) and the C2 benchmark config
(a[4096,4096] + b[4096,1], a.T() + b). Non-transcendental ops must be bit-exact; exp/log/
tanh/erf-based ops use the reference's f32 tolerance rtol 1e-5 / atol 1e-6
(tests/support/allclose.h:24).
"""
import numpy as np
import pytest

import kd
import support
from views import View, assert_same, contiguous, run_both, stepped, transposed

pytestmark = pytest.mark.gpu

TRANSCENDENTAL = {kd.OP[n] for n in ("POWER", "EXP", "LOG", "LOG1P", "EXPM1", "SQRT", "RSQRT", "SIN", "COS",
                                     "TANH", "SIGMOID", "GELU_EXACT", "GELU_TANH", "GELU_EXACT_BACKWARD",
                                     "GELU_TANH_BACKWARD")}
# sqrt and division are correctly rounded on both sides; keep them exact except rsqrt (1/sqrt).
TRANSCENDENTAL.discard(kd.OP["SQRT"])

ALL_OPS = list(range(36)) + [64, 65]


def layout_cases(n_inputs):
    shape = (6, 40)
    cases = {
        "contiguous": [contiguous(shape)] * (n_inputs + 1),
        "transposed": [contiguous(shape)] + [transposed(shape)] * n_inputs,
        "strided": [contiguous(shape)] + [stepped(shape)] * n_inputs,
        "row_broadcast": [contiguous(shape)] + [contiguous((40,))] + [contiguous(shape)] * (n_inputs - 1),
        "col_broadcast": [contiguous(shape)] + [contiguous(shape)] * (n_inputs - 1) + [contiguous((6, 1))],
        "zero_dim": [contiguous(shape)] + [contiguous(shape)] * (n_inputs - 1) + [contiguous(())],
        "odd_1d": [contiguous((1003,))] * (n_inputs + 1),
        "offset_1d": [View((1001,), (1,), 1)] + [View((1001,), (1,), 3)] * n_inputs,
        "batched_3d": [contiguous((3, 5, 70))] + [View((3, 5, 70), (1, 3 * 70, 3))] * n_inputs,
        "transposed_out": [transposed(shape)] + [contiguous(shape)] * n_inputs,
    }
    return cases


def op_out(op, dtype):
    return kd.BOOL if op in kd.COMPARE_OPS else dtype


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
@pytest.mark.parametrize("op", ALL_OPS, ids=lambda o: kd.OPS[o] if o < 36 else ("GELU_EXACT_BWD" if o == 64 else "GELU_TANH_BWD"))
def test_elementwise_matches_oracle_on_every_layout(kdb, oracle, op, dtype):
    if op in kd.FLOATING_OPS and dtype not in (kd.F32, kd.F64):
        pytest.skip("floating op on a non-floating dtype is rejected")
    rng = np.random.default_rng(1000 * op + dtype)
    n_in = kd.op_inputs(op)
    p = kd.params(reals=(-0.5, 0.75), integers=(-3, 20)) if op == kd.OP["CLAMP"] else kd.params(reals=(7.0, 0), integers=(7, 0))
    out_dtype = op_out(op, dtype)
    for name, views in layout_cases(n_in).items():
        got, want = run_both(
            kdb, oracle, views, dtype, out_dtype,
            lambda lay: kdb.call("elementwise", op, out_dtype, dtype, lay, p),
            lambda lay: oracle.oracle_elementwise(op, out_dtype, dtype, lay, p),
            rng, op)
        exact = op not in TRANSCENDENTAL
        tol = (1e-5, 1e-6) if dtype == kd.F32 else (1e-12, 1e-14)
        assert_same(got, want, exact, *tol, what=f"{kd.OPS[op] if op < 36 else op}/{name}")


@pytest.mark.parametrize("out_dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["to_f32", "to_f64", "to_i64", "to_bool"])
@pytest.mark.parametrize("in_dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
def test_convert_is_bit_exact(kdb, oracle, in_dtype, out_dtype):
    rng = np.random.default_rng(17 * in_dtype + out_dtype)
    for name, views in layout_cases(1).items():
        if name in ("row_broadcast", "col_broadcast", "zero_dim"):
            continue
        got, want = run_both(kdb, oracle, views, in_dtype, out_dtype,
                             lambda lay: kdb.call("convert", out_dtype, in_dtype, lay),
                             lambda lay: oracle.oracle_convert(out_dtype, in_dtype, lay), rng)
        assert_same(got, want, True, what=f"convert/{name}")


def test_float_to_int_saturates(kdb, oracle):
    """tests/test_cuda.cpp:482-500: NaN -> 0, 1e300 -> INT64_MAX, and wrapping sums."""
    x = np.array([np.nan, 1e300, -1e300, 2.5, -2.5, 9.3e18, -9.3e18], np.float64)
    dx = kdb.to_device(x)
    out = kdb.empty(x.shape, np.int64)
    lay = kd.element_layout((x.size,), [(8,), (8,)], [out.ptr, dx.ptr])
    kdb.call("convert", kd.I64, kd.F64, lay)
    np.testing.assert_array_equal(out.numpy(), [0, 2**63 - 1, -(2**63), 2, -2, 2**63 - 1, -(2**63)])


def test_int64_clamp_and_masked_fill_keep_every_bit(kdb):
    """tests/test_cuda.cpp:470-480: 2^53+1 survives clamp and masked_fill."""
    large = (1 << 53) + 1
    v = np.array([0, large + 10], np.int64)
    dv = kdb.to_device(v)
    out = kdb.empty(v.shape, np.int64)
    lay = kd.element_layout((2,), [(8,), (8,)], [out.ptr, dv.ptr])
    kdb.call("elementwise", kd.OP["CLAMP"], kd.I64, kd.I64, lay, kd.params(integers=(large, large)))
    np.testing.assert_array_equal(out.numpy(), [large, large])
    mask = kdb.to_device(np.array([1, 0], np.int64))
    lay = kd.element_layout((2,), [(8,), (8,), (8,)], [out.ptr, dv.ptr, mask.ptr])
    kdb.call("elementwise", kd.OP["MASKED_FILL"], kd.I64, kd.I64, lay, kd.params(integers=(large, 0)))
    np.testing.assert_array_equal(out.numpy(), [large, large + 10])


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
@pytest.mark.parametrize("count", [0, 1, 5, 4096, 100003])
def test_fill(kdb, dtype, count):
    npd = kd.NUMPY_DTYPE[dtype]
    value = np.array([-2.75 if npd in (np.float32, np.float64) else (2**53 + 1 if npd == np.int64 else 1)], npd)
    buf = kdb.to_device(np.zeros(count + 3, npd))
    kdb.call("fill", dtype, buf.ptr + npd().itemsize, count, value.ctypes.data)
    got = buf.numpy()
    want = np.zeros(count + 3, npd)
    want[1:1 + count] = value[0]
    np.testing.assert_array_equal(got, want)


# Tile-family shapes: tile counts off a multiple of 8 (the XCD-grouped tile order has a remainder
# path), batches of transposes (grid z > 1), vectorized tiles (rows and cols multiples of the
# vector width) and scalar tiles.
TILE_SHAPES = [(520, 260), (4, 256, 128), (3, 300, 197), (2, 130, 67), (1000, 64)]


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL], ids=["f32", "f64", "i64", "bool"])
@pytest.mark.parametrize("shape", TILE_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_transposed_tiles(kdb, oracle, dtype, shape):
    rng = np.random.default_rng(len(shape) * 1000 + shape[-1] + dtype)
    op = kd.OP["PLUS"]
    cases = {
        "transposed+transposed": [contiguous(shape), transposed(shape), transposed(shape)],
        "transposed+contiguous": [contiguous(shape), transposed(shape), contiguous(shape)],
        "transposed+column": [contiguous(shape), transposed(shape), contiguous(shape[:-1] + (1,))],
    }
    for name, views in cases.items():
        got, want = run_both(kdb, oracle, views, dtype, dtype,
                             lambda lay: kdb.call("elementwise", op, dtype, dtype, lay, kd.params()),
                             lambda lay: oracle.oracle_elementwise(op, dtype, dtype, lay, kd.params()), rng, op)
        assert_same(got, want, True, what=f"{name} {shape}")


C2 = (4096, 4096)


@pytest.mark.parametrize("case", ["add", "mul", "transposed_add"])
def test_c2_config_full_size(kdb, oracle, refdev, case):
    """BASELINE config C2 at its full size and from its recipe (manual_seed(1);
    a = rand({4096,4096}) * 2 - 1, b = rand({4096,1}) * 2 - 1): a (+|*) b and a.T() + b."""
    rng = np.random.default_rng(1)
    flat = np.empty(C2[0] * C2[1] + C2[0], np.float32)
    assert refdev.ref_uniform_pm1(1, flat.size, support.ptr(flat)) == 0, support.ref_error(refdev)
    a, b = flat[:C2[0] * C2[1]], flat[C2[0] * C2[1]:]
    if case == "transposed_add":
        views = [contiguous(C2), transposed(C2), contiguous((C2[0], 1))]
    else:
        views = [contiguous(C2), contiguous(C2), contiguous((C2[0], 1))]
    op = kd.OP["TIMES"] if case == "mul" else kd.OP["PLUS"]
    got, want = run_both(kdb, oracle, views, kd.F32, kd.F32,
                         lambda lay: kdb.call("elementwise", op, kd.F32, kd.F32, lay, kd.params()),
                         lambda lay: oracle.oracle_elementwise(op, kd.F32, kd.F32, lay, kd.params()), rng,
                         inputs=[a, b])
    assert_same(got, want, True, what=case)


def test_empty_is_a_noop(kdb):
    lay = kd.element_layout((0, 3), [(12, 4), (12, 4), (12, 4)], [0, 0, 0])
    lay.count = 0
    kdb.call("elementwise", kd.OP["PLUS"], kd.F32, kd.F32, lay, kd.params())

"""The oracle's optimizer steps (oracle_adam_step / oracle_sgd_step, restating reference
src/optim/optimizer.cpp:60-80 and :93-120) pinned bit for bit on the CPU against kael itself:

- kael's own SGD / Adam / AdamW on CPU tensors (the reference's host kernels, one op at a time);
- kael's composed device path (14 element launches and 7 scalar fills per Adam step) executed by
  the reference's host emulation of its device tasks (src/cuda/backend_fake.cpp);
- kael with the optional device branch (oracle/kael_fused.py) over the oracle, which must take
  the fused entry point and still give the same bits.

Several steps from the same starting point pin the moments too (the parameter after step s
depends on both moments). f32 and f64, with and without weight decay, odd sizes.
"""
import ctypes

import numpy as np
import pytest

import kd
import support

KINDS = {"sgd": 0, "adam": 1, "adamw": 2}


def oracle_steps(oracle, kind, dtype, p0, grads, lr, b1, b2, eps, wd):
    npd = kd.NUMPY_DTYPE[dtype]
    p = p0.copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    for s, g in enumerate(grads, start=1):
        g = np.ascontiguousarray(g, npd)
        if kind == "sgd":
            assert oracle.oracle_sgd_step(dtype, support.ptr(p), support.ptr(g), p.size, lr, wd) == 0
        else:
            assert oracle.oracle_adam_step(dtype, support.ptr(p), support.ptr(g), support.ptr(m), support.ptr(v), p.size,
                                           lr, b1, b2, eps, wd, int(kind == "adamw"), s) == 0
    return p


def kael_steps(lib, kind, device, dtype, p0, grads, lr, b1, b2, eps, wd):
    out = np.empty_like(p0)
    flat = np.ascontiguousarray(np.stack(grads), p0.dtype)
    rc = lib.ref_optim_steps(KINDS[kind], device, 0 if dtype == kd.F32 else 1, p0.size, len(grads), support.ptr(p0),
                             support.ptr(flat), support.ptr(out), lr, b1, b2, eps, wd)
    assert rc == 0, support.ref_error(lib)
    return out


CASES = [(kind, dtype, wd, n) for kind in ("sgd", "adam", "adamw") for dtype in (kd.F32, kd.F64)
         for wd in (0.0, 0.05) for n in (1, 1001)]


def case_inputs(kind, dtype, wd, n, steps=5):
    rng = np.random.default_rng(n + 7 * int(wd > 0) + 13 * list(KINDS).index(kind))
    npd = kd.NUMPY_DTYPE[dtype]
    p0 = rng.normal(0, 1, n).astype(npd)
    grads = [rng.normal(0, 1, n).astype(npd) * npd(10.0 ** -rng.integers(0, 4)) for _ in range(steps)]
    lr = 1e-3 if kind != "sgd" else 0.01
    return p0, grads, (lr, 0.9, 0.999, 1e-8, wd)


@pytest.mark.parametrize("kind,dtype,wd,n", CASES,
                         ids=[f"{k}-{'f32' if d == kd.F32 else 'f64'}-wd{w}-{n}" for k, d, w, n in CASES])
def test_oracle_equals_kael_cpu_and_composed_device_path(oracle, refdev, kind, dtype, wd, n):
    p0, grads, hyper = case_inputs(kind, dtype, wd, n)
    want = oracle_steps(oracle, kind, dtype, p0, grads, *hyper)
    np.testing.assert_array_equal(kael_steps(refdev, kind, 0, dtype, p0, grads, *hyper), want)
    np.testing.assert_array_equal(kael_steps(refdev, kind, 1, dtype, p0, grads, *hyper), want)


def test_fused_branch_takes_the_entry_point_and_keeps_the_bits(oracle, kael_oracle_fused):
    fn = kael_oracle_fused.ref_extension_calls
    fn.restype, fn.argtypes = ctypes.c_longlong, [ctypes.c_int]
    for kind, dtype, wd, n in CASES:
        p0, grads, hyper = case_inputs(kind, dtype, wd, n)
        before = fn(7) + fn(14)  # sgd_step, adam_step_many (one call per step for the one parameter)
        got = kael_steps(kael_oracle_fused, kind, 1, dtype, p0, grads, *hyper)
        assert fn(7) + fn(14) - before == len(grads), (kind, dtype, wd, n)
        np.testing.assert_array_equal(got, oracle_steps(oracle, kind, dtype, p0, grads, *hyper))


def numpy_adam(p0, grads, lr, b1, b2, eps, contract_first_moment=False):
    """Adam in numpy float32, one rounding per kael op; optionally with the first-moment update
    contracted (m * b1 kept exact before adding), the kind of slip an FMA would make."""
    f = np.float32
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for s, g in enumerate(grads, start=1):
        if contract_first_moment:
            m = (m.astype(np.float64) * np.float64(f(b1)) + (g * f(1.0 - b1)).astype(np.float64)).astype(f)
        else:
            m = m * f(b1) + g * f(1.0 - b1)
        v = v * f(b2) + (g * g) * f(1.0 - b2)
        denominator = np.sqrt(v / f(1.0 - b2 ** s)) + f(eps)
        p = p - (m / f(1.0 - b1 ** s)) / denominator * f(lr)
    return p


def test_planted_rounding_change_is_caught(refdev):
    """The bit-exact comparison sees one dropped rounding: a numpy restatement with one rounding
    per kael op equals kael's CPU Adam, and the same with the first-moment update contracted
    (as an FMA would compute it) does not."""
    p0, grads, (lr, b1, b2, eps, _) = case_inputs("adam", kd.F32, 0.0, 1001)
    want = kael_steps(refdev, "adam", 0, kd.F32, p0, grads, lr, b1, b2, eps, 0.0)
    np.testing.assert_array_equal(numpy_adam(p0, grads, lr, b1, b2, eps), want)
    assert not np.array_equal(numpy_adam(p0, grads, lr, b1, b2, eps, contract_first_moment=True), want)

"""kd_adam_step / kd_sgd_step (one launch per parameter tensor) against the oracle, bit for bit,
and against kael's own optimizers on this device (reference src/optim/optimizer.cpp:60-80,
:93-120): unmodified kael composes the update from element ops on the MI355X, and kael with the
optional device branch (oracle/kael_fused.py) calls these kernels; both must give the bits of
kael's CPU path. The oracle is pinned to kael's CPU optimizers in test_oracle_optim.py.
"""
import numpy as np
import pytest

import kd
import support
from test_oracle_optim import CASES, KINDS, case_inputs, kael_steps, oracle_steps

pytestmark = pytest.mark.gpu


def device_steps(kdb, kind, dtype, p0, grads, lr, b1, b2, eps, wd, offset=0):
    """The same steps through the C ABI; `offset` elements shift every buffer off 16-byte
    alignment (the scalar path)."""
    npd = kd.NUMPY_DTYPE[dtype]
    n = p0.size

    def buffer(values):
        padded = np.zeros(n + offset, npd)
        padded[offset:] = values
        return kdb.to_device(padded)

    size = np.dtype(npd).itemsize
    p, m, v = buffer(p0), buffer(np.zeros(n)), buffer(np.zeros(n))
    for s, g in enumerate(grads, start=1):
        dg = buffer(g)
        if kind == "sgd":
            kdb.call("sgd_step", dtype, p.ptr + offset * size, dg.ptr + offset * size, n, lr, wd)
        else:
            kdb.call("adam_step", dtype, p.ptr + offset * size, dg.ptr + offset * size, m.ptr + offset * size,
                     v.ptr + offset * size, n, lr, b1, b2, eps, wd, int(kind == "adamw"), s)
    return p.numpy()[offset:]


@pytest.mark.parametrize("kind,dtype,wd,n", CASES,
                         ids=[f"{k}-{'f32' if d == kd.F32 else 'f64'}-wd{w}-{n}" for k, d, w, n in CASES])
def test_kernels_equal_the_oracle(kdb, oracle, kind, dtype, wd, n):
    p0, grads, hyper = case_inputs(kind, dtype, wd, n)
    want = oracle_steps(oracle, kind, dtype, p0, grads, *hyper)
    np.testing.assert_array_equal(device_steps(kdb, kind, dtype, p0, grads, *hyper), want)
    np.testing.assert_array_equal(device_steps(kdb, kind, dtype, p0, grads, *hyper, offset=1), want)


@pytest.mark.parametrize("kind", list(KINDS))
def test_large_tensor_vector_path(kdb, oracle, kind):
    """3 145 728 elements (C4's largest weight is 768 x 256 = 196 608; this is GPT-2's fc1), f32."""
    p0, grads, hyper = case_inputs(kind, kd.F32, 0.01, 3 * 1024 * 1024 + 3, steps=3)
    want = oracle_steps(oracle, kind, kd.F32, p0, grads, *hyper)
    np.testing.assert_array_equal(device_steps(kdb, kind, kd.F32, p0, grads, *hyper), want)


def test_kael_composed_and_fused_paths_give_kael_cpu_bits(kael_hip, kael_hip_fused):
    for kind, dtype, wd, n in CASES:
        p0, grads, hyper = case_inputs(kind, dtype, wd, n)
        cpu = kael_steps(kael_hip, kind, 0, dtype, p0, grads, *hyper)
        np.testing.assert_array_equal(kael_steps(kael_hip, kind, 1, dtype, p0, grads, *hyper), cpu)
        np.testing.assert_array_equal(kael_steps(kael_hip_fused, kind, 1, dtype, p0, grads, *hyper), cpu)


def test_rejects_bad_arguments(kdb):
    x = kdb.to_device(np.zeros(4, np.float32))
    with pytest.raises(kd.KdError):
        kdb.call("adam_step", kd.I64, x.ptr, x.ptr, x.ptr, x.ptr, 4, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0, 1)
    with pytest.raises(kd.KdError):
        kdb.call("adam_step", kd.F32, x.ptr, x.ptr, x.ptr, x.ptr, 4, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0, 0)
    with pytest.raises(kd.KdError):
        kdb.call("sgd_step", kd.BOOL, x.ptr, x.ptr, 4, 0.01, 0.0)

"""kd_adam_step / kd_sgd_step (one launch per parameter tensor) and kd_adam_step_many (one launch
per 32 tensors) against the oracle, bit for bit,
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


MANY_SIZES = [0, 1, 3, 4, 5, 255, 1024, 1025, 2048, 4097, 196608, 65536 + 7]


def many_tables(kdb, dtype, sizes, offsets, steps, seed):
    """Device buffers for kd_adam_step_many: param, grad and both moments per tensor, each shifted
    `offsets[i]` elements off 16-byte alignment; returns (table, buffers, host copies)."""
    npd = kd.NUMPY_DTYPE[dtype]
    size = np.dtype(npd).itemsize
    rng = np.random.default_rng(seed)
    table = (kd.AdamTensor * len(sizes))()
    buffers, hosts = [], []
    for i, (n, off, step) in enumerate(zip(sizes, offsets, steps)):
        arrays = [rng.normal(0, 1, n).astype(npd), rng.normal(0, 0.1, n).astype(npd),
                  rng.normal(0, 0.01, n).astype(npd), rng.uniform(0, 0.001, n).astype(npd)]
        devs = []
        for a in arrays:
            padded = np.zeros(n + off + 1, npd)
            padded[off:off + n] = a
            devs.append(kdb.to_device(padded))
        table[i] = kd.AdamTensor(*(d.ptr + off * size for d in devs), n, step)
        buffers.append((devs, off, n))
        hosts.append(arrays)
    return table, buffers, hosts


def read_back(buffers, role):
    return [devs[role].numpy()[off:off + n] for devs, off, n in buffers]


@pytest.mark.parametrize("decay", ["none", "coupled", "decoupled"])
@pytest.mark.parametrize("dtype", [kd.F32, kd.F64], ids=["f32", "f64"])
def test_many_equals_one_call_per_tensor(kdb, oracle, decay, dtype):
    """70 tensors (three launches of up to 32), sizes from empty to 196 608, a third of them off
    16-byte alignment, each with its own step count: the bits of kd_adam_step per tensor and of the
    oracle, for param and both moments."""
    sizes = [MANY_SIZES[i % len(MANY_SIZES)] for i in range(70)]
    offsets = [1 if i % 3 == 1 else 0 for i in range(70)]
    steps = [1 + (i * 7) % 13 for i in range(70)]
    lr, b1, b2, eps = 3e-3, 0.9, 0.995, 1e-8
    wd = 0.0 if decay == "none" else 0.01
    decoupled = int(decay == "decoupled")
    table, many, hosts = many_tables(kdb, dtype, sizes, offsets, steps, seed=dtype)
    kdb.call("adam_step_many", dtype, table, len(sizes), lr, b1, b2, eps, wd, decoupled)
    t1, single, _ = many_tables(kdb, dtype, sizes, offsets, steps, seed=dtype)
    for i in range(len(sizes)):
        x = t1[i]
        kdb.call("adam_step", dtype, x.param, x.grad, x.first, x.second, x.count, lr, b1, b2, eps, wd, decoupled, x.step)
    for role in (0, 2, 3):
        for i, (a, b) in enumerate(zip(read_back(many, role), read_back(single, role))):
            np.testing.assert_array_equal(a, b, err_msg=f"tensor {i} role {role}")
    params, seconds = read_back(many, 0), read_back(many, 3)
    for i, (p, g, m, v) in enumerate(hosts):
        assert oracle.oracle_adam_step(dtype, support.ptr(p), support.ptr(g), support.ptr(m), support.ptr(v), p.size,
                                       lr, b1, b2, eps, wd, decoupled, steps[i]) == 0
        np.testing.assert_array_equal(params[i], p, err_msg=f"tensor {i} vs oracle")
        np.testing.assert_array_equal(seconds[i], v, err_msg=f"tensor {i} vs oracle")


def test_many_streams_a_large_tensor(kdb, oracle):
    """A tensor past the 32 MiB streaming threshold (nontemporal path) between two small ones."""
    sizes, offsets, steps = [7, 8 * 1024 * 1024 + 5, 300], [0, 0, 1], [2, 3, 4]
    table, many, hosts = many_tables(kdb, kd.F32, sizes, offsets, steps, seed=5)
    kdb.call("adam_step_many", kd.F32, table, 3, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0)
    params, firsts = read_back(many, 0), read_back(many, 2)
    for i, (p, g, m, v) in enumerate(hosts):
        assert oracle.oracle_adam_step(kd.F32, support.ptr(p), support.ptr(g), support.ptr(m), support.ptr(v), p.size,
                                       1e-3, 0.9, 0.999, 1e-8, 0.0, 0, steps[i]) == 0
        np.testing.assert_array_equal(params[i], p)
        np.testing.assert_array_equal(firsts[i], m)


def test_many_rejects_overlap_and_bad_entries(kdb):
    table, many, _ = many_tables(kdb, kd.F32, [16, 16], [0, 0], [1, 1], seed=9)
    shared = (kd.AdamTensor * 2)(table[0], table[1])
    shared[1].second = table[0].first + 32  # tensor 1 writes inside tensor 0's first moment
    with pytest.raises(kd.KdError):
        kdb.call("adam_step_many", kd.F32, shared, 2, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0)
    before = read_back(many, 0)
    same_grad = (kd.AdamTensor * 2)(table[0], table[1])
    same_grad[1].grad = table[0].grad  # a gradient read by two tensors is fine
    kdb.call("adam_step_many", kd.F32, same_grad, 2, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0)
    assert not np.array_equal(read_back(many, 0)[1], before[1])
    bad = (kd.AdamTensor * 1)(table[0])
    bad[0].step = 0
    with pytest.raises(kd.KdError):
        kdb.call("adam_step_many", kd.F32, bad, 1, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0)
    with pytest.raises(kd.KdError):
        kdb.call("adam_step_many", kd.I64, table, 2, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0)
    kdb.call("adam_step_many", kd.F32, None, 0, 1e-3, 0.9, 0.999, 1e-8, 0.0, 0)  # nothing to do

"""kd_bernoulli and kd_dropout (kael's bernoulli mask and dropout drawn on the device; reference
src/random.cpp:66-110, src/nn/functional.cpp:32-39) against the oracle, bit for bit: the output,
the mask and the generator state after the call, for counts around the 312-word twist blocks, start
positions inside a block, up to C4-sized activations (32 x 128 x 256 and 32 x 128 x 1024), both
float types and every mask dtype. Then kael itself on the MI355X: its dropout through the optional
device branch (libkael_hip_fused.so) and unmodified (libkael_hip.so, the host mask copied over)
against kael's CPU path, output, input gradient and the generator's next draw.
"""
import ctypes

import numpy as np
import pytest

import kd
import support
from test_oracle_random import draws, dropout_input, kael_dropout, same, seeded

pytestmark = pytest.mark.gpu

P = support.ptr
DT = {np.float32: kd.F32, np.float64: kd.F64}
COUNTS = [1, 155, 311, 312, 313, 624, 1000, 4099, 100003, 32 * 128 * 256]
STARTS = [(0, 0), (3, 1), (5, 311), (7, 312), (9, 5000)]  # (seed, draws before the call)


def start_state(oracle, seed, skip):
    state = seeded(oracle, seed)
    draws(oracle, state, skip)
    return state


@pytest.mark.parametrize("npt", [np.float32, np.float64])
@pytest.mark.parametrize("count", COUNTS)
@pytest.mark.parametrize("seed, skip", STARTS)
def test_dropout_against_oracle(kdb, oracle, npt, count, seed, skip):
    x = dropout_input(count, npt, seed)
    keep = 0.8 if count % 2 else 0.35
    want, want_mask = np.zeros_like(x), np.zeros_like(x)
    want_state = start_state(oracle, seed, skip)
    assert oracle.oracle_dropout(DT[npt], P(want), P(want_mask), P(x), count, keep, P(want_state)) == 0
    state = start_state(oracle, seed, skip)
    dx, dout, dmask = kdb.to_device(x), kdb.empty(x.shape, npt), kdb.empty(x.shape, npt)
    kdb.check(kdb.lib.kd_dropout(DT[npt], dout.ptr, dmask.ptr, dx.ptr, count, keep, P(state)), "kd_dropout")
    assert same(dout.numpy(), want)
    np.testing.assert_array_equal(dmask.numpy(), want_mask)
    np.testing.assert_array_equal(state, want_state)


@pytest.mark.parametrize("dtype, npt", [(kd.F32, np.float32), (kd.F64, np.float64), (kd.I64, np.int64),
                                        (kd.BOOL, np.bool_)])
@pytest.mark.parametrize("count", [1, 312, 313, 100003, 32 * 128 * 1024])
def test_bernoulli_against_oracle(kdb, oracle, dtype, npt, count):
    p = 0.3
    want = np.zeros(count, npt)
    want_state = start_state(oracle, 21, 77)
    assert oracle.oracle_bernoulli(dtype, P(want), count, p, P(want_state)) == 0
    state = start_state(oracle, 21, 77)
    dout = kdb.empty((count,), npt)
    kdb.check(kdb.lib.kd_bernoulli(dtype, dout.ptr, count, p, P(state)), "kd_bernoulli")
    np.testing.assert_array_equal(dout.numpy(), want)
    np.testing.assert_array_equal(state, want_state)
    if count >= 1000:
        assert abs(np.count_nonzero(want) / count - p) < 0.01


def test_consecutive_calls_continue_the_stream(kdb, oracle):
    """Three calls in a row (in place, no mask output) equal one oracle pass over the three inputs."""
    sizes = [1000, 311, 70001]
    xs = [dropout_input(n, np.float32, i) for i, n in enumerate(sizes)]
    want_state = start_state(oracle, 2, 0)
    wants = []
    for x in xs:
        w = np.zeros_like(x)
        assert oracle.oracle_dropout(kd.F32, P(w), None, P(x), x.size, 0.6, P(want_state)) == 0
        wants.append(w)
    state = start_state(oracle, 2, 0)
    for x, w in zip(xs, wants):
        d = kdb.to_device(x)
        kdb.check(kdb.lib.kd_dropout(kd.F32, d.ptr, None, d.ptr, x.size, 0.6, P(state)), "kd_dropout")
        assert same(d.numpy(), w)
    np.testing.assert_array_equal(state, want_state)


@pytest.mark.parametrize("variant", ["hip", "hip_fused"])
@pytest.mark.parametrize("npt, count", [(np.float32, 32 * 128 * 256), (np.float64, 100003), (np.float32, 5)])
def test_kael_dropout_on_the_device(request, variant, npt, count):
    """kael's nn::functional::dropout of a device tensor (p 0.1, C4's activation size) against kael's
    CPU path: output, input gradient of sum(dropout(x) * g), and the generator's next draw."""
    lib = request.getfixturevalue("kael_" + variant)
    x = dropout_input(count, npt, 3)
    g = np.random.default_rng(4).normal(0, 1, count).astype(npt)
    want, want_next, want_grad = kael_dropout(lib, 0, 3, 1234, x, 0.1, g)
    got, got_next, got_grad = kael_dropout(lib, 1, 3, 1234, x, 0.1, g)
    assert same(got, want)
    assert same(got_grad, want_grad)
    assert got_next == want_next

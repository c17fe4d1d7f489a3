"""The oracle's restatement of kael's random draws (std::mt19937_64 through libstdc++'s
uniform_real_distribution<double>; reference src/random.cpp:66-110) and of dropout
(src/nn/functional.cpp:32-39), pinned on the CPU:

  - the C++ standard's required value: the 10000th draw of a default-constructed std::mt19937_64
    is 9981545732273789042 ([rand.predef]);
  - libstdc++ itself (oracle/_ref shim): raw draws after any number of earlier draws, and the
    engine's stream form (312 words, then the position) after them, which is the state layout
    kd_bernoulli / kd_dropout take;
  - kael's own bernoulli and dropout on the CPU path (f32 / f64, masks of every dtype, inputs with
    infinities, NaN and signed zeros), and the generator's next draw after them;
  - kael's dropout with the C oracle as the device, unmodified and through the optional device
    branch (the branch must run), output and input gradient equal to the CPU path's.

kd_mt19937_64_seed (host code of the product library) is checked against libstdc++ here too, and
kd_bernoulli / kd_dropout reject bad arguments before touching a device.
"""
import ctypes

import numpy as np
import pytest

import kd
import support

P = support.ptr
DT = {np.float32: kd.F32, np.float64: kd.F64}


@pytest.fixture(scope="module")
def cpu_kael():
    return support.load_ref("ref")


def seeded(oracle, seed):
    state = np.zeros(313, np.uint64)
    oracle.oracle_mt19937_64_seed(P(state), seed)
    return state


def draws(oracle, state, count):
    out = np.zeros(count, np.uint64)
    assert oracle.oracle_mt19937_64_draws(P(state), count, P(out)) == 0
    return out


def libstdcxx(cpu_kael, seed, skip, count):
    out, state = np.zeros(max(count, 1), np.uint64), np.zeros(313, np.uint64)
    assert cpu_kael.ref_mt_draws(seed, skip, count, P(out), P(state)) == 0, support.ref_error(cpu_kael)
    return out[:count], state


def test_standard_required_value(oracle):
    state = seeded(oracle, 5489)  # std::mt19937_64's default seed
    assert int(draws(oracle, state, 10000)[-1]) == 9981545732273789042


@pytest.mark.parametrize("seed, skip, count", [(0, 0, 5), (3, 0, 700), (4, 311, 2), (4, 312, 1), (1, 1000, 937),
                                               (2**64 - 1, 5, 313)])
def test_draws_and_state_layout_against_libstdcxx(oracle, cpu_kael, seed, skip, count):
    want, want_state = libstdcxx(cpu_kael, seed, skip, count)
    state = seeded(oracle, seed)
    draws(oracle, state, skip)
    np.testing.assert_array_equal(draws(oracle, state, count), want)
    np.testing.assert_array_equal(state, want_state)


@pytest.mark.parametrize("seed", [0, 3, 5489, 2**63 + 11])
def test_product_seed_matches_libstdcxx(seed, cpu_kael):
    lib = kd.Backend().lib  # host code only: no device needed
    state = np.zeros(313, np.uint64)
    lib.kd_mt19937_64_seed(P(state), seed)
    _, want = libstdcxx(cpu_kael, seed, 0, 0)
    np.testing.assert_array_equal(state, want)


def uniform_continuation(oracle, state):
    """The next kael::rand F64 value from this state (generate_canonical of one draw)."""
    x = float(int(draws(oracle, state, 1)[0]))  # Python rounds an integer to the nearest double
    u = x / 2.0**64
    return np.nextafter(1.0, 0.0) if u >= 1.0 else u


@pytest.mark.parametrize("dtype", [kd.F32, kd.F64, kd.I64, kd.BOOL])
@pytest.mark.parametrize("seed, skip, count, p", [(0, 0, 1000, 0.3), (7, 311, 2000, 0.9), (9, 12, 313, 1.0),
                                                  (9, 12, 313, 0.0), (5, 0, 1, 0.5)])
def test_bernoulli_against_kael(oracle, cpu_kael, dtype, seed, skip, count, p):
    npt = {kd.F32: np.float32, kd.F64: np.float64, kd.I64: np.int64, kd.BOOL: np.bool_}[dtype]
    want, nxt = np.zeros(count, npt), ctypes.c_double()
    assert cpu_kael.ref_bernoulli(seed, skip, dtype, count, p, P(want), ctypes.byref(nxt)) == 0, \
        support.ref_error(cpu_kael)
    state = seeded(oracle, seed)
    draws(oracle, state, skip)
    got = np.zeros(count, npt)
    assert oracle.oracle_bernoulli(dtype, P(got), count, p, P(state)) == 0
    np.testing.assert_array_equal(got, want)
    assert uniform_continuation(oracle, state) == nxt.value
    if 0.0 < p < 1.0 and count >= 1000:
        assert 0 < int(np.count_nonzero(want)) < count


def dropout_input(count, npt, seed=0):
    x = np.random.default_rng(seed).normal(0, 2, count).astype(npt)
    specials = np.array([np.inf, -np.inf, np.nan, -0.0, 0.0, -1.5, 3.0e38 if npt is np.float32 else 1e300], npt)
    x[:len(specials)] = specials[:count]
    return x


def same(a, b):
    """Equal values, NaN equal to NaN (the sign and payload of a NaN made by inf * 0 are not fixed)."""
    return np.array_equal(a, b, equal_nan=True) and np.array_equal(np.signbit(a) & ~np.isnan(a),
                                                                  np.signbit(b) & ~np.isnan(b))


def kael_dropout(lib, device, seed, skip, x, p, g=None):
    out, nxt = np.zeros_like(x), ctypes.c_double()
    grad = np.zeros_like(x) if g is not None else None
    assert lib.ref_dropout(device, seed, skip, DT[x.dtype.type], P(x), x.size, p, P(out), ctypes.byref(nxt),
                           P(g) if g is not None else None, P(grad) if g is not None else None) == 0, \
        support.ref_error(lib)
    return out, nxt.value, grad


@pytest.mark.parametrize("npt", [np.float32, np.float64])
@pytest.mark.parametrize("seed, skip, count, p", [(0, 0, 1000, 0.1), (3, 100, 5000, 0.5), (4, 311, 700, 0.9),
                                                  (8, 0, 7, 0.25)])
def test_dropout_against_kael(oracle, cpu_kael, npt, seed, skip, count, p):
    x = dropout_input(count, npt, seed)
    want, nxt, _ = kael_dropout(cpu_kael, 0, seed, skip, x, p)
    state = seeded(oracle, seed)
    draws(oracle, state, skip)
    got, mask = np.zeros_like(x), np.zeros_like(x)
    assert oracle.oracle_dropout(DT[npt], P(got), P(mask), P(x), count, 1.0 - p, P(state)) == 0
    assert same(got, want)
    assert set(np.unique(mask)) <= {0.0, 1.0}
    assert uniform_continuation(oracle, state) == nxt


@pytest.mark.parametrize("variant", ["oracle", "oracle_fused"])
@pytest.mark.parametrize("npt", [np.float32, np.float64])
def test_dropout_on_the_oracle_device(request, cpu_kael, variant, npt):
    """kael's dropout with the C oracle as the device: unmodified (the host mask copied over) and
    through the device branch (kael::device::dropout, counted): output, input gradient and the
    generator's next draw equal to the CPU path's."""
    lib = request.getfixturevalue("kael_" + variant)
    x = dropout_input(3000, npt, 5)
    g = np.random.default_rng(6).normal(0, 1, x.size).astype(npt)
    want, want_next, want_grad = kael_dropout(lib, 0, 11, 17, x, 0.3, g)
    fn = lib.ref_extension_calls
    fn.restype, fn.argtypes = ctypes.c_longlong, [ctypes.c_int]
    before = fn(22) if variant == "oracle_fused" else 0
    got, got_next, got_grad = kael_dropout(lib, 1, 11, 17, x, 0.3, g)
    if variant == "oracle_fused":
        assert fn(22) == before + 1
    assert same(got, want) and same(got_grad, want_grad)
    assert got_next == want_next


def test_entry_points_reject_bad_arguments():
    lib = kd.Backend().lib
    state = np.zeros(313, np.uint64)
    lib.kd_mt19937_64_seed(P(state), 1)
    buf = np.zeros(4, np.float32)
    assert lib.kd_dropout(kd.F32, P(buf), None, P(buf), 4, 0.0, P(state)) == -1  # keep must be > 0
    assert lib.kd_dropout(kd.F32, P(buf), None, P(buf), 4, 1.5, P(state)) == -1
    assert lib.kd_dropout(kd.I64, P(buf), None, P(buf), 4, 0.5, P(state)) == -1
    assert lib.kd_bernoulli(kd.F32, P(buf), 4, -0.1, P(state)) == -1
    assert lib.kd_bernoulli(kd.F32, P(buf), -1, 0.5, P(state)) == -1
    bad = state.copy()
    bad[312] = 313
    assert lib.kd_bernoulli(kd.F32, P(buf), 4, 0.5, P(bad)) == -1
    assert lib.kd_dropout(kd.F32, P(buf), None, P(buf), 4, 0.5, None) == -1
    assert lib.kd_dropout(kd.F32, P(buf), None, P(buf), 0, 0.5, P(state)) == 0  # empty: nothing to do

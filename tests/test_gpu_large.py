"""Element counts above 2^31 (64-bit index paths): the elementwise nd64 kernel (IS_ZERO
of bool is logical not), a reduction whose single chunk is longer than 2^31, and argmax
positions past 2^31. Bool data (1 byte per element) keeps each buffer near 2 GiB; results
are exact.
"""
import numpy as np
import pytest

import kd

pytestmark = pytest.mark.gpu

N = (1 << 31) + 7


@pytest.fixture(scope="module")
def big_bool(kdb):
    rng = np.random.default_rng(0)
    # A sparse pattern is enough and cheap to generate: blocks of ones at a few offsets.
    host = np.zeros(N, np.bool_)
    for start in (0, 12345, (1 << 31) - 3, N - 5):
        host[start:start + 4] = True
    host[rng.integers(0, N, 1000)] = True
    dev = kdb.to_device(host)
    yield host, dev
    del dev


def test_elementwise_is_zero_over_2_pow_31_elements(kdb, big_bool):
    host, dev = big_bool
    out = kdb.empty((N,), np.bool_)
    lay = kd.element_layout((N,), [(1,), (1,)], [out.ptr, dev.ptr])
    kdb.call("elementwise", kd.OP["IS_ZERO"], kd.BOOL, kd.BOOL, lay, kd.params())
    got = out.numpy()
    np.testing.assert_array_equal(got, ~host)


def test_sum_of_a_chunk_longer_than_2_pow_31(kdb, big_bool):
    host, dev = big_bool
    res = kdb.empty((1,), np.int64)
    kdb.call("reduce", kd.REDUCE_SUM, kd.I64, kd.BOOL, res.ptr, dev.ptr, N, 1)
    assert int(res.numpy()[0]) == int(np.count_nonzero(host))


def test_argmax_position_past_2_pow_31(kdb):
    host = np.zeros(N, np.bool_)
    host[N - 2] = True
    dev = kdb.to_device(host)
    idx = kdb.empty((1,), np.int64)
    kdb.call("arg_reduce", 1, kd.BOOL, idx.ptr, dev.ptr, N, 1)
    assert int(idx.numpy()[0]) == N - 2
    kdb.call("arg_reduce", 0, kd.BOOL, idx.ptr, dev.ptr, N, 1)
    assert int(idx.numpy()[0]) == 0

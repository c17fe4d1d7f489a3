"""The gradients of Linear-shaped products (y = x . W^T, x [B, M, K], W [N, K]; reference
src/nn/layers.cpp:42-43, MatmulBackward src/autograd/functions_linalg.cpp:29-49) through kael's
optional device branches with the C oracle as the device: the weight gradient's fold over the batch
(one product X_flat^T . g_flat) and the strided products, element by element against kael's CPU
path (the reference's f32 device tolerance 1e-4 + 1e-4 |cpu|, tests/test_cuda.cpp:40-43). The
fold branch must run (the strided-product counter moves) and an empty last dim must fall back to
kael's own path.
"""
import ctypes
import os

import numpy as np
import pytest

import support
from test_gpu_kael_gradients import SELECT_CASES, assert_reference_close, linear_grads, select_grads

SHAPES = [(3, 37, 53, 29), (5, 1, 7, 3), (2, 30, 64, 48), (4, 16, 32, 24)]


@pytest.mark.parametrize("shape", SHAPES, ids=["x".join(map(str, s)) for s in SHAPES])
def test_linear_gradients_through_the_fused_branches(kael_oracle_fused, shape):
    lib = kael_oracle_fused
    fn = lib.ref_extension_calls
    fn.restype, fn.argtypes = ctypes.c_longlong, [ctypes.c_int]
    cpu_w, cpu_x = linear_grads(lib, 0, shape)
    before = fn(5)  # matmul_strided
    dev_w, dev_x = linear_grads(lib, 1, shape)
    assert fn(5) > before
    assert_reference_close(dev_w, cpu_w, "W.grad")
    assert_reference_close(dev_x, cpu_x, "x.grad")


@pytest.mark.parametrize("shape", [(2, 3, 0, 4), (2, 3, 5, 0)], ids=["k0", "n0"])
def test_empty_last_dim_keeps_kaels_path(kael_oracle_fused, shape):
    b, m, k, n = shape
    wg, xg = np.ones((n, k), np.float32), np.ones((b, m, k), np.float32)
    assert kael_oracle_fused.ref_linear_grads(1, b, m, k, n, 3, support.ptr(wg), support.ptr(xg)) == 0, \
        support.ref_error(kael_oracle_fused)
    assert not wg.any() and not xg.any()


@pytest.mark.parametrize("shape", [(3, 37, 53, 29), (2, 1, 7, 3), (4, 16, 32, 24)], ids=["3x37x53x29", "2x1x7x3", "4x16x32x24"])
def test_head_gradients_through_the_fused_branches(kael_oracle_fused, shape):
    """The tied head's weight . h^T with the left-operand gradient folded over the batch (one
    product) against kael's CPU path, on the oracle device."""
    from test_gpu_kael_gradients import head_grads

    lib = kael_oracle_fused
    cpu_w, cpu_h = head_grads(lib, 0, shape)
    dev_w, dev_h = head_grads(lib, 1, shape)
    assert_reference_close(dev_w, cpu_w, "W.grad")
    assert_reference_close(dev_h, cpu_h, "h.grad")


@pytest.mark.parametrize("shape", [(2, 3, 0, 4), (2, 0, 5, 4), (2, 3, 5, 0)], ids=["k0", "m0", "n0"])
def test_head_empty_dims_keep_kaels_path(kael_oracle_fused, shape):
    b, m, k, n = shape
    wg, hg = np.ones((n, k), np.float32), np.ones((b, m, k), np.float32)
    assert kael_oracle_fused.ref_head_grads(1, b, m, k, n, 3, support.ptr(wg), support.ptr(hg)) == 0, \
        support.ref_error(kael_oracle_fused)
    assert not wg.any() and not hg.any()


@pytest.mark.parametrize("which", range(len(SELECT_CASES)), ids=SELECT_CASES)
def test_select_gradients_through_the_fused_branches(kael_oracle_fused, which):
    """Select gradients on the oracle device equal kael's CPU path value for value, including the
    slices no select reached (zeros), repeated indices (summed), gradients of the whole tensor
    mixed in, a retained intermediate and anomaly detection."""
    cpu_x, cpu_p = select_grads(kael_oracle_fused, 0, which)
    dev_x, dev_p = select_grads(kael_oracle_fused, 1, which)
    assert np.array_equal(dev_x, cpu_x) and np.array_equal(dev_p, cpu_p)
    if SELECT_CASES[which] in ("two_of_three", "same_index_twice"):
        # one slice of dim 2 has no select: its gradient is zero
        assert not cpu_x.reshape(2, 3, 3, 4)[:, :, 1 if which == 1 else 2].any()


def test_select_gradients_reject_unknown_case(kael_oracle_fused):
    xg, pg = np.empty(72, np.float32), np.empty(72, np.float32)
    assert kael_oracle_fused.ref_select_grads(1, 99, 1, support.ptr(xg), support.ptr(pg)) != 0


def test_select_gradients_with_the_graph_retained_accumulate(kael_oracle_fused):
    """Backward twice over the same graph (retain_graph): each pass writes its own select gradients,
    so x.grad is exactly twice one pass's (g + g rounds to 2g)."""
    once, _ = select_grads(kael_oracle_fused, 1, SELECT_CASES.index("attention_split"))
    twice, _ = select_grads(kael_oracle_fused, 1, SELECT_CASES.index("retained_graph_twice"))
    assert np.array_equal(twice, 2 * once)


SMALL_GPT = (11, 16, 2, 2, 8, 3)  # vocab, context, layers, heads, dimension, batch


@pytest.mark.parametrize("variant", ["oracle", "oracle_fused"])
def test_gpt_gradients_on_the_oracle_device(request, variant):
    """ref_gpt_grads (the one-backward C4 check's harness) on a small char-GPT with the C oracle as
    the device, unmodified kael and with its device branches: every parameter gradient against
    kael's CPU path at the reference's f32 device tolerance, the initial parameters bit for bit."""
    lib = request.getfixturevalue("kael_" + variant)
    total = lib.ref_gpt_param_total(*SMALL_GPT[:5])
    out = {}
    for device in (0, 1):
        loss, grads, params = ctypes.c_float(), np.zeros(total, np.float32), np.zeros(total, np.float32)
        assert lib.ref_gpt_grads(device, *SMALL_GPT, ctypes.byref(loss), support.ptr(grads), support.ptr(params)) == 0, \
            support.ref_error(lib)
        out[device] = (loss.value, grads, params)
    np.testing.assert_array_equal(out[1][2], out[0][2])
    assert np.count_nonzero(out[0][1]) > total // 2
    assert_reference_close(out[1][1], out[0][1], "gradients")
    assert abs(out[1][0] - out[0][0]) <= 1e-5 * abs(out[0][0])

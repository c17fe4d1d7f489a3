"""Gradients and trained parameters through kael's autograd on the MI355X against kael's CPU path.

  - Linear-shaped products y = x . W^T with x [B, M, K] and a 2-D weight W [N, K] (kael's Linear,
    reference src/nn/layers.cpp:42-43; MatmulBackward src/autograd/functions_linalg.cpp:29-49):
    W.grad and x.grad element by element, at C4's four Linear shapes and ragged ones, through
    unmodified kael (libkael_hip.so: one product per batch item, then sum_to_shape) and through
    kael's optional device branches (libkael_hip_fused.so: the weight gradient as one product over
    the folded batch, X_flat^T . g_flat, on the split-K path).
  - C4 (char-GPT, Adam): every one of the 3 216 896 parameters after 5 Adam steps, for both builds.

  - C4 after one forward and backward: every parameter gradient, with no exception.

Tolerance: the reference's f32 device tolerance, |dev - cpu| <= 1e-4 + 1e-4 |cpu|
(tests/test_cuda.cpp:40-43), elementwise. For trained parameters, Adam's first updates are
lr * g / (|g| + eps): an element whose CPU gradient is within rounding of zero can take an update
of different sign on the two sides (at most 2 lr per step), so only elements whose first-step CPU
gradient is that small (NEAR_ZERO_GRADIENT) may exceed the tolerance, by no more than 2 * lr * steps.
"""
import ctypes

import numpy as np
import pytest

import support

pytestmark = pytest.mark.gpu

P = support.ptr
# (batch, m, k, n): C4's qkv, proj, fc1 (K 256) and fc2 (K 1024) weights over 32 x 128 tokens,
# then ragged shapes (no whole tiles, K not a multiple of 16, a single token).
SHAPES = [(32, 128, 256, 768), (32, 128, 256, 256), (32, 128, 256, 1024), (32, 128, 1024, 256),
          (3, 37, 53, 29), (5, 1, 7, 3), (2, 130, 200, 96)]


def linear_grads(lib, device, shape, seed=7):
    b, m, k, n = shape
    wg, xg = np.empty((n, k), np.float32), np.empty((b, m, k), np.float32)
    assert lib.ref_linear_grads(device, b, m, k, n, seed, P(wg), P(xg)) == 0, support.ref_error(lib)
    return wg, xg


def assert_reference_close(got, want, what):
    bad = np.abs(got.astype(np.float64) - want) > 1e-4 + 1e-4 * np.abs(want)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} elements beyond 1e-4 + 1e-4|cpu|"


@pytest.mark.parametrize("variant", ["hip", "hip_fused"])
@pytest.mark.parametrize("shape", SHAPES, ids=["x".join(map(str, s)) for s in SHAPES])
def test_linear_gradients_match_cpu(request, variant, shape):
    lib = request.getfixturevalue("kael_" + variant)
    cpu_w, cpu_x = linear_grads(lib, 0, shape)
    dev_w, dev_x = linear_grads(lib, 1, shape)
    assert_reference_close(dev_w, cpu_w, "W.grad")
    assert_reference_close(dev_x, cpu_x, "x.grad")


# (batch, m, k, n) of the tied LM head's product weight . h^T: C4's (32 x 128 tokens, d 256, vocab
# 96), then ragged shapes.
HEAD_SHAPES = [(32, 128, 256, 96), (3, 37, 53, 29), (2, 1, 7, 3)]


def head_grads(lib, device, shape, seed=9):
    b, m, k, n = shape
    wg, hg = np.empty((n, k), np.float32), np.empty((b, m, k), np.float32)
    assert lib.ref_head_grads(device, b, m, k, n, seed, P(wg), P(hg)) == 0, support.ref_error(lib)
    return wg, hg


@pytest.mark.parametrize("variant", ["hip", "hip_fused"])
@pytest.mark.parametrize("shape", HEAD_SHAPES, ids=["x".join(map(str, s)) for s in HEAD_SHAPES])
def test_head_gradients_match_cpu(request, variant, shape):
    """The tied head's weight gradient: per batch item and a batch sum (unmodified kael), one
    product over the folded batch (the device branch); both against kael's CPU path."""
    lib = request.getfixturevalue("kael_" + variant)
    cpu_w, cpu_h = head_grads(lib, 0, shape)
    dev_w, dev_h = head_grads(lib, 1, shape)
    assert_reference_close(dev_w, cpu_w, "W.grad")
    assert_reference_close(dev_h, cpu_h, "h.grad")


C4 = (96, 128, 4, 4, 256, 32)  # vocab, context, layers, heads, dimension, batch
# A first-step gradient this close to zero is within the two sides' rounding differences, so its
# sign (and Adam's first update, lr * g / (|g| + eps), about +-lr) may differ between them.
NEAR_ZERO_GRADIENT = 1e-6
LR = 1e-3  # kael's Adam default (include/kael/optim/adam.h:11-17)


SELECT_CASES = ["attention_split", "two_of_three", "same_index_twice", "mixed_with_whole", "two_dims",
                "retained_intermediate", "anomaly_detection", "select_of_select", "retained_graph_twice"]


def select_grads(lib, device, which, seed=11):
    xg, pg = np.empty(72, np.float32), np.empty(72, np.float32)
    assert lib.ref_select_grads(device, which, seed, P(xg), P(pg)) == 0, support.ref_error(lib)
    return xg, pg


@pytest.mark.parametrize("variant", ["hip", "hip_fused"])
@pytest.mark.parametrize("which", range(len(SELECT_CASES)), ids=SELECT_CASES)
def test_select_gradients_match_cpu(request, variant, which):
    """Select gradients (kael's zero fill, copy and sum on the device): every value equal to kael's
    CPU path."""
    lib = request.getfixturevalue("kael_" + variant)
    cpu_x, cpu_p = select_grads(lib, 0, which)
    dev_x, dev_p = select_grads(lib, 1, which)
    assert np.array_equal(dev_x, cpu_x) and np.array_equal(dev_p, cpu_p)
    assert (cpu_p != 0).any() == (SELECT_CASES[which] == "retained_intermediate")


def chargpt(lib, device, steps):
    total = lib.ref_gpt_param_total(*C4[:5])
    losses, params, secs = np.zeros(steps, np.float32), np.zeros(total, np.float32), ctypes.c_double()
    assert lib.ref_train_gpt_params(device, steps, *C4, P(losses), P(params), ctypes.byref(secs)) == 0, \
        support.ref_error(lib)
    return losses, params


def chargpt_grads(lib, device):
    total = lib.ref_gpt_param_total(*C4[:5])
    loss, grads, params = ctypes.c_float(), np.zeros(total, np.float32), np.zeros(total, np.float32)
    assert lib.ref_gpt_grads(device, *C4, ctypes.byref(loss), P(grads), P(params)) == 0, support.ref_error(lib)
    return loss.value, grads, params


@pytest.mark.timeout(300)
@pytest.mark.parametrize("variant", ["hip", "hip_fused"])
def test_c4_every_gradient_after_one_backward(request, variant):
    """C4's forward, cross-entropy and backward once (seed 3): every one of the 3 216 896 parameter
    gradients against kael's CPU path, |dev - cpu| <= 1e-4 + 1e-4 |cpu| with no exception, and the
    initial parameters bit for bit (the same seeded init on both sides)."""
    lib = request.getfixturevalue("kael_" + variant)
    cpu_loss, cpu_g, cpu_p = chargpt_grads(lib, 0)
    dev_loss, dev_g, dev_p = chargpt_grads(lib, 1)
    assert cpu_g.size == 3216896
    np.testing.assert_array_equal(dev_p, cpu_p)
    assert abs(dev_loss - cpu_loss) <= 1e-4 * abs(cpu_loss)
    assert np.count_nonzero(cpu_g) > cpu_g.size // 2  # the check sees real gradients
    excess = np.abs(dev_g.astype(np.float64) - cpu_g) - (1e-4 + 1e-4 * np.abs(cpu_g.astype(np.float64)))
    print(f"\nC4 {variant}: loss {dev_loss} vs {cpu_loss}; largest |dg| {np.abs(dev_g - cpu_g).max():.3e}, "
          f"largest relative {np.max(np.abs(dev_g - cpu_g) / (np.abs(cpu_g) + 1e-12)):.3e}")
    assert excess.max() <= 0, f"{int((excess > 0).sum())} gradients beyond 1e-4 + 1e-4|cpu|"


@pytest.mark.timeout(300)
@pytest.mark.parametrize("variant", ["hip", "hip_fused"])
def test_c4_every_parameter_after_five_adam_steps(request, variant):
    lib = request.getfixturevalue("kael_" + variant)
    steps = 5
    cpu_l, cpu_p = chargpt(lib, 0, steps)
    dev_l, dev_p = chargpt(lib, 1, steps)
    assert cpu_p.size == 3216896
    np.testing.assert_allclose(dev_l, cpu_l, rtol=1e-4)
    diff = np.abs(dev_p.astype(np.float64) - cpu_p)
    bad = diff > 1e-4 + 1e-4 * np.abs(cpu_p)
    _, g1, _ = chargpt_grads(lib, 0)  # kael's CPU gradients of the first step
    near_zero = np.abs(g1) <= NEAR_ZERO_GRADIENT
    moved = np.abs(dev_p - cpu_p).max()
    print(f"\nC4 {variant}: {cpu_p.size} parameters after {steps} Adam steps, {bad.sum()} beyond 1e-4 + 1e-4|p| "
          f"(first-step |g| of those: {np.abs(g1[bad]).max() if bad.any() else 0:.2e}; {near_zero.sum()} gradients "
          f"within {NEAR_ZERO_GRADIENT:g} of zero), max |dp| = {moved:.2e}; losses {dev_l.tolist()}")
    assert not (bad & ~near_zero).any(), \
        f"{int((bad & ~near_zero).sum())} parameters beyond the tolerance whose first gradient is not near zero"
    assert diff.max() <= 2 * LR * steps, f"largest parameter difference {diff.max():.3e}"

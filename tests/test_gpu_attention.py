"""kd_causal_attention / kd_causal_attention_backward (kael's causal self-attention chain,
reference src/nn/transformer.cpp:114-136, as one launch forward and two backward) on the MI355X
against the C oracle's restatement of kael's composed ops (oracle/kd_oracle.c), which the CPU tests
pin to kael's CPU path and to the mathematics.

Tolerance: the reference's f32 device tolerance 1e-4 + 1e-4 |oracle| (tests/test_cuda.cpp:40-43),
elementwise, for the output, the rows' log-sum-exp and the qkv gradient. The kernels use no atomics:
a second call gives the same bits. Shapes: C4's attention (32 x 128 tokens, 4 heads; here 4 of its
batch rows), GPT-2's 12 heads, ragged lengths (no whole block of 32), one token, and 1024 positions.
Then kael's CausalSelfAttention module on the device through the fused branch against kael's CPU
path.
"""
import numpy as np
import pytest

import kd
import support
from test_oracle_attention import close, inputs, module_grads, oracle_attention

pytestmark = pytest.mark.gpu

P = support.ptr
SHAPES = [(1, 1, 1), (2, 37, 3), (4, 128, 4), (1, 200, 2), (2, 64, 12), (1, 1024, 1)]


def device_attention(kdb, qkv, dout, b, t, h):
    dqkv_in, ddout = kdb.to_device(qkv), kdb.to_device(dout)
    out, lse, dq = kdb.empty((b, t, h * 64), np.float32), kdb.empty((b, h, t), np.float32), kdb.empty(qkv.shape, np.float32)
    kdb.call("causal_attention", kd.F32, out.ptr, lse.ptr, dqkv_in.ptr, b, t, h, 64)
    kdb.call("causal_attention_backward", kd.F32, dq.ptr, ddout.ptr, dqkv_in.ptr, out.ptr, lse.ptr, b, t, h, 64)
    return out.numpy(), lse.numpy(), dq.numpy()


@pytest.mark.parametrize("shape", SHAPES, ids=["x".join(map(str, s)) for s in SHAPES])
def test_attention_matches_the_oracle(kdb, oracle, shape):
    b, t, h = shape
    qkv, dout = inputs(b, t, h, 64)
    want = oracle_attention(oracle, qkv, dout, b, t, h, 64)
    got = device_attention(kdb, qkv, dout, b, t, h)
    for g, w, what in zip(got, want, ("out", "lse", "qkv.grad")):
        close(g, w.astype(np.float64), what)
    again = device_attention(kdb, qkv, dout, b, t, h)
    for g, a in zip(got, again):
        np.testing.assert_array_equal(g, a)


def test_attention_rejects_unsupported_shapes(kdb):
    x = kdb.to_device(np.zeros(3 * 64 * 4, np.float32))
    with pytest.raises(kd.KdError):
        kdb.call("causal_attention", kd.F64, x.ptr, x.ptr, x.ptr, 1, 1, 1, 64)
    with pytest.raises(kd.KdError):
        kdb.call("causal_attention", kd.F32, x.ptr, x.ptr, x.ptr, 1, 1, 2, 32)
    with pytest.raises(kd.KdError):
        kdb.call("causal_attention_backward", kd.F32, x.ptr, x.ptr, x.ptr, x.ptr, x.ptr, 1, 0, 1, 64)
    # missing or misaligned operands are rejected on the host, before any launch
    with pytest.raises(kd.KdError):
        kdb.call("causal_attention", kd.F32, None, x.ptr, x.ptr, 1, 1, 1, 64)
    with pytest.raises(kd.KdError):
        kdb.call("causal_attention", kd.F32, x.ptr, x.ptr, x.ptr + 4, 1, 1, 1, 64)
    with pytest.raises(kd.KdError):
        kdb.call("causal_attention_backward", kd.F32, x.ptr, None, x.ptr, x.ptr, x.ptr, 1, 1, 1, 64)


@pytest.mark.parametrize("shape", [(32, 128, 256, 4), (2, 9, 128, 2), (1, 200, 768, 12)],
                         ids=["c4_32x128x256x4", "2x9x128x2", "1x200x768x12"])
def test_module_through_the_fused_branch_on_the_device(kael_hip_fused, shape):
    """kael's CausalSelfAttention module with the attention on kd_causal_attention against kael's
    CPU path: output, input gradient and every parameter gradient."""
    cpu = module_grads(kael_hip_fused, 0, shape)
    dev = module_grads(kael_hip_fused, 1, shape)
    for got, want, what in zip(dev, cpu, ("out", "x.grad", "parameter grads")):
        close(got, want.astype(np.float64), what)


@pytest.mark.parametrize("seed", range(8))
def test_attention_random_shapes(kdb, oracle, seed):
    """Seeded random shapes (1-3 batch rows, 1-300 positions, 1-6 heads): every ragged tail of the
    32-row blocks, the forward and backward against the oracle at the device tolerance."""
    rng = np.random.default_rng(1000 + seed)
    b, t, h = int(rng.integers(1, 4)), int(rng.integers(1, 301)), int(rng.integers(1, 7))
    qkv, dout = inputs(b, t, h, 64, seed)
    want = oracle_attention(oracle, qkv, dout, b, t, h, 64)
    got = device_attention(kdb, qkv, dout, b, t, h)
    for g, w, what in zip(got, want, ("out", "lse", "qkv.grad")):
        try:
            close(g, w.astype(np.float64), what)
        except AssertionError as e:
            raise AssertionError(f"seed {seed}: {b}x{t}x{h}: {e}") from None

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

kd_cached_attention (new queries against a KV cache, read in place through strides) against the
oracle's cached restatement at the same tolerance: decode (one query, 1-1024 keys, every ragged
32-key group), chunks of queries after a past, a whole prompt with no past, strided views of the
fused projection and contiguous cache tensors; then kael's module with a KV cache through the
cached branch against kael's CPU path.
"""
import numpy as np
import pytest

import kd
import support
from test_oracle_attention import cached_module, close, inputs, module_grads, oracle_attention, oracle_cached, qkv_views

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


def device_cached(kdb, q, k, v, b, h, t, keys, arrays):
    """kd_cached_attention over device copies of the host arrays that q, k and v point into."""
    dev = {id(a): kdb.to_device(a) for a in arrays}
    def remap(view):
        ptr, strides = view
        for a in arrays:
            if a.ctypes.data <= ptr < a.ctypes.data + a.nbytes:
                return dev[id(a)].ptr + (ptr - a.ctypes.data), strides
        raise ValueError("pointer outside the given arrays")
    (qp, qs), (kp, ks), (vp, vs) = remap(q), remap(k), remap(v)
    out = kdb.empty((b, t, h * 64), np.float32)
    kdb.call("cached_attention", kd.F32, out.ptr, qp, P(qs), kp, P(ks), vp, P(vs), b, h, t, keys, 64)
    return out.numpy()


CACHED = [(1, 12, 1, 1), (1, 12, 1, 31), (1, 12, 1, 32), (1, 12, 1, 33), (1, 12, 1, 100), (1, 12, 1, 1024),
          (2, 3, 5, 37), (1, 2, 64, 64), (3, 1, 7, 300)]


@pytest.mark.parametrize("shape", CACHED, ids=["x".join(map(str, s)) for s in CACHED])
def test_cached_attention_matches_the_oracle(kdb, oracle, shape):
    """(batch, heads, new queries, keys): the queries are the last rows of a fused projection of
    `keys` positions, the keys and values its per-head views (strided) and, for the second call,
    contiguous [B, H, keys, 64] copies (kael's cache after its cat)."""
    b, h, t, keys = shape
    qkv, _ = inputs(b, keys, h, 64, seed=t + keys)
    q, _, _ = qkv_views(qkv, b, keys, h, 64, start=keys - t)
    _, k, v = qkv_views(qkv, b, keys, h, 64)
    want = oracle_cached(oracle, q, k, v, b, h, t, keys).astype(np.float64)
    got = device_cached(kdb, q, k, v, b, h, t, keys, [qkv])
    close(got, want, "cached (strided)")
    np.testing.assert_array_equal(device_cached(kdb, q, k, v, b, h, t, keys, [qkv]), got)
    x = qkv.reshape(b, keys, 3, h, 64)
    kc = np.ascontiguousarray(x[:, :, 1].transpose(0, 2, 1, 3))
    vc = np.ascontiguousarray(x[:, :, 2].transpose(0, 2, 1, 3))
    cs = np.array([h * keys * 64, keys * 64, 64], np.int64)
    got_c = device_cached(kdb, q, (kc.ctypes.data, cs), (vc.ctypes.data, cs), b, h, t, keys, [qkv, kc, vc])
    close(got_c, want, "cached (contiguous cache)")


def test_cached_attention_rejects_bad_arguments(kdb):
    x = kdb.to_device(np.zeros(3 * 64 * 8, np.float32))
    s = np.array([0, 0, 64], np.int64)
    bad = np.array([0, -1, 64], np.int64)
    args = lambda dtype, strides, t, keys, d: (dtype, x.ptr, x.ptr, P(strides), x.ptr, P(s), x.ptr, P(s), 1, 1, t,
                                               keys, d)
    for a in (args(kd.F64, s, 1, 1, 64), args(kd.F32, s, 1, 1, 32), args(kd.F32, s, 2, 1, 64),
              args(kd.F32, s, 0, 1, 64), args(kd.F32, bad, 1, 1, 64)):
        with pytest.raises(kd.KdError):
            kdb.call("cached_attention", *a)
    with pytest.raises(kd.KdError):
        kdb.call("cached_attention", kd.F32, None, x.ptr, P(s), x.ptr, P(s), x.ptr, P(s), 1, 1, 1, 1, 64)


@pytest.mark.parametrize("shape", [(1, 7, 40, 1, 768, 12), (2, 16, 48, 8, 256, 4), (1, 130, 131, 1, 128, 2)],
                         ids=["gpt2_heads_tokens", "c4_heads_chunks", "past130"])
def test_cached_module_through_the_branch_on_the_device(kael_hip_fused, shape):
    """kael's CausalSelfAttention with a KV cache (a prompt, then tokens or chunks, no gradient) with
    the attention on kd_cached_attention, against kael's CPU path with the cache."""
    cpu, _ = cached_module(kael_hip_fused, 0, shape)
    dev, _ = cached_module(kael_hip_fused, 1, shape)
    close(dev, cpu.astype(np.float64), "cached module")

"""The oracle's restatement of kael's causal self-attention chain (oracle/kd_oracle.c:
oracle_causal_attention / _backward, reference src/nn/transformer.cpp:114-136) pinned on the CPU:

  - against kael's own ops on its CPU path (oracle/ref_shim.cpp ref_attention_chain: the view,
    selects, transposes, the product, scale, triu mask, softmax, product and merge copy of
    CausalSelfAttention::forward, then kael's autograd), output and qkv gradient, at the
    reference's f32 device tolerance 1e-4 + 1e-4 |cpu| (tests/test_cuda.cpp:40-43);
  - against a float64 numpy statement of the mathematics (softmax over the unmasked keys, its
    Jacobian), which also pins the rows' log-sum-exp that the fused backward consumes (not a kael
    value), and fails a dropped scale, a mask off by one, or q and k swapped in the backward.

Then kael's CausalSelfAttention module and a small GPT through the fused branch with the oracle as
the device (oracle/kael_fused.py: the attention as one device call and one backward node for f32
heads of 64), against kael's CPU path, and the branch's call counters.

The cached restatement (oracle_cached_attention: new queries against the cache's keys and values,
reference src/nn/transformer.cpp:103-138 with a cache) is pinned to the uncached one, which the
checks above pin: with no past it is the uncached chain bit for bit; the attention of the last T
queries against all L keys is bit for bit the last T rows of the full attention over L positions;
strided views and contiguous copies give the same bits. kael's module with a KV cache (a prompt,
then single tokens and chunks) through the branch on the oracle device matches kael's CPU path.
"""
import ctypes

import numpy as np
import pytest

import support
from test_oracle_kael_fused import calls

P = support.ptr
SHAPES = [(1, 1, 1, 64), (2, 9, 2, 64), (1, 33, 1, 64), (2, 5, 3, 16)]


def inputs(b, t, h, d, seed=3):
    rng = np.random.default_rng(seed + b + t + h + d)
    qkv = rng.uniform(-1, 1, (b, t, 3 * h * d)).astype(np.float32)
    dout = rng.uniform(-1, 1, (b, t, h * d)).astype(np.float32)
    return qkv, dout


def oracle_attention(oracle, qkv, dout, b, t, h, d):
    out = np.empty((b, t, h * d), np.float32)
    lse = np.empty((b, h, t), np.float32)
    dq = np.empty_like(qkv)
    assert oracle.oracle_causal_attention(0, P(out), P(lse), P(qkv), b, t, h, d) == 0
    assert oracle.oracle_causal_attention_backward(0, P(dq), P(dout), P(qkv), P(out), P(lse), b, t, h, d) == 0
    return out, lse, dq


def numpy_attention(qkv, dout, b, t, h, d):
    """float64: out, lse and the qkv gradient of sum(out * dout)."""
    x = qkv.astype(np.float64).reshape(b, t, 3, h, d)
    q, k, v = (x[:, :, i].transpose(0, 2, 1, 3) for i in range(3))  # [b, h, t, d]
    s = q @ k.transpose(0, 1, 3, 2) / np.sqrt(d)
    s = np.where(np.triu(np.ones((t, t), bool), 1), -np.inf, s)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    lse = (m + np.log(e.sum(-1, keepdims=True)))[..., 0]
    p = e / e.sum(-1, keepdims=True)
    o = p @ v
    go = dout.astype(np.float64).reshape(b, t, h, d).transpose(0, 2, 1, 3)
    dp = go @ v.transpose(0, 1, 3, 2)
    dv = p.transpose(0, 1, 3, 2) @ go
    ds = p * (dp - (dp * p).sum(-1, keepdims=True)) / np.sqrt(d)
    dq = ds @ k
    dk = ds.transpose(0, 1, 3, 2) @ q
    grad = np.stack([g.transpose(0, 2, 1, 3) for g in (dq, dk, dv)], axis=2).reshape(b, t, 3 * h * d)
    return o.transpose(0, 2, 1, 3).reshape(b, t, h * d), lse, grad


def close(got, want, what, rel=1e-4, abs_=1e-4):
    err = np.abs(got.astype(np.float64) - want)
    bad = err > abs_ + rel * np.abs(want)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} elements, worst {err.max():.3g}"


@pytest.mark.parametrize("shape", SHAPES, ids=["x".join(map(str, s)) for s in SHAPES])
def test_oracle_matches_kaels_cpu_chain(oracle, kael_oracle, shape):
    b, t, h, d = shape
    qkv, dout = inputs(b, t, h, d)
    out, _, dq = oracle_attention(oracle, qkv, dout, b, t, h, d)
    kout, kdq = np.empty_like(out), np.empty_like(qkv)
    assert kael_oracle.ref_attention_chain(0, P(qkv), P(dout), b, t, h, d, P(kout), P(kdq)) == 0, \
        support.ref_error(kael_oracle)
    close(out, kout.astype(np.float64), "out")
    close(dq, kdq.astype(np.float64), "qkv.grad")


@pytest.mark.parametrize("shape", SHAPES, ids=["x".join(map(str, s)) for s in SHAPES])
def test_oracle_matches_the_mathematics(oracle, shape):
    b, t, h, d = shape
    qkv, dout = inputs(b, t, h, d)
    out, lse, dq = oracle_attention(oracle, qkv, dout, b, t, h, d)
    want_out, want_lse, want_dq = numpy_attention(qkv, dout, b, t, h, d)
    close(out, want_out, "out", 1e-5, 1e-6)
    close(lse, want_lse, "lse", 1e-6, 1e-6)
    close(dq, want_dq, "qkv.grad", 1e-4, 1e-5)
    # the first query sees only key 0: its output row is v[0], its lse the one scaled score
    x = qkv.reshape(b, t, 3, h, d).astype(np.float64)
    np.testing.assert_allclose(out.reshape(b, t, h, d)[:, 0], x[:, 0, 2], rtol=0, atol=0)
    np.testing.assert_allclose(lse[:, :, 0], (x[:, 0, 0] * x[:, 0, 1]).sum(-1) / np.sqrt(d), rtol=1e-6, atol=1e-6)


def test_oracle_rejects_other_dtypes_and_empty_shapes(oracle):
    x = np.zeros(64 * 3, np.float64)
    out, lse = np.zeros(64), np.zeros(1)
    assert oracle.oracle_causal_attention(1, P(out), P(lse), P(x), 1, 1, 1, 64) != 0
    assert oracle.oracle_causal_attention(0, P(out), P(lse), P(x), 1, 0, 1, 64) != 0


def module_grads(lib, device, shape, seed=5):
    b, t, c, h = shape
    out, xg = np.empty((b, t, c), np.float32), np.empty((b, t, c), np.float32)
    grads = np.empty(4 * c * c + 4 * c, np.float32)
    assert lib.ref_attention_module(device, b, t, c, h, seed, P(out), P(xg), P(grads)) == 0, support.ref_error(lib)
    return out, xg, grads


@pytest.mark.parametrize("shape, fused", [((2, 9, 128, 2), True), ((1, 40, 64, 1), True), ((2, 9, 32, 2), False)],
                         ids=["2x9x128x2", "1x40x64x1", "2x9x32x2_heads_of_16"])
def test_module_through_the_fused_branch(kael_oracle_fused, shape, fused):
    """kael's CausalSelfAttention (its two Linears and the attention) on the oracle device through
    the fused branch, against kael's CPU path: output, input gradient, every parameter gradient;
    heads of 16 keep kael's ops (the counters do not move)."""
    lib = kael_oracle_fused
    cpu = module_grads(lib, 0, shape)
    before = calls(lib)
    dev = module_grads(lib, 1, shape)
    after = calls(lib)
    for got, want, what in zip(dev, cpu, ("out", "x.grad", "parameter grads")):
        close(got, want.astype(np.float64), what)
    ran = after["causal_attention"] - before["causal_attention"], \
        after["causal_attention_backward"] - before["causal_attention_backward"]
    assert ran == ((1, 1) if fused else (0, 0))


def test_gpt_with_heads_of_64_through_the_fused_branch(kael_oracle_fused):
    """A one-layer char-GPT with two heads of 64 (vocab 96, context 16, batch 2): 3 Adam steps with
    the attention on the fused branch, losses against kael's CPU path."""
    lib = kael_oracle_fused
    steps = 3
    args = (steps, 96, 16, 1, 2, 128, 2)
    cpu_l, dev_l = np.zeros(steps, np.float32), np.zeros(steps, np.float32)
    t = ctypes.c_double()
    assert lib.ref_train_gpt(0, *args, cpu_l.ctypes.data_as(ctypes.c_void_p), ctypes.byref(t)) == 0, support.ref_error(lib)
    before = calls(lib)
    assert lib.ref_train_gpt(1, *args, dev_l.ctypes.data_as(ctypes.c_void_p), ctypes.byref(t)) == 0, support.ref_error(lib)
    after = calls(lib)
    np.testing.assert_allclose(dev_l, cpu_l, rtol=1e-4)
    assert after["causal_attention"] - before["causal_attention"] >= steps
    assert after["causal_attention_backward"] - before["causal_attention_backward"] == steps


# ---- attention against a KV cache ---------------------------------------------------------------

def qkv_views(qkv, b, t, h, d, start=0):
    """Pointers and (batch, head, position) strides of the q / k / v per-head views of qkv
    [b, t, 3, h, d] from position `start` (what selects and transposes give kael)."""
    base = qkv.ctypes.data + start * 3 * h * d * 4
    strides = np.array([t * 3 * h * d, d, 3 * h * d], np.int64)
    return [(base + part * h * d * 4, strides) for part in range(3)]


def oracle_cached(oracle, q, k, v, b, h, t, keys, d=64):
    out = np.zeros((b, t, h * d), np.float32)
    (qp, qs), (kp, ks), (vp, vs) = q, k, v
    rc = oracle.oracle_cached_attention(0, P(out), qp, P(qs), kp, P(ks), vp, P(vs), b, h, t, keys, d)
    assert rc == 0, oracle.oracle_last_error()
    return out


@pytest.mark.parametrize("shape", [(1, 1, 1), (2, 9, 2), (1, 40, 3)], ids=["1x1x1", "2x9x2", "1x40x3"])
def test_cached_oracle_without_past_is_the_uncached_chain(oracle, shape):
    b, t, h = shape
    qkv, dout = inputs(b, t, h, 64)
    want, _, _ = oracle_attention(oracle, qkv, dout, b, t, h, 64)
    q, k, v = qkv_views(qkv, b, t, h, 64)
    np.testing.assert_array_equal(oracle_cached(oracle, q, k, v, b, h, t, t), want)


@pytest.mark.parametrize("shape", [(1, 10, 1, 1), (2, 33, 2, 5), (1, 70, 3, 70)], ids=["L10_T1", "L33_T5", "L70_T70"])
def test_cached_oracle_rows_are_the_full_attentions_last_rows(oracle, shape):
    b, length, h, t = shape
    qkv, dout = inputs(b, length, h, 64, seed=11)
    full, _, _ = oracle_attention(oracle, qkv, dout, b, length, h, 64)
    q, _, _ = qkv_views(qkv, b, length, h, 64, start=length - t)
    _, k, v = qkv_views(qkv, b, length, h, 64)
    got = oracle_cached(oracle, q, k, v, b, h, t, length)
    np.testing.assert_array_equal(got, full[:, length - t:])


def test_cached_oracle_reads_strided_and_contiguous_operands_alike(oracle):
    b, length, h, t = 2, 21, 3, 4
    qkv, _ = inputs(b, length, h, 64, seed=17)
    q, k, v = qkv_views(qkv, b, length, h, 64, start=length - t)
    _, k, v = qkv_views(qkv, b, length, h, 64)
    strided = oracle_cached(oracle, q, k, v, b, h, t, length)
    x = qkv.reshape(b, length, 3, h, 64)
    kc = np.ascontiguousarray(x[:, :, 1].transpose(0, 2, 1, 3))
    vc = np.ascontiguousarray(x[:, :, 2].transpose(0, 2, 1, 3))
    cs = np.array([h * length * 64, length * 64, 64], np.int64)
    contiguous = oracle_cached(oracle, q, (kc.ctypes.data, cs), (vc.ctypes.data, cs), b, h, t, length)
    np.testing.assert_array_equal(strided, contiguous)


def test_cached_oracle_rejects_bad_shapes(oracle):
    x = np.zeros(64 * 3 * 4, np.float32)
    s = np.array([0, 0, 64], np.int64)
    out = np.zeros(64 * 4, np.float32)
    assert oracle.oracle_cached_attention(1, P(out), P(x), P(s), P(x), P(s), P(x), P(s), 1, 1, 1, 1, 64) != 0
    assert oracle.oracle_cached_attention(0, P(out), P(x), P(s), P(x), P(s), P(x), P(s), 1, 1, 2, 1, 64) != 0


def cached_module(lib, device, shape, seed=6):
    b, prompt, total, step, c, h = shape
    cached, full = np.empty((b, total, c), np.float32), np.empty((b, total, c), np.float32)
    assert lib.ref_cached_attention_module(device, b, prompt, total, step, c, h, seed, P(cached), P(full)) == 0, \
        support.ref_error(lib)
    return cached, full


@pytest.mark.parametrize("shape, fused", [((1, 5, 12, 1, 128, 2), True), ((2, 3, 20, 4, 64, 1), True),
                                          ((1, 4, 9, 1, 32, 2), False)],
                         ids=["prompt5_tokens", "batch2_chunks4", "heads_of_16"])
def test_cached_module_through_the_branch(kael_oracle_fused, shape, fused):
    """kael's CausalSelfAttention with a KV cache (a prompt, then single tokens or chunks; no
    gradient) on the oracle device through the cached branch, against kael's CPU path with the
    cache; kael's own cached outputs against its cacheless forward on the CPU; the branch runs once
    per forward call (heads of 16 keep kael's ops)."""
    lib = kael_oracle_fused
    b, prompt, total, step = shape[:4]
    cpu_cached, cpu_full = cached_module(lib, 0, shape)
    close(cpu_cached, cpu_full.astype(np.float64), "kael cached vs cacheless")
    before = calls(lib)
    dev_cached, _ = cached_module(lib, 1, shape)
    after = calls(lib)
    close(dev_cached, cpu_cached.astype(np.float64), "cached")
    forwards = 1 + -(-(total - prompt) // step)
    assert after["cached_attention"] - before["cached_attention"] == (forwards if fused else 0)

"""Config C5 end to end (GPT-2 small, f32, batch 1, greedy with a KV cache) at the config's
length, against kael's own CPU path (reference examples/gpt2_generate.cpp:62-95 ->
nn::generate, src/nn/transformer.cpp:256-295):

  - the benchmark's exact run (kael's seed-4 GPT-2 small, which bench.py draws with
    kd_gpt_kael_init, its seed-4 64-token prompt, 256 new tokens): the decode engine's tokens equal
    kael's CPU generate token for token, and the teacher-forced logits of all 320 positions are
    within 1e-4 of each row's largest |logit|;
  - kael's seed-4 GPT-2 small over a 1024-token sequence (every position of the context, the
    cache filled to max_positions): the engine's cached logits against kael's full forward;
  - kael's unmodified nn::generate running on the MI355X through this backend
    (oracle/_ref/libkael_hip.so: kael's host code, every tensor on the device), and the same with
    kael's optional device branches (libkael_hip_fused.so), 256 tokens each, token for token
    against kael's CPU generate, with their tokens/s printed beside the CPU's.

Greedy argmax could flip where two logits tie within rounding; where a row's winner differs, the
test requires the CPU's top two logits to be within the tolerance (none do at these seeds).
"""
import ctypes
import os
import sys
import time

import numpy as np
import pytest

import kd
import support

pytestmark = pytest.mark.gpu

sys.path.insert(0, str(support.ROOT))
import bench  # noqa: E402  (the benchmark's weights and prompt, so the test covers its exact run)

VOCAB, CTX, LAYERS, HEADS, DIM = 50257, 1024, 12, 12, 768
PROMPT, NEW = 64, 256


def threads():
    return min(16, max(1, os.cpu_count() or 1))


def kael_model(ref, weights=None):
    """kael's GPT-2 small from manual_seed(4); with `weights` (name -> array) its parameters are
    overwritten with them."""
    h = ref.ref_gpt_create(VOCAB, CTX, LAYERS, HEADS, DIM, 4, 1)
    assert h, support.ref_error(ref)
    if weights is not None:
        for i, (name, _) in enumerate(_names(ref, h)):
            a = np.ascontiguousarray(weights[name], np.float32)
            assert ref.ref_gpt_set_param(h, i, a.ctypes.data_as(ctypes.c_void_p)) == 0, support.ref_error(ref)
    return h


def _names(ref, h):
    name = ctypes.create_string_buffer(256)
    shape = (ctypes.c_int64 * 8)()
    rank = ctypes.c_int()
    out = []
    for i in range(ref.ref_gpt_param_count(h)):
        assert ref.ref_gpt_param(h, i, name, 256, shape, ctypes.byref(rank), None) == 0
        out.append((name.value.decode(), tuple(shape[d] for d in range(rank.value))))
    return out


def cpu_generate(ref, h, prompt, new):
    p = np.ascontiguousarray(prompt, np.int64)
    out = np.zeros(len(p) + new, np.int64)
    secs = ctypes.c_double()
    assert ref.ref_gpt_generate(h, p.ctypes.data_as(ctypes.c_void_p), len(p), new, out.ctypes.data_as(ctypes.c_void_p),
                                ctypes.byref(secs)) == 0, support.ref_error(ref)
    return out, secs.value


def cpu_forward(ref, h, tokens):
    t = np.ascontiguousarray(tokens, np.int64)
    out = np.empty((len(t), VOCAB), np.float32)
    assert ref.ref_gpt_forward(h, t.ctypes.data_as(ctypes.c_void_p), 1, len(t),
                               out.ctypes.data_as(ctypes.c_void_p)) == 0, support.ref_error(ref)
    return out


def engine(kdb, weights):
    g = kd.Gpt(kdb)
    for name, a in weights:
        g.load(name, a)
    return g


def check_logits(got, want, rtol=1e-4):
    """Every row within rtol of its largest |logit|; argmax equal unless the CPU's top two are
    within that tolerance."""
    scale = np.abs(want).max(axis=1, keepdims=True)
    err = np.abs(got - want) / scale
    worst = int(err.max(axis=1).argmax())
    assert err.max() <= rtol, f"position {worst}: max |dlogit| / max|logit| = {err.max():.3e}"
    differ = np.nonzero(got.argmax(axis=1) != want.argmax(axis=1))[0]
    for r in differ:
        top = np.sort(want[r])[-2:]
        assert top[1] - top[0] <= rtol * scale[r, 0], f"position {r}: argmax differs without a near-tie"
    return float(err.max())


@pytest.fixture(scope="module")
def bench_run(kdb, refdev):
    """The benchmark's weights and prompt; kael's CPU generate of its 256 tokens."""
    refdev.ref_set_threads(threads())
    weights = bench.gpt2_weights()
    prompt = np.random.default_rng(4).integers(0, VOCAB, PROMPT)
    h = kael_model(refdev, dict(weights))
    try:
        seq, secs = cpu_generate(refdev, h, prompt, NEW)
        logits = cpu_forward(refdev, h, seq[:-1])  # positions 0 .. 318 predict tokens 1 .. 319
    finally:
        refdev.ref_gpt_destroy(h)
    return weights, prompt, seq, secs, logits


@pytest.mark.timeout(300)
def test_bench_run_token_for_token(kdb, bench_run):
    weights, prompt, seq, cpu_secs, _ = bench_run
    g = engine(kdb, weights)
    g.prefill(prompt)
    t0 = time.perf_counter()
    g.decode(NEW - 1)
    t1 = time.perf_counter()
    np.testing.assert_array_equal(g.sequence(), seq)
    print(f"\nC5 bench run: {NEW} tokens identical to kael's CPU generate (first {seq[PROMPT:PROMPT + 8].tolist()}); "
          f"engine decode {(NEW - 1) / (t1 - t0):.0f} tokens/s, kael CPU {NEW / cpu_secs:.2f} tokens/s "
          f"({threads()} threads)")


def test_bench_run_teacher_forced_logits(kdb, bench_run):
    weights, _, seq, _, want = bench_run
    g = engine(kdb, weights)
    got = g.forward_logits(seq[:-1])
    err = check_logits(got, want)
    print(f"\nC5 bench run: {len(want)} positions, max |dlogit| / max|logit| = {err:.2e}")


@pytest.mark.timeout(300)
def test_full_context_teacher_forced_logits(kdb, refdev):
    """kael's seed-4 model over 1024 tokens: the engine's cached steps at every position up to
    max_positions - 1 against kael's full forward over the sequence."""
    refdev.ref_set_threads(threads())
    h = kael_model(refdev)
    try:
        params = support.export_gpt_params(refdev, h)
        tokens = np.random.default_rng(44).integers(0, VOCAB, CTX)
        want = cpu_forward(refdev, h, tokens)
    finally:
        refdev.ref_gpt_destroy(h)
    g = engine(kdb, params)
    got = g.forward_logits(tokens)
    err = check_logits(got, want)
    print(f"\nC5 1024 positions: max |dlogit| / max|logit| = {err:.2e}")


@pytest.fixture(scope="module")
def kael_cpu_tokens(kael_hip):
    """kael's CPU generate from kael's own seed-4 model (the library the device runs use)."""
    kael_hip.ref_set_threads(threads())
    h = kael_model(kael_hip)
    prompt = np.random.default_rng(4).integers(0, VOCAB, PROMPT)
    try:
        seq, secs = cpu_generate(kael_hip, h, prompt, NEW)
    finally:
        kael_hip.ref_gpt_destroy(h)
    return prompt, seq, secs


@pytest.mark.timeout(300)
@pytest.mark.parametrize("variant", ["hip", "hip_fused"])
def test_kael_generate_unchanged_on_the_device(request, kael_cpu_tokens, variant):
    """kael's own nn::generate (examples/gpt2_generate.cpp's call) with the model and prompt on the
    MI355X: the unmodified kael host code (hip) and kael with its optional device branches
    (hip_fused)."""
    lib = request.getfixturevalue("kael_hip" if variant == "hip" else "kael_hip_fused")
    prompt, seq, cpu_secs = kael_cpu_tokens
    h = kael_model(lib)
    out = np.zeros(PROMPT + NEW, np.int64)
    secs = ctypes.c_double()
    p = np.ascontiguousarray(prompt, np.int64)
    try:
        assert lib.ref_gpt_generate_on(h, 1, p.ctypes.data_as(ctypes.c_void_p), PROMPT, NEW,
                                       out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(secs)) == 0, support.ref_error(lib)
    finally:
        lib.ref_gpt_destroy(h)
    np.testing.assert_array_equal(out, seq)
    print(f"\nkael nn::generate on the MI355X ({variant}): {NEW} tokens in {secs.value:.2f} s = "
          f"{NEW / secs.value:.1f} tokens/s (prefill included); kael CPU {NEW / cpu_secs:.2f} tokens/s")


def streamed(lib, device, prompt, new, stop_after):
    h = kael_model(lib)
    out, seen = np.zeros(len(prompt) + new, np.int64), np.zeros(new, np.int64)
    total, count = ctypes.c_int64(), ctypes.c_int64()
    p = np.ascontiguousarray(prompt, np.int64)
    try:
        assert lib.ref_gpt_generate_streamed(h, device, p.ctypes.data_as(ctypes.c_void_p), len(p), new, stop_after,
                                             out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(total),
                                             seen.ctypes.data_as(ctypes.c_void_p), ctypes.byref(count)) == 0, \
            support.ref_error(lib)
    finally:
        lib.ref_gpt_destroy(h)
    return out[:total.value], seen[:count.value]


@pytest.mark.timeout(300)
def test_generate_with_on_token_on_the_engine(kael_hip_fused):
    """examples/gpt2_generate.cpp hands generate an on_token printer: through kael's branch the
    engine calls it once per token with a [1, 1] device tensor and stops when it returns false,
    exactly as kael's CPU loop does (here after 9 of 40 tokens, then to the end)."""
    lib = kael_hip_fused
    lib.ref_set_threads(threads())
    prompt = np.random.default_rng(8).integers(0, VOCAB, 12)
    for stop_after in (9, 40):
        cpu_seq, cpu_seen = streamed(lib, 0, prompt, 40, stop_after)
        dev_seq, dev_seen = streamed(lib, 1, prompt, 40, stop_after)
        np.testing.assert_array_equal(dev_seq, cpu_seq)
        np.testing.assert_array_equal(dev_seen, cpu_seen)
        assert len(cpu_seen) == stop_after and len(cpu_seq) == 12 + stop_after


def sampled(lib, device, prompt, batch, new, temperature, top_k, seed):
    h = kael_model(lib)
    out, t, after = np.zeros(batch * (len(prompt) + new), np.int64), ctypes.c_double(), ctypes.c_double()
    p = np.ascontiguousarray(prompt, np.int64)
    try:
        assert lib.ref_gpt_generate_sampled(h, device, p.ctypes.data_as(ctypes.c_void_p), len(p), batch, new,
                                            temperature, top_k, seed, out.ctypes.data_as(ctypes.c_void_p),
                                            ctypes.byref(t), ctypes.byref(after)) == 0, support.ref_error(lib)
    finally:
        lib.ref_gpt_destroy(h)
    return out.reshape(batch, -1), t.value, after.value


@pytest.mark.timeout(300)
@pytest.mark.parametrize("variant", ["hip", "hip_fused"])
def test_kael_sampled_generate_with_its_cache_on_the_device(request, variant):
    """kael's nn::generate with sampling (temperature 0.8, top-k 1, seed 9) of a prompt repeated
    over two rows: its own loop with the KV cache runs on the device (the decode engine takes batch 1
    only), sample_next on the host. top-k 1 leaves one token with probability 1, so the draws are
    fixed and the device sequences must equal kael's CPU ones. Through the fused build the attention
    of every cached step is one kd_cached_attention call."""
    lib = request.getfixturevalue("kael_hip" if variant == "hip" else "kael_hip_fused")
    lib.ref_set_threads(threads())
    prompt = np.random.default_rng(9).integers(0, VOCAB, 16)
    new = 24
    cpu, cpu_s, cpu_next = sampled(lib, 0, prompt, 2, new, 0.8, 1, 9)
    dev, dev_s, dev_next = sampled(lib, 1, prompt, 2, new, 0.8, 1, 9)
    np.testing.assert_array_equal(dev, cpu)
    assert dev_next == cpu_next
    print(f"\nkael nn::generate sampled with its KV cache, 2 rows, on the MI355X ({variant}): {new} tokens in "
          f"{dev_s:.2f} s = {2 * new / dev_s:.1f} tokens/s; kael CPU {2 * new / cpu_s:.2f} tokens/s")


@pytest.mark.timeout(300)
@pytest.mark.parametrize("temperature, top_k", [(0.8, 40), (1.0, 0)], ids=["example_t0.8_k40", "default_t1_none"])
def test_kael_sampled_generate_on_the_engine(kael_hip_fused, temperature, top_k):
    """The reference example's sampling (examples/gpt2_generate.cpp: temperature 0.8, top-k 40), and
    GenerateOptions' defaults (temperature 1, top_k 0: nothing masked, the whole vocabulary summed),
    through kael's nn::generate: the fused build runs it on the decode engine with the device
    sampler, the draws taken from kael's generator; the tokens must equal kael's CPU generate with
    the same seed (its sample_next on the host), for 64 tokens after a 16-token prompt, and the
    generator's next draw afterwards must be the same (the engine used exactly one draw per token)."""
    lib = kael_hip_fused
    lib.ref_set_threads(threads())
    prompt = np.random.default_rng(11).integers(0, VOCAB, 16)
    new = 64
    cpu, cpu_s, cpu_next = sampled(lib, 0, prompt, 1, new, temperature, top_k, 5)
    dev, dev_s, dev_next = sampled(lib, 1, prompt, 1, new, temperature, top_k, 5)
    np.testing.assert_array_equal(dev, cpu)
    assert dev_next == cpu_next
    assert len(set(cpu[0, 16:].tolist())) > 8  # sampled, not one repeated token
    print(f"\nkael nn::generate, temperature {temperature}, top-k {top_k}, on the MI355X decode engine: {new} tokens in "
          f"{dev_s:.2f} s = {new / dev_s:.1f} tokens/s (engine set-up and prefill included); kael CPU "
          f"{new / cpu_s:.2f} tokens/s")

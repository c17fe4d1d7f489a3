"""The GPT-2 decode engine (kd_gpt_*) against kael's own GPT on the CPU path.

Weights come from kael itself (GPT constructor with manual_seed, src/nn/transformer.cpp:171-207),
exported parameter by parameter, so both sides run the identical model. Checks:
  - a small model (the config of reference tests/test_cuda.cpp:584-609, in f32): logits of every
    position with the KV cache, and the greedy generation, token for token;
  - GPT-2 small (config C5, seed 4): teacher-forced logits over a 64-token prompt plus decode
    steps, within 1e-4 relative, and identical greedy tokens.
"""
import ctypes

import numpy as np
import pytest

import kd
import support

pytestmark = pytest.mark.gpu


def export_params(ref, handle):
    return support.export_gpt_params(ref, handle)


def build(kdb, ref, vocab, positions, layers, heads, dim, seed):
    h = ref.ref_gpt_create(vocab, positions, layers, heads, dim, seed, 1)
    assert h, support.ref_error(ref)
    params = export_params(ref, h)
    g = kd.Gpt(kdb, vocab, positions, layers, heads, dim, True)
    for name, data in params:
        g.load(name, data)
    return h, g


def cpu_cached_logits(ref, h, tokens, prompt, vocab):
    t = np.ascontiguousarray(tokens, np.int64)
    rows = len(t) - prompt + 1
    out = np.empty((rows, vocab), np.float32)
    assert ref.ref_gpt_cached_logits(h, t.ctypes.data_as(ctypes.c_void_p), prompt, len(t),
                                     out.ctypes.data_as(ctypes.c_void_p)) == 0, support.ref_error(ref)
    return out


def cpu_generate(ref, h, prompt, new):
    p = np.ascontiguousarray(prompt, np.int64)
    out = np.zeros(len(p) + new, np.int64)
    secs = ctypes.c_double()
    assert ref.ref_gpt_generate(h, p.ctypes.data_as(ctypes.c_void_p), len(p), new, out.ctypes.data_as(ctypes.c_void_p),
                                ctypes.byref(secs)) == 0, support.ref_error(ref)
    return out, secs.value


def test_small_model_logits_and_generation(kdb, refdev):
    ref = refdev
    h, g = build(kdb, ref, 11, 16, 2, 2, 8, 31)
    try:
        rng = np.random.default_rng(0)
        tokens = rng.integers(0, 11, 12)
        want = cpu_cached_logits(ref, h, tokens, 1, 11)  # position 0 alone, then one token at a time
        got = g.forward_logits(tokens)
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
        prompt = tokens[:6]
        seq, _ = cpu_generate(ref, h, prompt, 8)
        g.prefill(prompt)
        new = g.decode(7)
        np.testing.assert_array_equal(np.concatenate([g.sequence()]), seq)
        np.testing.assert_array_equal(new, seq[7:])
    finally:
        ref.ref_gpt_destroy(h)


def test_gpt2_small_teacher_forced_logits(kdb, refdev):
    ref = refdev
    ref.ref_set_threads(min(16, max(1, __import__("os").cpu_count() or 1)))
    h, g = build(kdb, ref, 50257, 1024, 12, 12, 768, 4)
    try:
        rng = np.random.default_rng(4)
        prompt_len, extra = 64, 6
        tokens = rng.integers(0, 50257, prompt_len + extra)
        want = cpu_cached_logits(ref, h, tokens, prompt_len, 50257)  # prefill's last row, then 6 steps
        got = g.forward_logits(tokens)[prompt_len - 1:]
        scale = np.abs(want).max()
        err = np.abs(got - want).max()
        assert err <= 1e-4 * scale, f"max |dlogit| {err} vs scale {scale}"
        np.testing.assert_array_equal(got.argmax(axis=1), want.argmax(axis=1))
        seq, _ = cpu_generate(ref, h, tokens[:prompt_len], 4)
        g.prefill(tokens[:prompt_len])
        g.decode(3)
        np.testing.assert_array_equal(g.sequence(), seq)
    finally:
        ref.ref_gpt_destroy(h)


def test_hugging_face_checkpoint_loads_into_the_engine(kdb, refdev, tmp_path):
    """A GPT-2 checkpoint in Hugging Face layout (kael's own weights written as model.safetensors)
    through Gpt.load_gpt2_safetensors: the engine then computes kael's logits."""
    from safetensors.numpy import save_file

    ref = refdev
    h = ref.ref_gpt_create(11, 16, 2, 2, 8, 31, 1)
    assert h, support.ref_error(ref)
    try:
        path = tmp_path / "model.safetensors"
        save_file(support.hf_gpt2_tensors(support.export_gpt_params(ref, h)), str(path))
        g = kd.Gpt(kdb, 11, 16, 2, 2, 8, True)
        g.load_gpt2_safetensors(path)
        tokens = np.random.default_rng(1).integers(0, 11, 10)
        want = cpu_cached_logits(ref, h, tokens, 1, 11)
        np.testing.assert_allclose(g.forward_logits(tokens), want, rtol=1e-5, atol=1e-6)
        seq, _ = cpu_generate(ref, h, tokens[:4], 6)
        g.prefill(tokens[:4])
        g.decode(5)
        np.testing.assert_array_equal(g.sequence(), seq)
    finally:
        ref.ref_gpt_destroy(h)


@pytest.mark.parametrize("prefix", [True, False], ids=["transformer_prefix", "bare"])
def test_checkpoint_load_rules(kdb, refdev, tmp_path, prefix):
    """kd_gpt_load_safetensors as kael's load_gpt2_weights + load_state_dict (reference
    src/nn/transformer.cpp:297-308, src/nn/module.cpp:94-109): with or without the `transformer.`
    prefix it loads; a missing parameter or a weight in the wrong layout is an error before anything
    is copied; an F16 checkpoint loads widened, giving kael's logits for the f16-rounded weights."""
    from safetensors.numpy import save_file

    ref = refdev
    h = ref.ref_gpt_create(11, 16, 2, 2, 8, 31, 1)
    assert h, support.ref_error(ref)
    try:
        params = support.export_gpt_params(ref, h)
        tokens = np.random.default_rng(2).integers(0, 11, 8)
        hf = support.hf_gpt2_tensors(params, prefix_blocks=prefix)
        path = tmp_path / "model.safetensors"
        save_file(hf, str(path))
        g = kd.Gpt(kdb, 11, 16, 2, 2, 8, True)
        g.load_gpt2_safetensors(path)
        np.testing.assert_allclose(g.forward_logits(tokens), cpu_cached_logits(ref, h, tokens, 1, 11), rtol=1e-5, atol=1e-6)

        block = "transformer.h.1." if prefix else "h.1."
        missing = dict(hf)
        del missing[block + "mlp.c_fc.bias"]
        save_file(missing, str(tmp_path / "missing.safetensors"))
        with pytest.raises(kd.KdError, match="missing parameter blocks.1.mlp.fc1.bias"):
            kd.Gpt(kdb, 11, 16, 2, 2, 8, True).load_gpt2_safetensors(tmp_path / "missing.safetensors")
        wrong = dict(hf)
        wrong[block + "attn.c_attn.weight"] = np.ascontiguousarray(wrong[block + "attn.c_attn.weight"].T)
        save_file(wrong, str(tmp_path / "wrong.safetensors"))
        with pytest.raises(kd.KdError, match="shape"):
            kd.Gpt(kdb, 11, 16, 2, 2, 8, True).load_gpt2_safetensors(tmp_path / "wrong.safetensors")

        half = {k: v.astype(np.float16) for k, v in hf.items()}
        save_file(half, str(tmp_path / "half.safetensors"))
        g16 = kd.Gpt(kdb, 11, 16, 2, 2, 8, True)
        g16.load_gpt2_safetensors(tmp_path / "half.safetensors")
        for i, (name, data) in enumerate(params):  # kael with the same rounded weights
            rounded = np.ascontiguousarray(data.astype(np.float16).astype(np.float32))
            assert ref.ref_gpt_set_param(h, i, rounded.ctypes.data_as(ctypes.c_void_p)) == 0, support.ref_error(ref)
        np.testing.assert_allclose(g16.forward_logits(tokens), cpu_cached_logits(ref, h, tokens, 1, 11), rtol=1e-5,
                                   atol=1e-6)
    finally:
        ref.ref_gpt_destroy(h)


def check_prefill_and_steps(g, ref, h, prompt, steps, vocab, rtol):
    """Prefill `prompt`, then `steps` greedy decode steps; the logits after the prefill and
    after every step against kael's cached forward over kael's own greedy sequence."""
    seq, _ = cpu_generate(ref, h, prompt, steps + 1)
    want = cpu_cached_logits(ref, h, seq, len(prompt), vocab)  # rows: positions len-1 .. len+steps
    g.prefill(prompt)
    got = [g.logits()]
    for _ in range(steps):
        g.decode(1)
        got.append(g.logits())
    got = np.stack(got)
    scale = np.abs(want).max()
    err = np.abs(got - want[:steps + 1]).max()
    assert err <= rtol * scale, f"max |dlogit| {err} vs scale {scale}"
    np.testing.assert_array_equal(g.sequence(), seq[:len(prompt) + steps + 1])
    return got


@pytest.mark.parametrize("prompt_len", [1, 5, 16])
def test_small_model_batched_prefill(kdb, refdev, prompt_len):
    """head_dim 4, prompts of one position up to the whole context; batched and stepwise prefill
    both against kael, and against each other."""
    ref = refdev
    h = ref.ref_gpt_create(11, 24, 2, 2, 8, 31, 1)
    assert h, support.ref_error(ref)
    try:
        params = export_params(ref, h)
        prompt = np.random.default_rng(prompt_len).integers(0, 11, prompt_len)
        steps = min(4, 24 - prompt_len - 1)
        runs = []
        for stepwise in (False, True):
            g = kd.Gpt(kdb, 11, 24, 2, 2, 8, True, stepwise_prefill=stepwise)
            for name, data in params:
                g.load(name, data)
            runs.append(check_prefill_and_steps(g, ref, h, prompt, steps, 11, 1e-5))
        np.testing.assert_allclose(runs[0], runs[1], rtol=1e-5, atol=1e-6)
    finally:
        ref.ref_gpt_destroy(h)


def test_gpt2_small_batched_prefill(kdb, refdev):
    """Config C5 with prompts of 1, 64 and 100 positions (split-K partial products on 64-row
    tiles, one and two of them), 129, 300 (128-row tiles) and 600 positions (decode steps past
    512 cached keys): the prompt's last logits and three decode steps within 1e-4 of the largest
    logit, kael's greedy tokens."""
    ref = refdev
    ref.ref_set_threads(min(16, max(1, __import__("os").cpu_count() or 1)))
    h, g = build(kdb, ref, 50257, 1024, 12, 12, 768, 4)
    try:
        rng = np.random.default_rng(5)
        for prompt_len in (1, 64, 100, 129, 300, 600):
            check_prefill_and_steps(g, ref, h, rng.integers(0, 50257, prompt_len), 3, 50257, 1e-4)
    finally:
        ref.ref_gpt_destroy(h)


def test_odd_head_dim_is_rejected(kdb):
    with pytest.raises(kd.KdError):
        kd.Gpt(kdb, 11, 16, 1, 4, 24, True)  # head_dim 6


@pytest.mark.parametrize("prompt_len", [10, 16, 23])
def test_generation_past_the_context(kdb, refdev, prompt_len):
    """Greedy generation that outgrows max_positions (16): once the KV cache is full, every token
    clears it and reruns the last 16 tokens from position 0, as nn::generate does (reference
    src/nn/transformer.cpp:270-284); a prompt longer than the context runs its last 16 tokens.
    Tokens identical to kael's generate; the logits of each window rerun against kael's forward
    over the same window (batched and stepwise prefill)."""
    ref = refdev
    h = ref.ref_gpt_create(11, 16, 2, 2, 8, 31, 1)
    assert h, support.ref_error(ref)
    try:
        params = export_params(ref, h)
        prompt = np.random.default_rng(100 + prompt_len).integers(0, 11, prompt_len)
        new = 30
        seq, _ = cpu_generate(ref, h, prompt, new)
        for stepwise in (False, True):
            g = kd.Gpt(kdb, 11, 16, 2, 2, 8, True, stepwise_prefill=stepwise)
            for name, data in params:
                g.load(name, data)
            g.prefill(prompt)
            got = [g.sequence()[-1]]
            for _ in range(new - 1):
                got.extend(g.decode(1))
                total = len(prompt) + len(got) - 1  # tokens that went into the last forward
                if total > 16:  # a window rerun: its last position's logits
                    want = cpu_cached_logits(ref, h, seq[total - 16:total], 16, 11)[0]
                    np.testing.assert_allclose(g.logits(), want, rtol=1e-5, atol=1e-5)
            np.testing.assert_array_equal(np.array(got), seq[len(prompt):])
            np.testing.assert_array_equal(g.sequence(), seq)
        g = kd.Gpt(kdb, 11, 16, 2, 2, 8, True)  # the same in one decode call
        for name, data in params:
            g.load(name, data)
        g.prefill(prompt)
        np.testing.assert_array_equal(g.decode(new - 1), seq[len(prompt) + 1:])
    finally:
        ref.ref_gpt_destroy(h)


def test_unknown_flags_are_rejected(kdb):
    cfg = kd.GptConfig(11, 16, 1, 2, 8, 1, 4)  # bit 2: no such mode
    h = ctypes.c_void_p()
    assert kdb.lib.kd_gpt_supported(ctypes.byref(cfg)) == -1  # KD_E_INVALID
    assert kdb.lib.kd_gpt_create(ctypes.byref(h), ctypes.byref(cfg)) == -1


def oracle_pick(oracle, logits, temperature, top_k, u):
    tok = ctypes.c_int64()
    assert oracle.oracle_sample_topk(logits.ctypes.data_as(ctypes.c_void_p), logits.size, temperature, top_k, u,
                                     ctypes.byref(tok)) == 0, oracle.oracle_last_error()
    return tok.value


@pytest.mark.parametrize("vocab, temperature, top_k", [(11, 0.8, 3), (97, 1.3, 40), (97, 0.5, 96), (97, 2.0, 1),
                                                        (97, 0.004, 40), (50257, 0.8, 40), (50257, 1.0, 500),
                                                        (11, 0.8, 0), (97, 1.0, 97), (50257, 1.0, 0)],
                         ids=["v11_k3", "v97_k40", "v97_k96", "v97_k1", "v97_k40_cold", "v50257_k40", "v50257_k500",
                              "v11_none", "v97_k_vocab", "v50257_none"])
def test_sampled_picks_match_the_oracle(kdb, refdev, oracle, vocab, temperature, top_k):
    """kael's sample_next on the device (kd_gpt_set_sampling, kd_gpt_set_uniforms): after the prefill and
    after every decode step the engine's pick equals the oracle's restatement of sample_next on the
    same logits with the same draw, and the draws are used one per token. The cold case spreads
    the kept weights below 2^-24, where the device sums in sequence instead of across the wave;
    GPT-2's vocabulary takes the bound from the head kernel's 1024 workgroup maxima (k = 40) or,
    with more candidate workgroups than the pick reads, the full scan and the sequential sums over
    more than 64 kept entries (k = 500). Without a top-k (top_k 0, kael's default, or top_k =
    vocab) nothing is masked: every entry is kept and summed in index order."""
    ref = refdev
    h, g = build(kdb, ref, vocab, 32, 2, 2, 8, 13)
    try:
        rng = np.random.default_rng(vocab + top_k)
        prompt = rng.integers(0, vocab, 6)
        steps = 20
        u = rng.uniform(0, 1, steps + 1)
        g.set_sampling(temperature, top_k)
        g.set_uniforms(u)
        g.prefill(prompt)
        picks = [g.sequence()[-1]]
        assert picks[0] == oracle_pick(oracle, g.logits(), temperature, top_k, u[0])
        for s in range(1, steps + 1):
            picks.extend(g.decode(1))
            assert picks[-1] == oracle_pick(oracle, g.logits(), temperature, top_k, u[s]), s
        assert g.draws_used() == steps + 1
        if (top_k > 1 or top_k == 0) and temperature >= 0.1:  # (the cold case nearly always picks the largest)
            assert len(set(picks)) > 1
        # the same draws in one decode call give the same tokens
        g.set_uniforms(u)
        g.prefill(prompt)
        np.testing.assert_array_equal(g.decode(steps), picks[1:])
        # greedy again after sampling: kael's greedy tokens
        g.set_sampling(0.0)
        seq, _ = cpu_generate(ref, h, prompt, 8)
        g.prefill(prompt)
        np.testing.assert_array_equal(g.decode(7), seq[len(prompt) + 1:])
    finally:
        ref.ref_gpt_destroy(h)


@pytest.mark.parametrize("vocab, spread", [(3000, "top"), (6000, "top"), (6000, "all")])
def test_sampled_picks_with_tied_logits(kdb, refdev, oracle, vocab, spread):
    """The device's top-k over vocabularies spanning several key slots of the picking workgroup (the
    last one partial) with exactly tied logits (duplicated rows of the tied embedding): 40 copies of
    the row with about the third largest logit spread over slots and waves, the cut at the tied
    value (kael keeps every entry equal to the k-th largest, so more than k are kept), small k
    (the listed candidates above the lanes' maxima bound) and k > 1024 (every key); or every row
    alike, so that the bound lists more keys than the workgroup stages and the kept list (all of
    the vocabulary) goes to the global scratch."""
    ref = refdev
    h = ref.ref_gpt_create(vocab, 32, 1, 2, 8, 21, 1)
    assert h, support.ref_error(ref)
    try:
        params = export_params(ref, h)
        wte = dict(params)["token_embedding.weight"]
        g = kd.Gpt(kdb, vocab, 32, 1, 2, 8, True)
        for name, data in params:
            g.load(name, data)
        rng = np.random.default_rng(vocab)
        prompt = rng.integers(0, vocab, 5)
        g.prefill(prompt)  # greedy, for the prompt's logits
        lg = g.logits()
        if spread == "top":
            # copies off the prompt's tokens leave the prompt's hidden state as it is
            source = next(int(i) for i in np.argsort(-lg, kind="stable")[2:] if i not in prompt)
            copies = rng.choice(np.setdiff1d(np.arange(vocab), np.append(prompt, source)), 40, replace=False)
        else:
            source, copies = 0, np.arange(vocab)
        wte[copies] = wte[source]
        g.load("token_embedding.weight", wte)
        g.prefill(prompt)
        lg = g.logits()
        assert np.count_nonzero(lg == lg[source]) >= min(41, vocab)  # identical rows, identical logits
        rank = int(np.count_nonzero(lg > lg[source]))
        if spread == "top":
            cases = [(0.9, rank + 1), (0.9, rank + 20), (1.1, vocab - 50)]
        else:
            cases = [(0.9, 40), (1.1, 1500)]
        for temperature, top_k in cases:
            steps = 6
            u = rng.uniform(0, 1, steps + 1)
            g.set_sampling(temperature, top_k)
            g.set_uniforms(u)
            g.prefill(prompt)
            got = g.sequence()[-1]
            assert got == oracle_pick(oracle, g.logits(), temperature, top_k, u[0]), (temperature, top_k)
            for s in range(1, steps + 1):
                got = g.decode(1)[0]
                assert got == oracle_pick(oracle, g.logits(), temperature, top_k, u[s]), (temperature, top_k, s)
            assert g.draws_used() == steps + 1
        g.set_sampling(0.0)
    finally:
        ref.ref_gpt_destroy(h)


def test_sampling_arguments_and_missing_draws_fail(kdb, refdev):
    ref = refdev
    big = kd.Gpt(kdb, 65537, 16, 1, 2, 8, True)
    with pytest.raises(kd.KdError, match="65536"):
        big.set_sampling(0.8, 40)
    del big
    h, g = build(kdb, ref, 11, 16, 1, 2, 8, 3)
    try:
        for t, k in [(0.8, -1), (-1.0, 3)]:
            with pytest.raises(kd.KdError):
                g.set_sampling(t, k)
        with pytest.raises(kd.KdError):
            g.set_uniforms(np.array([0.5, 1.0]))
        g.set_sampling(0.9, 4)
        g.set_uniforms(np.array([0.25, 0.75]))
        g.prefill(np.array([1, 2, 3]))
        g.decode(1)
        with pytest.raises(kd.KdError, match="no uniform draw left"):
            g.decode(1)
        with pytest.raises(kd.KdError):
            g.forward_logits(np.array([1, 2]))
    finally:
        ref.ref_gpt_destroy(h)

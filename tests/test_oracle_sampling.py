"""The oracle's restatement of kael's sampled next token (oracle/kd_oracle.c oracle_sample_topk:
sample_next with a temperature and a top-k or none, reference src/nn/transformer.cpp:39-50, with softmax's
CPU row kernel, src/ops/nn.cpp:60-71, and multinomial, src/random.cpp:106-160) pinned on the CPU:

  - against kael's own ops (oracle/ref_shim.cpp ref_sample_next: logits / temperature, topk,
    masked_fill, softmax, multinomial on kael's CPU path, after manual_seed and a number of earlier
    draws), with the oracle given the uniform that kael's generator returns at that point: the same
    id for random logits of 5 to 50257 entries, temperatures around 1, top-k from 1 to vocab - 1
    and none (top_k 0, kael's default, and top_k = vocab: nothing masked), ties at the k-th value,
    near-degenerate and spread-out rows;
  - against the definition of a top-k categorical draw on tiny rows: for a grid of uniforms the pick
    is the kept entry whose cumulative-probability interval holds u (probabilities from float64
    arithmetic, the grid kept away from the interval ends);
  - bad arguments are rejected.
"""
import ctypes

import numpy as np
import pytest

import support
from test_oracle_random import draws, seeded, uniform_continuation

P = support.ptr


@pytest.fixture(scope="module")
def cpu_kael():
    return support.load_ref("ref")


def oracle_pick(oracle, logits, temperature, top_k, u):
    tok = ctypes.c_int64()
    rc = oracle.oracle_sample_topk(P(logits), logits.size, temperature, top_k, u, ctypes.byref(tok))
    assert rc == 0, oracle.oracle_last_error()
    return tok.value


def kael_pick(cpu_kael, seed, skip, logits, temperature, top_k):
    tok = ctypes.c_int64()
    assert cpu_kael.ref_sample_next(seed, skip, P(logits), logits.size, temperature, top_k, ctypes.byref(tok)) == 0, \
        support.ref_error(cpu_kael)
    return tok.value


def kael_uniform(oracle, seed, skip):
    state = seeded(oracle, seed)
    draws(oracle, state, skip)
    return uniform_continuation(oracle, state)


def rows():
    rng = np.random.default_rng(7)
    yield "gpt2_like", rng.normal(0, 3, 50257).astype(np.float32)
    yield "small", rng.normal(0, 1, 97).astype(np.float32)
    yield "flat", np.zeros(64, np.float32)                    # every entry tied at the k-th value
    ties = rng.normal(0, 1, 200).astype(np.float32)
    ties[::7] = ties.max()                                   # many entries tied with the maximum
    yield "ties", ties
    peaked = rng.normal(0, 1, 500).astype(np.float32)
    peaked[123] = 60.0                                       # one entry takes almost all the mass
    yield "peaked", peaked
    yield "spread", rng.uniform(-200, 200, 1000).astype(np.float32)  # most exponentials underflow


@pytest.mark.parametrize("name, logits", list(rows()), ids=[n for n, _ in rows()])
def test_oracle_picks_what_kael_picks(oracle, cpu_kael, name, logits):
    v = logits.size
    for i, (temperature, top_k) in enumerate([(0.8, 40), (1.0, 1), (1.7, 5), (0.8, v - 1), (0.33, 2), (1.0, 0),
                                              (0.8, v)]):
        top_k = top_k if top_k in (0, v) else min(top_k, v - 1)
        for seed, skip in [(i, 0), (100 + i, 313), (7 * i + 1, 5)]:
            u = kael_uniform(oracle, seed, skip)
            want = kael_pick(cpu_kael, seed, skip, logits, temperature, top_k)
            got = oracle_pick(oracle, logits, temperature, top_k, u)
            assert got == want, (name, temperature, top_k, seed, skip, u)


@pytest.mark.parametrize("k, kept", [(3, [1, 3, 0]), (0, [0, 1, 2, 3, 4]), (5, [0, 1, 2, 3, 4])],
                         ids=["top3", "none", "k_vocab"])
def test_picks_follow_the_cumulative_intervals(oracle, k, kept):
    """Five logits, top-3 (the three largest kept) or no top-k (all five): the kept entries' softmax
    probabilities in float64; u inside each interval (away from its ends) picks that entry, and
    the masked entries are never picked."""
    logits = np.array([0.5, 2.0, -1.0, 1.5, 0.1], np.float32)
    t = 1.0
    e = np.exp(logits[sorted(kept)].astype(np.float64) - logits.max())
    p = e / e.sum()
    edges = np.concatenate([[0.0], np.cumsum(p)])
    for j, idx in enumerate(sorted(kept)):
        for f in (0.05, 0.5, 0.95):
            u = edges[j] + f * (edges[j + 1] - edges[j])
            assert oracle_pick(oracle, logits, t, k, u) == idx


def test_oracle_rejects_bad_arguments(oracle):
    x = np.zeros(10, np.float32)
    tok = ctypes.c_int64()
    for args in [(x, 10, 1.0, -1, 0.5), (x, 10, 0.0, 3, 0.5), (x, 10, 1.0, 3, 1.0), (x, 1, 1.0, 1, 0.5)]:
        a, v, t, k, u = args
        assert oracle.oracle_sample_topk(P(a), v, t, k, u, ctypes.byref(tok)) != 0
    bad = np.zeros(10, np.float32)
    bad[3] = np.nan
    assert oracle.oracle_sample_topk(P(bad), 10, 1.0, 3, 0.5, ctypes.byref(tok)) != 0

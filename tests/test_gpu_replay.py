"""bench.py's C3 / C4 training steps: the recorded device calls of kael's own loops
(tests/golden/*_step_calls.jsonl.gz) replayed against the C ABI on the GPU, every index operand
checked before its kernel runs.

C3's trace holds every upload (inputs and Kaiming-uniform parameters from manual_seed(2)), so the
replay recomputes kael's run: both steps' losses within 1e-5 of the losses kael reported when the
trace was recorded (rtol 1e-5: the products run on the MFMA path here, in kael's order on the C
oracle). C4's trace holds the token ids and targets; its parameters are kael's seed-3 model as
bench.py draws it (kd_gpt_kael_init), so the replay also recomputes kael's run. Repeating the last
step must keep the losses finite and the buffers in bounds (no index re-check)."""
import math
from pathlib import Path

import kd

import numpy as np
import pytest

import replay

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def c4_uploads(backend):
    """The 52 parameter uploads of C4's trace (after its ids and targets): kael's seed-3 char-GPT."""
    return {2 + i: a for i, (_, a) in enumerate(kd.kael_gpt_parameters(backend, 3, 96, 128, 4, 4, 256))}


def run_trace(kdb, name, repeats):
    recs = replay.load(GOLDEN / f"{name}_step_calls.jsonl.gz")
    setup, steps = replay.split_steps(recs)
    rp = replay.Replay(kdb, recs, c4_uploads(kdb) if name == "c4" else None)
    rp.run(setup)
    for s in steps:
        rp.run(s)
    for _ in range(repeats):
        rp.run(steps[-1], checked=False)
    kdb.synchronize()
    return rp, replay.traced_losses(recs)


def test_c3_replay_reproduces_kael_losses(kdb):
    rp, kael = run_trace(kdb, "c3", 0)
    per_step = len(rp.losses) // 2
    got = [rp.losses[per_step - 1], rp.losses[2 * per_step - 1]]
    np.testing.assert_allclose(got, kael, rtol=1e-5)


def test_c4_replay_reproduces_kael_losses(kdb):
    rp, kael = run_trace(kdb, "c4", 2)
    assert len(kael) == 2
    per_step = len(rp.losses) // 4
    got = [rp.losses[per_step - 1], rp.losses[2 * per_step - 1]]
    np.testing.assert_allclose(got, kael, rtol=1e-5)
    assert abs(got[0] - math.log(96)) > 0.01  # a real model, not uniform logits
    assert all(math.isfinite(x) for x in rp.losses)

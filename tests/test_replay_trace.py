"""The recorded C3 / C4 step traces that bench.py replays (tests/golden/*_step_calls.jsonl.gz,
written by tests/golden/make_step_traces.py from kael's own training loops): well-formed without
a device. Every record is a known backend call, every device pointer lies inside an allocation
that is live at that point, the trace holds the setup and two steps, and the steps issue the
calls that C3 (MLP, SGD) and C4 (char-GPT, Adam) need."""
from pathlib import Path

import pytest

import replay

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_trace_is_well_formed(name):
    recs = replay.load(GOLDEN / f"{name}_step_calls.jsonl.gz")
    replay.validate(recs)
    setup, steps = replay.split_steps(recs)
    assert len(steps) == 2 and setup
    losses = replay.traced_losses(recs)
    assert len(losses) == 2 and all(0 < x < 10 for x in losses)
    ops = {r["op"] for r in steps[-1]}
    assert {"matmul_strided", "cross_entropy_rows", "cross_entropy_grad", "d2h"} <= ops
    assert ("sgd_step" if name == "c3" else "adam_step_many") in ops
    if name == "c4":
        # the fused LayerNorms and their backward passes, the fused attention and its backward, the
        # Linear products with their bias, the column sums and the one-call index range checks are
        # in the step; the attention's own products, mask and softmax are not
        assert {"layer_norm_rows", "layer_norm_rows_backward", "causal_attention", "causal_attention_backward",
                "matmul_strided_bias", "reduce_columns", "gather", "scatter_add", "index_bounds"} <= ops
        assert not {"softmax_rows", "softmax_rows_backward", "matmul_strided_heads"} & ops
    # the step's products: C3 has 3 (forward 2, backward 3 minus the input gradient), C4 dozens
    assert replay.matmul_flops(steps[-1]) > (1e7 if name == "c3" else 1e10)


def test_validate_rejects_pointer_outside_allocation():
    recs = [{"op": "alloc", "id": 0, "bytes": 16},
            {"op": "d2d", "t": [0, 8], "s": [0, 0], "bytes": 16}]
    with pytest.raises(replay.ReplayError):
        replay.validate(recs)
    recs[1]["bytes"] = 8
    replay.validate(recs)
    recs.append({"op": "free", "id": 0})
    recs.append({"op": "fill", "dtype": 0, "t": [0, 0], "count": 1, "value": "00000000"})
    with pytest.raises(replay.ReplayError):
        replay.validate(recs)


@pytest.mark.parametrize("kind", ["matmul_strided", "layer_norm_rows", "elementwise", "causal_attention",
                                  "adam_step_many", "scatter_add"])
def test_validate_rejects_overrunning_extents(kind):
    """A record whose sizes or strides reach past an allocation is refused on the CPU before any
    launch, for each kind of extent: strided products, row kernels, element layouts, attention,
    the Adam table, index operands. The unmodified C4 record of that kind passes."""
    import copy
    import gzip
    import json

    recs = [json.loads(line) for line in gzip.open(GOLDEN / "c4_step_calls.jsonl.gz", "rt")]
    at = next(i for i, r in enumerate(recs) if r["op"] == kind)
    replay.validate(recs[:at + 1])
    bad = copy.deepcopy(recs[:at + 1])
    r = bad[at]
    # twice the size along one dim: past the allocation (the caching allocator's blocks round up to
    # powers of two, so one more row may still fit)
    if kind == "matmul_strided":
        r["sizes"][1] *= 2  # output rows
    elif kind == "layer_norm_rows":
        r["rows"] *= 2
    elif kind == "elementwise":
        r["layout"]["count"] *= 2
        r["layout"]["shape"][0] *= 2
    elif kind == "causal_attention":
        r["length"] *= 2
    elif kind == "adam_step_many":
        r["tensors"][0]["count"] *= 2
    else:
        r["layout"]["count"] *= 2
        r["layout"]["shape"][0] *= 2
    with pytest.raises(replay.ReplayError):
        replay.validate(bad)


class _HostBuffer:
    def __init__(self, n):
        self.data = bytearray(n)
        self.nbytes = n
        self.ptr = id(self.data)


class _StandIn:
    """Enough of kd.Backend to bind a trace without a device: allocations are host bytes, the
    library's calls are never made (binding only builds the argument structures)."""

    class _Lib:
        def __getattr__(self, name):
            return lambda *a: 0

    def __init__(self):
        self.lib = self._Lib()

    def empty(self, shape, dtype):
        return _HostBuffer(int(shape[0]))

    def check(self, rc, what=""):
        assert rc == 0, what

    def synchronize(self):
        pass


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_every_record_binds(name):
    """Every record of the trace turns into a bound C-ABI call (no kind left unknown), so a GPU replay
    cannot stop half way on a record it does not know."""
    recs = replay.load(GOLDEN / f"{name}_step_calls.jsonl.gz")
    rp = replay.Replay(_StandIn(), recs)
    kinds = {r["op"] for r, (call, _) in zip(recs, rp.bound) if call is not None}
    assert "alloc" not in kinds and "mark" not in kinds
    assert len([1 for call, _ in rp.bound if call is not None]) == \
        len([r for r in recs if r["op"] not in ("alloc", "free", "mark", "result")])


def test_uploads_replace_the_parameter_copies():
    """C4's parameter uploads given as kael's seed-3 model bind (their sizes match, and where the
    trace recorded the bytes, the LayerNorm ones and zero biases, they equal them); a wrong size, a
    byte that differs from a recorded copy, or an ordinal past the trace's copies is an error."""
    import kd
    import numpy as np

    recs = replay.load(GOLDEN / "c4_step_calls.jsonl.gz")
    params = kd.kael_gpt_parameters(kd.Backend(), 3, 96, 128, 4, 4, 256)
    uploads = {2 + i: a for i, (_, a) in enumerate(params)}
    replay.Replay(_StandIn(), recs, uploads)
    with pytest.raises(replay.ReplayError):
        replay.Replay(_StandIn(), recs, {2: params[0][1][:-1]})
    ln = dict(params)["blocks.0.ln1.weight"]
    with pytest.raises(replay.ReplayError):
        replay.Replay(_StandIn(), recs, {4: ln * 2})  # recorded as ones
    with pytest.raises(replay.ReplayError):
        replay.Replay(_StandIn(), recs, {10**6: np.zeros(4, np.uint8)})

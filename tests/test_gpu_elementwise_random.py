"""Randomised layouts for kd_elementwise against the C oracle (seeded, so every run checks the
same cases). Each case draws an output shape of rank 1-5, an output view (contiguous,
permuted, stepped or offset) and, per input, a broadcast-compatible shape (size-1 dims,
missing leading dims, 0-d) under a view of its own kind, then one op of one, two or three
inputs in a dtype it accepts. This reaches every launch path of the backend (vector path with
and without broadcast inputs, transposed tiles, the generic decode, empty shapes) with the
plan chosen by kd_layout_build, which mirrors kael's TensorIterator. Rule: bit-exact, except
the transcendental ops (rtol 1e-5 / atol 1e-6 in f32). A few large cases (over 32 MiB moved)
take the nontemporal variants.
"""
import numpy as np
import pytest

import kd
from views import View, assert_same, contiguous, run_both

pytestmark = pytest.mark.gpu

OPS = ["PLUS", "MINUS", "TIMES", "DIVIDES", "MAXIMUM", "MINIMUM", "EQUAL", "LESS", "LOGICAL_XOR", "NEGATE",
       "ABSOLUTE", "IS_ZERO", "EXP", "TANH", "CLAMP", "WHERE", "MASKED_FILL", "GELU_TANH_BACKWARD"]
TRANSCENDENTAL = {kd.OP[n] for n in ("EXP", "TANH", "GELU_TANH_BACKWARD")}
SIZES = [1, 1, 2, 3, 5, 8, 16, 33, 64, 130]


def permuted(shape, rng):
    """A view of `shape` over a contiguous tensor whose dims are a permutation of it."""
    rank = len(shape)
    perm = rng.permutation(rank)
    base = contiguous(tuple(shape[p] for p in perm))
    strides = [0] * rank
    for i, p in enumerate(perm):
        strides[p] = base.strides[i]
    return View(tuple(shape), tuple(strides))


def stepped_view(shape, rng):
    """Every step-th element along each dim (steps 1-3) of a larger tensor, with an offset."""
    steps = [int(rng.integers(1, 4)) for _ in shape]
    wide = contiguous(tuple(n * s for n, s in zip(shape, steps)))
    return View(tuple(shape), tuple(st * s for st, s in zip(wide.strides, steps)), int(rng.integers(0, 5)))


def random_view(shape, rng, stepped=True):
    if len(shape) == 0:
        return contiguous(())
    kind = rng.integers(0, 4)
    if kind == 2 and not stepped:
        kind = 1
    if kind == 0:
        return contiguous(shape)
    if kind == 1:
        return permuted(shape, rng)
    if kind == 2:
        return stepped_view(shape, rng)
    v = contiguous(shape)
    return View(v.shape, v.strides, int(rng.integers(1, 9)))


def broadcast_shape(out_shape, rng):
    """An input shape that broadcasts to out_shape (trailing alignment)."""
    if rng.random() < 0.05:
        return ()
    shape = list(out_shape)
    while shape and rng.random() < 0.2:
        shape.pop(0)
    return tuple(1 if rng.random() < 0.25 else n for n in shape)


def dtypes_for(op):
    if op in kd.FLOATING_OPS:
        return [kd.F32, kd.F64]
    return [kd.F32, kd.F64, kd.I64, kd.BOOL]


def make_case(rng, large=False):
    op = kd.OP[OPS[int(rng.integers(0, len(OPS)))]]
    dtype = dtypes_for(op)[int(rng.integers(0, len(dtypes_for(op))))]
    if large:
        out_shape = (2048, 2048 + int(rng.integers(0, 2)) * 4)
    else:
        rank = int(rng.integers(1, 6))
        out_shape = tuple(SIZES[int(rng.integers(0, len(SIZES)))] for _ in range(rank))
        if rng.random() < 0.03:
            out_shape = out_shape[:-1] + (0,)
    views = [random_view(out_shape, rng, stepped=not large)]
    for _ in range(kd.op_inputs(op)):
        views.append(random_view(broadcast_shape(out_shape, rng), rng, stepped=not large))
    return op, dtype, views


CASES = [make_case(np.random.default_rng(seed)) for seed in range(400)]
LARGE = [make_case(np.random.default_rng(10_000 + seed), large=True) for seed in range(6)]


def describe(views):
    return " ".join(f"{v.shape}/{v.strides}+{v.offset}" for v in views)


def check(kdb, oracle, op, dtype, views, seed):
    out_dtype = kd.BOOL if op in kd.COMPARE_OPS else dtype
    p = kd.params(reals=(-0.5, 0.75), integers=(-3, 20)) if op == kd.OP["CLAMP"] else kd.params(reals=(7.0, 0),
                                                                                                 integers=(7, 0))
    rng = np.random.default_rng(seed)
    got, want = run_both(kdb, oracle, views, dtype, out_dtype,
                         lambda lay: kdb.call("elementwise", op, out_dtype, dtype, lay, p),
                         lambda lay: oracle.oracle_elementwise(op, out_dtype, dtype, lay, p), rng, op)
    tol = (1e-5, 1e-6) if dtype == kd.F32 else (1e-12, 1e-14)
    name = kd.OPS[op] if op < len(kd.OPS) else "GELU_TANH_BACKWARD"
    assert_same(got, want, op not in TRANSCENDENTAL, *tol, what=f"{name} dtype {dtype}: {describe(views)}")


@pytest.mark.parametrize("block", range(8))
def test_random_layouts(kdb, oracle, block):
    for i in range(block * 50, (block + 1) * 50):
        check(kdb, oracle, *CASES[i], seed=i)


@pytest.mark.parametrize("i", range(len(LARGE)))
def test_random_large_layouts(kdb, oracle, i):
    check(kdb, oracle, *LARGE[i], seed=10_000 + i)


def test_the_cases_reach_every_layout_kind():
    """The generator covers what the kernels distinguish: broadcast inputs, 0-d inputs, permuted
    (transposed) and stepped views, offsets, empty outputs, and ranks 1 to 5."""
    views = [v for _, _, vs in CASES for v in vs]
    assert any(len(v.shape) == 0 for v in views)
    assert any(vs[i].shape != vs[0].shape for _, _, vs in CASES for i in range(1, len(vs)))
    assert any(v.offset > 0 for v in views)
    assert any(list(v.strides) != list(contiguous(v.shape).strides) for v in views)
    assert any(0 in vs[0].shape for _, _, vs in CASES)
    assert {len(vs[0].shape) for _, _, vs in CASES} == {1, 2, 3, 4, 5}

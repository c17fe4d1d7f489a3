"""prod / all / any / argmax / argmin / cumsum through kael with the optional device branches
(oracle/kael_fused.py: reference src/ops/reduce.cpp:362-369,399-451 and src/ops/sequence.cpp:95-117
run these through a host copy; the branches call the backend's kd_reduce PROD / ALL / ANY,
kd_arg_reduce and kd_cumsum), against kael's own CPU path in the same process, on the CPU with the
C oracle as kael's device.

The cases reach what the golden suite does not: chunks long enough for the split paths, every
reduced-dim position (kept-first permutation copies), transposed inputs, NaN and ties (the first
NaN / the first extreme wins), wrapping int64 products and sums, bool inputs and empty chunks.
Integer, bool and position results must be identical; float products within the reference's
f32 / f64 tolerances (kael accumulates in double in its own order); a float cumsum within the
error bound of kael's sequential float sum, k * u * sum|x| at position k (the device sums in
double).
"""
import numpy as np
import pytest

import support

# (op, args, shape, dtype, fill, view). fill names how the input is drawn (make_input).
CASES = [
    ("prod", "dims:1", (64, 300), np.float32, "near_one", "none"),
    ("prod", "dims:0,2,keepdim:1", (3, 4, 5), np.float64, "uniform", "none"),
    ("prod", "", (1 << 16,), np.float32, "near_one", "none"),
    ("prod", "dims:0", (40, 33), np.int64, "small_int", "transpose:0:1"),
    ("prod", "", (1000,), np.int64, "large_int", "none"),
    ("prod", "dims:0", (7, 9), np.bool_, "bool", "none"),
    ("all", "dims:1", (512, 33), np.bool_, "mostly_true", "none"),
    ("all", "", (5000,), np.float32, "nan_and_zero", "none"),
    ("all", "dims:0", (17, 1000), np.int64, "small_int", "none"),
    ("all", "dims:0", (0, 5), np.float32, "uniform", "none"),
    ("any", "dims:1", (512, 33), np.bool_, "mostly_false", "none"),
    ("any", "", (70000,), np.float64, "zeros_one_nan", "none"),
    ("any", "dims:1", (3, 0), np.int64, "small_int", "none"),
    ("any", "dims:0,keepdim:1", (100, 6), np.float32, "mostly_zero", "transpose:0:1"),
    ("argmax", "dim:1", (300, 1000), np.float32, "ties", "none"),
    ("argmax", "dim:0,keepdim:1", (513, 40), np.float64, "uniform", "none"),
    ("argmax", "", (1 << 18,), np.float32, "nans", "none"),
    ("argmax", "dim:1", (6, 5000), np.int64, "ties", "transpose:0:1"),
    ("argmax", "dim:0", (9, 70), np.bool_, "bool", "none"),
    ("argmin", "dim:1", (300, 1000), np.float32, "ties", "none"),
    ("argmin", "", (100003,), np.float64, "nans", "none"),
    ("argmin", "dim:-1", (4, 5, 6), np.int64, "small_int", "permute:2:0:1"),
    ("cumsum", "dim:1", (5, 5000), np.float32, "uniform", "none"),
    ("cumsum", "dim:0", (300, 7), np.float64, "uniform", "none"),
    ("cumsum", "dim:1", (4, 100000), np.int64, "large_int", "none"),
    ("cumsum", "dim:1", (64, 257), np.bool_, "bool", "none"),
    ("cumsum", "dim:0", (3, 0), np.float32, "uniform", "none"),
    ("cumsum", "dim:-1", (40, 30), np.float32, "uniform", "transpose:0:1"),
]


def make_input(shape, dtype, fill, seed):
    rng = np.random.default_rng(seed)
    n = int(np.prod(shape))
    if fill == "uniform":
        x = rng.uniform(-1, 1, n)
    elif fill == "near_one":
        x = 1 + rng.uniform(-1e-3, 1e-3, n)
    elif fill == "small_int":
        x = rng.integers(-3, 4, n)
    elif fill == "large_int":
        x = rng.integers(-(1 << 62), 1 << 62, n)
    elif fill == "bool":
        x = rng.random(n) < 0.5
    elif fill == "mostly_true":
        x = rng.random(n) < 0.98
    elif fill == "mostly_false":
        x = rng.random(n) < 0.02
    elif fill == "mostly_zero":
        x = np.where(rng.random(n) < 0.01, rng.uniform(-1, 1, n), 0.0)
    elif fill == "nan_and_zero":
        x = rng.uniform(0.5, 1, n)
        x[rng.integers(0, n, 3)] = np.nan
        x[n // 2 + 7] = 0.0
    elif fill == "zeros_one_nan":
        x = np.zeros(n)
        x[n - 3] = np.nan
    elif fill == "ties":
        x = rng.integers(-5, 6, n)
    elif fill == "nans":
        x = rng.uniform(-1, 1, n)
        x[[n // 3, n // 3 + 11, n - 1]] = np.nan
    else:
        raise ValueError(fill)
    return x.astype(dtype).reshape(shape)


def run_case(lib, index):
    op, args, shape, dtype, fill, view = CASES[index]
    x = make_input(shape, dtype, fill, 1000 + index)
    bound = max(1024, x.size * 8)
    cpu = support.run_op(lib, op, args, [x], [view], 0, bound)
    dev = support.run_op(lib, op, args, [x], [view], 1, bound)
    return x, cpu, dev


def check(case, x, cpu, dev):
    op, args, shape, dtype, fill, view = case
    assert dev.shape == cpu.shape and dev.dtype == cpu.dtype, (dev.shape, dev.dtype, cpu.shape, cpu.dtype)
    if cpu.dtype.kind in "iub" or op in ("argmax", "argmin", "all", "any"):
        np.testing.assert_array_equal(dev, cpu)
    elif op == "prod":
        ok, msg = support.golden_close(dev, cpu)
        assert ok, msg
    else:  # float cumsum: kael sums sequentially in the element type
        axis = int(args.split(":")[1])
        v = support.apply_view(x, view)
        u = np.finfo(cpu.dtype).eps / 2
        positions = np.arange(1, v.shape[axis] + 1).reshape([-1 if d == axis % v.ndim else 1 for d in range(v.ndim)])
        limit = positions * u * np.cumsum(np.abs(v.astype(np.float64)), axis=axis) + np.finfo(cpu.dtype).tiny
        assert np.all(np.abs(dev.astype(np.float64) - cpu.astype(np.float64)) <= limit)


@pytest.mark.parametrize("index", range(len(CASES)),
                         ids=[f"{c[0]}-{np.dtype(c[3]).name}-{'x'.join(map(str, c[2]))}-{c[5].split(':')[0]}"
                              for c in CASES])
def test_device_branch_matches_kael_cpu(kael_oracle_fused, index):
    x, cpu, dev = run_case(kael_oracle_fused, index)
    check(CASES[index], x, cpu, dev)


def test_every_case_runs_through_the_branches(kael_oracle_fused):
    """The oracle backend counts its extension calls (numbered in oracle/oracle_backend.cpp)."""
    from test_oracle_kael_fused import calls
    counted = {"prod": "reduce_extra", "all": "reduce_extra", "any": "reduce_extra", "argmax": "arg_reduce",
               "argmin": "arg_reduce", "cumsum": "cumsum_rows"}
    for index, case in enumerate(CASES):
        x = make_input(case[2], case[3], case[4], 1000 + index)
        before = calls(kael_oracle_fused)[counted[case[0]]]
        support.run_op(kael_oracle_fused, case[0], case[1], [x], [case[5]], 1, max(1024, x.size * 8))
        ran = calls(kael_oracle_fused)[counted[case[0]]] - before
        # Empty inputs never reach the device: cumsum returns early, and the reductions launch
        # nothing for zero outputs (the call itself still happens for zero-size chunks).
        assert ran == (0 if case[0] == "cumsum" and x.size == 0 else 1), (case, ran)


def test_planted_mistake_is_caught():
    """A last-NaN-wins argmax and a float cumsum off by 1e-4 fail the comparisons above."""
    x = make_input((1 << 18,), np.float32, "nans", 7)
    want = np.array(np.argmax(np.isnan(x)))
    wrong = np.array(len(x) - 1)
    with pytest.raises(AssertionError):
        check(CASES[16], x, want, wrong)
    v = make_input((5, 5000), np.float32, "uniform", 8)
    good = np.cumsum(v, axis=1, dtype=np.float32)
    with pytest.raises(AssertionError):
        check(CASES[22], v, good, good + np.float32(1e-4))

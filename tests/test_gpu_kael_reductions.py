"""prod / all / any / argmax / argmin / cumsum through kael with the optional device branches on
the MI355X (kd_reduce PROD / ALL / ANY, kd_arg_reduce, kd_cumsum in place of kael's host copies,
reference src/ops/reduce.cpp:362-369,399-451, src/ops/sequence.cpp:95-117), against kael's CPU
path in the same process: the cases of test_oracle_kael_reductions.py plus config-sized ones
(C2's [4096, 4096] along both dims, a 2^24-element argmax and product, long cumsum rows) that
take the kernels' split and segmented paths. The same comparison rules: identical integers, bools
and positions; float products within the reference's tolerances; float cumsum within kael's
sequential-sum error bound.
"""
import numpy as np
import pytest

import support
from test_oracle_kael_reductions import CASES, check, make_input, run_case

pytestmark = pytest.mark.gpu

LARGE = [
    ("argmax", "dim:1", (4096, 4096), np.float32, "uniform", "none"),
    ("argmin", "dim:0", (4096, 4096), np.float32, "ties", "none"),
    ("argmax", "", (1 << 24,), np.float32, "nans", "none"),
    ("prod", "", (1 << 24,), np.float64, "near_one", "none"),
    ("all", "dims:1", (4096, 4096), np.float32, "nan_and_zero", "none"),
    ("any", "", (1 << 24,), np.bool_, "mostly_false", "none"),
    ("cumsum", "dim:1", (16, 1 << 20), np.int64, "large_int", "none"),
    ("cumsum", "dim:1", (4, 200000), np.float32, "uniform", "none"),
]


@pytest.mark.parametrize("index", range(len(CASES)),
                         ids=[f"{c[0]}-{np.dtype(c[3]).name}-{'x'.join(map(str, c[2]))}-{c[5].split(':')[0]}"
                              for c in CASES])
def test_device_branch_matches_kael_cpu(kael_hip_fused, index):
    x, cpu, dev = run_case(kael_hip_fused, index)
    check(CASES[index], x, cpu, dev)


@pytest.mark.parametrize("case", LARGE, ids=[f"{c[0]}-{np.dtype(c[3]).name}-{'x'.join(map(str, c[2]))}"
                                             for c in LARGE])
def test_config_sized_inputs(kael_hip_fused, case):
    op, args, shape, dtype, fill, view = case
    x = make_input(shape, dtype, fill, 77)
    bound = max(1024, x.size * 8)
    cpu = support.run_op(kael_hip_fused, op, args, [x], [view], 0, bound)
    dev = support.run_op(kael_hip_fused, op, args, [x], [view], 1, bound)
    check(case, x, cpu, dev)

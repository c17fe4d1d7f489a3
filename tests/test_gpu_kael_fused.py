"""kael with the optional device branches that call the backend's fused entry points
(oracle/kael_fused.py applies them to a test build: softmax / log_softmax / standardize as row
kernels, cross-entropy losses and gradient in one kernel each, GELU backward as one element op,
matmul reading transposed and batch-broadcast operands in place).

The same checks as for unmodified kael: its golden suite (783 PyTorch known answers, reference
tests/test_golden.cpp:236-292 tolerances), its 36 device-behaviour cases (reference
tests/test_cuda.cpp) and the C3 / C4 training configs against kael's CPU path from the same seeds
(every step's loss within 1e-4 relative; C3's final parameters too). The training tests also
report the step time next to unmodified kael on the same device.
"""
import ctypes

import numpy as np
import pytest

import support
from test_oracle_device_suite import NAMES

pytestmark = pytest.mark.gpu

CASES = support.golden_cases()


def test_golden_suite_through_the_fused_branches(kael_hip_fused):
    failures = []
    for case in CASES:
        try:
            got, want = support.run_golden(kael_hip_fused, case, 1)
            ok, msg = support.golden_close(got, want)
        except Exception as e:  # a kael::Error from the backend is a failure too
            ok, msg = False, str(e)
        if not ok:
            failures.append(f"{case['op']}/{case['case']}: {msg}")
    assert not failures, f"{len(failures)} of {len(CASES)} cases:\n" + "\n".join(failures[:40])


@pytest.mark.parametrize("name", NAMES)
def test_device_case_through_the_fused_branches(kael_hip_fused, name):
    support.run_suite_case(kael_hip_fused, name)


def _mlp(lib, device, steps=100):
    losses, params, seconds = np.zeros(steps, np.float32), np.zeros(101770, np.float32), ctypes.c_double()
    assert lib.ref_train_mlp(device, steps, losses.ctypes.data_as(ctypes.c_void_p),
                             params.ctypes.data_as(ctypes.c_void_p), ctypes.byref(seconds)) == 0, support.ref_error(lib)
    return losses, params, seconds.value


def _chargpt(lib, device, steps):
    losses, seconds = np.zeros(steps, np.float32), ctypes.c_double()
    assert lib.ref_train_chargpt(device, steps, losses.ctypes.data_as(ctypes.c_void_p),
                                 ctypes.byref(seconds)) == 0, support.ref_error(lib)
    return losses, seconds.value


def test_c3_mlp_through_the_fused_branches(kael_hip_fused, kael_hip):
    cpu_l, cpu_p, tc = _mlp(kael_hip_fused, 0)
    _mlp(kael_hip_fused, 1)  # loads kernels, fills kael's block cache
    gpu_l, gpu_p, tg = _mlp(kael_hip_fused, 1)
    _mlp(kael_hip, 1)
    _, _, tu = _mlp(kael_hip, 1)
    np.testing.assert_allclose(gpu_l, cpu_l, rtol=1e-4)
    np.testing.assert_allclose(gpu_p, cpu_p, rtol=1e-4, atol=1e-5)
    print(f"\nC3 MLP 100 SGD steps: CPU {tc:.3f} s; MI355X with the fused branches {tg:.3f} s, "
          f"unmodified kael {tu:.3f} s")


def test_c4_char_gpt_through_the_fused_branches(kael_hip_fused, kael_hip):
    steps = 3
    _chargpt(kael_hip_fused, 1, steps)
    gpu_l, tg = _chargpt(kael_hip_fused, 1, steps)
    _chargpt(kael_hip, 1, steps)
    _, tu = _chargpt(kael_hip, 1, steps)
    cpu_l, tc = _chargpt(kael_hip_fused, 0, steps)
    np.testing.assert_allclose(gpu_l, cpu_l, rtol=1e-4)
    print(f"\nC4 char-GPT {steps} Adam steps: CPU {tc / steps:.3f} s/step; MI355X with the fused branches "
          f"{tg / steps:.4f} s/step, unmodified kael {tu / steps:.4f} s/step")

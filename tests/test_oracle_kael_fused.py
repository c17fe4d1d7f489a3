"""kael's optional device branches (oracle/kael_fused.py: softmax / log_softmax / standardize as
row kernels, cross-entropy losses and gradient in one call each, GELU backward as one element op,
matmul over strided operands, the fused optimizer steps, and prod / all / any / argmax / argmin /
cumsum on the device instead of through a host copy) checked on the CPU, with the C oracle as
kael's device.

kael's golden suite (783 PyTorch known answers, reference tests/test_golden.cpp:236-292
tolerances), its 36 device-behaviour cases (reference tests/test_cuda.cpp) and 100 steps of the C3
MLP against kael's CPU path must all pass through the patched branches, and each branch must
actually have run: the oracle backend counts the calls of every fused entry point.
"""
import ctypes

import numpy as np
import pytest

import support
from test_oracle_device_suite import NAMES

CASES = support.golden_cases()
# Numbered as the oracle backend counts them (oracle/oracle_backend.cpp).
EXTENSIONS = ["softmax_rows", "standardize_rows", "cross_entropy_rows", "cross_entropy_grad", "gelu_backward_op",
              "matmul_strided", "adam_step", "sgd_step", "reduce_extra", "arg_reduce", "cumsum_rows",
              "softmax_rows_backward", "standardize_rows_backward", "reduce_columns", "adam_step_many",
              "matmul_strided_heads", "layer_norm_rows", "layer_norm_rows_backward", "matmul_strided_bias",
              "index_bounds", "causal_attention", "causal_attention_backward", "dropout", "cached_attention"]
# The entry points a char-GPT training step reaches (forward, backward, Adam over the parameter list;
# layer_norm_rows(_backward): every LayerNorm; reduce_columns: the bias gradients summed over every
# token; matmul_strided_heads: the attention products over per-head views; matmul_strided_bias: every
# Linear with a bias; index_bounds: the range checks of the token and position ids and of the targets).
TRAINING = ["softmax_rows", "layer_norm_rows", "cross_entropy_rows", "cross_entropy_grad", "gelu_backward_op",
            "matmul_strided", "adam_step_many", "softmax_rows_backward", "layer_norm_rows_backward", "reduce_columns",
            "matmul_strided_heads", "matmul_strided_bias", "index_bounds"]


def calls(lib):
    fn = lib.ref_extension_calls
    fn.restype, fn.argtypes = ctypes.c_longlong, [ctypes.c_int]
    return {name: fn(i) for i, name in enumerate(EXTENSIONS)}


def test_golden_suite_through_the_fused_branches(kael_oracle_fused):
    before = calls(kael_oracle_fused)
    failures = []
    for case in CASES:
        try:
            got, want = support.run_golden(kael_oracle_fused, case, 1)
            ok, msg = support.golden_close(got, want)
        except Exception as e:
            ok, msg = False, str(e)
        if not ok:
            failures.append(f"{case['op']}/{case['case']}: {msg}")
    assert not failures, f"{len(failures)} of {len(CASES)} cases:\n" + "\n".join(failures[:40])
    after = calls(kael_oracle_fused)
    # The golden manifest holds tensor ops (no layer norm, cross-entropy or gradients): of the fused
    # branches it reaches softmax / log_softmax, the products, and prod / all / any / argmax / argmin
    # (20 all, 20 any, 14 prod, 8 argmax and 8 argmin cases, every one now computed on the device).
    for name in ("softmax_rows", "matmul_strided", "reduce_extra", "arg_reduce"):
        assert after[name] > before[name], f"{name} never ran: {after}"


@pytest.mark.parametrize("name", NAMES)
def test_device_case_through_the_fused_branches(kael_oracle_fused, name):
    before = calls(kael_oracle_fused)
    support.run_suite_case(kael_oracle_fused, name)
    if name == "sequence_ops_match_cpu":  # cumsum of a device tensor (reference tests/test_cuda.cpp:576)
        assert calls(kael_oracle_fused)["cumsum_rows"] > before["cumsum_rows"]


def test_c3_mlp_through_the_fused_branches_matches_cpu(kael_oracle_fused):
    lib = kael_oracle_fused
    steps = 100
    cpu_l, gpu_l = np.zeros(steps, np.float32), np.zeros(steps, np.float32)
    cpu_p, gpu_p = np.zeros(101770, np.float32), np.zeros(101770, np.float32)
    t = ctypes.c_double()
    assert lib.ref_train_mlp(0, steps, cpu_l.ctypes.data_as(ctypes.c_void_p), cpu_p.ctypes.data_as(ctypes.c_void_p),
                             ctypes.byref(t)) == 0, support.ref_error(lib)
    before = calls(lib)
    assert lib.ref_train_mlp(1, steps, gpu_l.ctypes.data_as(ctypes.c_void_p), gpu_p.ctypes.data_as(ctypes.c_void_p),
                             ctypes.byref(t)) == 0, support.ref_error(lib)
    after = calls(lib)
    np.testing.assert_allclose(gpu_l, cpu_l, rtol=1e-4)
    np.testing.assert_allclose(gpu_p, cpu_p, rtol=1e-4, atol=1e-5)
    # Per step: one loss and one gradient call, and the Linear products x . W^T with W^T read in place.
    assert after["cross_entropy_rows"] - before["cross_entropy_rows"] == steps
    assert after["cross_entropy_grad"] - before["cross_entropy_grad"] == steps
    assert after["matmul_strided"] - before["matmul_strided"] >= 2 * steps


def test_small_gpt_training_through_every_fused_branch_matches_cpu(kael_oracle_fused):
    """A char-GPT small enough for the scalar oracle (vocab 96, context 16, 2 layers, 2 heads,
    dim 32, batch 4; config C4's structure): 3 Adam steps through the patched branches against
    kael's CPU path, and every fused entry point runs (attention softmax, the LayerNorms, the
    cross-entropy and its gradient, GELU backward, products with W^T and the attention's K^T
    read in place)."""
    lib = kael_oracle_fused
    steps = 3
    args = (steps, 96, 16, 2, 2, 32, 4)
    cpu_l, dev_l = np.zeros(steps, np.float32), np.zeros(steps, np.float32)
    t = ctypes.c_double()
    assert lib.ref_train_gpt(0, *args, cpu_l.ctypes.data_as(ctypes.c_void_p), ctypes.byref(t)) == 0, support.ref_error(lib)
    before = calls(lib)
    assert lib.ref_train_gpt(1, *args, dev_l.ctypes.data_as(ctypes.c_void_p), ctypes.byref(t)) == 0, support.ref_error(lib)
    after = calls(lib)
    np.testing.assert_allclose(dev_l, cpu_l, rtol=1e-4)
    ran = {name: after[name] - before[name] for name in TRAINING}
    assert all(n > 0 for n in ran.values()), ran

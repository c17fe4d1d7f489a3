"""kael's device-behaviour cases (oracle/device_suite.cpp, restating reference
tests/test_cuda.cpp:133-623) on the CPU: once with the reference's own host emulation of its
device tasks (src/cuda/backend_fake.cpp), which shows every case holds for kael's reference
device semantics, and once with the C oracle as the device, which pins the oracle at the level
of kael's whole tensor API (transfers, autograd, modules, optimizers, generation).
"""
import pytest

import support

NAMES = [
    "transfers_round_trip", "same_device_returns_the_same_tensor", "non_contiguous_tensors_transfer",
    "factories_create_on_the_device", "host_only_access_fails_clearly", "reading_values_copies_to_host",
    "mixed_devices_are_rejected", "scalars_follow_the_tensor_device", "copy_between_devices_works",
    "unary_ops_match_cpu_on_every_layout", "double_precision_matches_cpu", "binary_ops_match_cpu_with_broadcast",
    "integer_ops_match_cpu", "bool_reductions_match_cpu", "non_finite_values_match_cpu",
    "long_sums_match_cpu_and_are_deterministic", "empty_tensors_work", "matmul_shapes_match_cpu",
    "matmul_batches_vectors_and_integers_match_cpu", "indexing_matches_cpu", "out_of_range_indices_still_throw",
    "backward_matches_cpu_and_stays_on_the_device", "gradients_cross_devices_back_to_the_origin",
    "view_and_indexing_gradients_match_cpu", "gradcheck_runs_on_the_device",
    "module_to_keeps_parameter_identity_and_values", "module_to_moves_existing_gradients",
    "integer_clamp_and_masked_fill_keep_every_bit", "integer_scatter_add_wraps_around",
    "integer_sum_wraps_and_float_conversion_saturates", "layers_match_cpu", "training_matches_cpu_step_by_step",
    "device_blocks_are_cached", "sequence_ops_match_cpu", "gpt_matches_cpu_including_the_cache_and_generation",
    "stepped_indices_work_on_the_device",
]


def test_the_suite_holds_every_reference_case(refdev):
    """36 cases, one per TEST/TEST_P of the reference's device suite."""
    assert support.suite_cases(refdev) == NAMES


def test_the_comparisons_catch_planted_mismatches(refdev):
    """A wrong value, NaN, infinity sign, shape, dtype, device or integer bit is reported."""
    assert refdev.ref_suite_self_check() == 0


@pytest.mark.parametrize("name", NAMES)
def test_case_on_the_reference_emulation(refdev, name):
    support.run_suite_case(refdev, name)


@pytest.mark.parametrize("name", NAMES)
def test_case_on_the_oracle_device(kael_oracle, name):
    support.run_suite_case(kael_oracle, name)

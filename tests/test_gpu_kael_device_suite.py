"""kael's device-behaviour cases (oracle/device_suite.cpp, restating reference
tests/test_cuda.cpp:133-623) with the MI355X backend as kael's device: transfers, factories,
errors, every unary op on every layout, broadcasting binary ops, integer and non-finite
semantics, matmul shapes, indexing, autograd on the device, module moves, AdamW training,
the caching allocator, sequence ops and GPT generation, each against kael's CPU results.
"""
import pytest

import support
from test_oracle_device_suite import NAMES

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", NAMES)
def test_case_on_the_mi355x_backend(kael_hip, name):
    support.run_suite_case(kael_hip, name)

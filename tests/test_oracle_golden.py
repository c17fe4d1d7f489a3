"""Pins the C oracle (oracle/kd_oracle.c) with the reference's golden suite.

The reference kael core, compiled unmodified, runs each of the 783 golden cases
(tests/golden/manifest.txt, PyTorch known answers) with every input on its "device", where
kael::device is implemented by the oracle (oracle/oracle_backend.cpp). kael's own host code
(TensorIterator, reduction planning, indexing) thus drives the restated device semantics, and
the answers must match PyTorch at the reference's tolerances (tests/support/allclose.h:21-32).
The same run on the reference's own host emulation of its device tasks (src/cuda/backend_fake.cpp)
is the control: both must pass the same cases.
"""
import pytest

import support

CASES = support.golden_cases()
OPS = sorted({c["op"] for c in CASES})


def _run(lib, op, device):
    failures = []
    for case in (c for c in CASES if c["op"] == op):
        try:
            got, want = support.run_golden(lib, case, device)
            ok, msg = support.golden_close(got, want)
        except Exception as e:
            ok, msg = False, str(e)
        if not ok:
            failures.append(f"{op}/{case['case']}: {msg}")
    return failures


def test_manifest_size():
    assert len(CASES) == 783


@pytest.mark.parametrize("op", OPS)
def test_oracle_backend_passes_golden(kael_oracle, op):
    failures = _run(kael_oracle, op, 1)
    assert not failures, "\n".join(failures)


@pytest.mark.parametrize("op", ["add", "matmul", "softmax", "sum", "gather", "scatter_add_", "where", "max"])
def test_reference_emulation_passes_golden(refdev, op):
    failures = _run(refdev, op, 1)
    assert not failures, "\n".join(failures)


@pytest.mark.parametrize("op", ["add", "matmul", "softmax", "log_softmax", "gelu_tanh", "sum", "max"])
def test_reference_cpu_path_passes_golden(refdev, op):
    failures = _run(refdev, op, 0)
    assert not failures, "\n".join(failures)

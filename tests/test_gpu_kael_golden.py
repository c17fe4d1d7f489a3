"""kael's own golden suite (reference tests/golden/manifest.txt, 783 PyTorch known answers; runner
semantics of tests/test_golden.cpp:236-292) run through kael's unmodified host code with every
input on the device, i.e. through kael.cpp_amd/host/backend_hip.cpp and the HIP kernels.

This is the drop-in check: kael's TensorIterator, reduction planning, autograd-free ops and
indexing issue their device calls exactly as they would to any backend, and the answers must
match PyTorch with the reference's tolerances (f32 rtol 1e-5 / atol 1e-6, f64 1e-12 / 1e-14,
exact for int64 and bool).
"""
import pytest

import support

pytestmark = pytest.mark.gpu

CASES = support.golden_cases()


@pytest.mark.parametrize("op", sorted({c["op"] for c in CASES}))
def test_golden_cases_on_device(kael_hip, op):
    failures = []
    for case in (c for c in CASES if c["op"] == op):
        try:
            got, want = support.run_golden(kael_hip, case, 1)
            ok, msg = support.golden_close(got, want)
        except Exception as e:  # a kael::Error from the backend is a failure too
            ok, msg = False, str(e)
        if not ok:
            failures.append(f"{op}/{case['case']}: {msg}")
    assert not failures, "\n".join(failures)

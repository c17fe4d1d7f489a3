import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parent))

import support  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def oracle():
    if not support.ORACLE_LIB.is_file():
        pytest.fail(f"{support.ORACLE_LIB} missing: run `python -c 'import __graft_entry__ as g; g.build()'`")
    return support.load_oracle()


def _ref_or_skip(variant):
    path = support.ref_path(variant)
    if not path.is_file():
        pytest.skip(f"{path.name} not built (needs the reference sources at build time)")
    return support.load_ref(variant)


@pytest.fixture(scope="session")
def refdev():
    """kael core + the reference's host emulation of its device tasks."""
    return _ref_or_skip("ref")


@pytest.fixture(scope="session")
def kael_oracle():
    """kael core + kael::device implemented by the C oracle."""
    return _ref_or_skip("oracle")


@pytest.fixture(scope="session")
def kdb():
    """The MI355X backend; GPU tests only."""
    import kd

    backend = kd.load()
    if not backend.lib.kd_available():
        pytest.fail(f"no usable gfx950 device: {backend.error()}")
    return backend


@pytest.fixture(scope="session")
def kael_hip(kdb):
    """kael core + kael::device implemented by the MI355X backend; GPU tests only."""
    return _ref_or_skip("hip")


@pytest.fixture(scope="session")
def kael_oracle_fused():
    """kael with its optional device branches (oracle/kael_fused.py) over the C oracle: the
    patched branches checked on the CPU."""
    return _ref_or_skip("oracle_fused")


@pytest.fixture(scope="session")
def kael_hip_fused(kdb):
    """The same with kael's optional device branches applied (oracle/kael_fused.py): softmax,
    log_softmax, standardize, cross-entropy and GELU backward call the fused entry points and
    matmul reads strided operands in place; GPU tests only."""
    return _ref_or_skip("hip_fused")

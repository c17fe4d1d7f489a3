"""The gradients of Linear-shaped products (y = x . W^T, x [B, M, K], W [N, K]; reference
src/nn/layers.cpp:42-43, MatmulBackward src/autograd/functions_linalg.cpp:29-49) through kael's
optional device branches with the C oracle as the device: the weight gradient's fold over the batch
(one product X_flat^T . g_flat) and the strided products, element by element against kael's CPU
path (the reference's f32 device tolerance 1e-4 + 1e-4 |cpu|, tests/test_cuda.cpp:40-43). The
fold branch must run (the strided-product counter moves) and an empty last dim must fall back to
kael's own path.
"""
import ctypes
import os

import numpy as np
import pytest

import support
from test_gpu_kael_gradients import SELECT_CASES, assert_reference_close, linear_grads, select_grads

SHAPES = [(3, 37, 53, 29), (5, 1, 7, 3), (2, 30, 64, 48), (4, 16, 32, 24)]


@pytest.mark.parametrize("shape", SHAPES, ids=["x".join(map(str, s)) for s in SHAPES])
def test_linear_gradients_through_the_fused_branches(kael_oracle_fused, shape):
    lib = kael_oracle_fused
    fn = lib.ref_extension_calls
    fn.restype, fn.argtypes = ctypes.c_longlong, [ctypes.c_int]
    cpu_w, cpu_x = linear_grads(lib, 0, shape)
    before = fn(5)  # matmul_strided
    dev_w, dev_x = linear_grads(lib, 1, shape)
    assert fn(5) > before
    assert_reference_close(dev_w, cpu_w, "W.grad")
    assert_reference_close(dev_x, cpu_x, "x.grad")


@pytest.mark.parametrize("shape", [(2, 3, 0, 4), (2, 3, 5, 0)], ids=["k0", "n0"])
def test_empty_last_dim_keeps_kaels_path(kael_oracle_fused, shape):
    b, m, k, n = shape
    wg, xg = np.ones((n, k), np.float32), np.ones((b, m, k), np.float32)
    assert kael_oracle_fused.ref_linear_grads(1, b, m, k, n, 3, support.ptr(wg), support.ptr(xg)) == 0, \
        support.ref_error(kael_oracle_fused)
    assert not wg.any() and not xg.any()


@pytest.mark.parametrize("shape", [(3, 37, 53, 29), (2, 1, 7, 3), (4, 16, 32, 24)], ids=["3x37x53x29", "2x1x7x3", "4x16x32x24"])
def test_head_gradients_through_the_fused_branches(kael_oracle_fused, shape):
    """The tied head's weight . h^T with the left-operand gradient folded over the batch (one
    product) against kael's CPU path, on the oracle device."""
    from test_gpu_kael_gradients import head_grads

    lib = kael_oracle_fused
    cpu_w, cpu_h = head_grads(lib, 0, shape)
    dev_w, dev_h = head_grads(lib, 1, shape)
    assert_reference_close(dev_w, cpu_w, "W.grad")
    assert_reference_close(dev_h, cpu_h, "h.grad")


@pytest.mark.parametrize("shape", [(2, 3, 0, 4), (2, 0, 5, 4), (2, 3, 5, 0)], ids=["k0", "m0", "n0"])
def test_head_empty_dims_keep_kaels_path(kael_oracle_fused, shape):
    b, m, k, n = shape
    wg, hg = np.ones((n, k), np.float32), np.ones((b, m, k), np.float32)
    assert kael_oracle_fused.ref_head_grads(1, b, m, k, n, 3, support.ptr(wg), support.ptr(hg)) == 0, \
        support.ref_error(kael_oracle_fused)
    assert not wg.any() and not hg.any()


@pytest.mark.parametrize("which", range(len(SELECT_CASES)), ids=SELECT_CASES)
def test_select_gradients_through_the_fused_branches(kael_oracle_fused, which):
    """Deferred select gradients on the oracle device equal kael's CPU path value for value,
    including the slices no select reached (zeros), repeated indices (summed), gradients of the
    whole tensor mixed in, a retained intermediate and anomaly detection (deferral off)."""
    cpu_x, cpu_p = select_grads(kael_oracle_fused, 0, which)
    dev_x, dev_p = select_grads(kael_oracle_fused, 1, which)
    assert np.array_equal(dev_x, cpu_x) and np.array_equal(dev_p, cpu_p)
    if SELECT_CASES[which] in ("two_of_three", "same_index_twice"):
        # one slice of dim 2 has no select: its gradient is zero
        assert not cpu_x.reshape(2, 3, 3, 4)[:, :, 1 if which == 1 else 2].any()


def test_select_gradients_reject_unknown_case(kael_oracle_fused):
    xg, pg = np.empty(72, np.float32), np.empty(72, np.float32)
    assert kael_oracle_fused.ref_select_grads(1, 99, 1, support.ptr(xg), support.ptr(pg)) != 0


_TRACE_SELECT = """
import ctypes, sys
import numpy as np
lib = ctypes.CDLL(sys.argv[1])
xg, pg = np.empty(72, np.float32), np.empty(72, np.float32)
sys.exit(lib.ref_select_grads(1, int(sys.argv[2]), ctypes.c_uint64(11), xg.ctypes.data_as(ctypes.c_void_p),
                              pg.ctypes.data_as(ctypes.c_void_p)))
"""


@pytest.mark.parametrize("which, unmodified, fused", [(0, 3, 0), (1, 2, 1), (2, 3, 1)],
                         ids=["attention_split", "two_of_three", "same_index_twice"])
def test_select_gradients_skip_the_zero_fills(tmp_path, which, unmodified, fused):
    """The device calls of one backward pass (the oracle backend's call trace): kael fills a
    zero tensor of the full shape [2, 3, 3, 4] per select; with the select gradients deferred,
    only a full tensor that some slice of the selected dim never reaches is filled (once)."""
    import json
    import subprocess
    import sys

    fills = {}
    for name in ("libkael_oracle.so", "libkael_oracle_fused.so"):
        trace = tmp_path / f"{name}.jsonl"
        env = dict(os.environ, KD_ORACLE_TRACE=str(trace))
        subprocess.run([sys.executable, "-c", _TRACE_SELECT, str(support.REF_DIR / name), str(which)],
                       env=env, check=True, timeout=120)
        recs = [json.loads(line) for line in trace.read_text().splitlines() if line.strip()]
        fills[name] = sum(1 for r in recs if r["op"] == "fill" and r["count"] == 72)
    assert fills == {"libkael_oracle.so": unmodified, "libkael_oracle_fused.so": fused}


def test_select_gradients_with_the_graph_retained_accumulate(kael_oracle_fused):
    """Backward twice over the same graph (retain_graph): each pass defers and writes its own select
    gradients, so x.grad is exactly twice one pass's (g + g rounds to 2g)."""
    once, _ = select_grads(kael_oracle_fused, 1, SELECT_CASES.index("attention_split"))
    twice, _ = select_grads(kael_oracle_fused, 1, SELECT_CASES.index("retained_graph_twice"))
    assert np.array_equal(twice, 2 * once)

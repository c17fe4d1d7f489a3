"""Host-side pieces that need no GPU: the C-ABI library loads and exports every symbol that
include/kd_api.h declares, the struct mirrors have the reference sizes, and kd_layout_build
(the TensorIterator mirror, reference src/iterator.cpp:47-63, 152-172) agrees with kael's own
coalesce_dims and with the oracle's restatement on random broadcast/strided operand sets.
"""
import ctypes
import re

import numpy as np
import pytest

import kd
import support
from views import layout_of

HEADER = support.ROOT / "include" / "kd_api.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(kd_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_match_binding():
    assert declared_functions() == kd.EXPORTED


def test_library_loads_and_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(kd.LIB_PATH))
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, missing


def test_struct_sizes_match_reference():
    # reference include/kael/device_kernels.h:70-94 (ElementLayout 368 B, IndexLayout 272 B)
    assert ctypes.sizeof(kd.ElementLayout) == 368
    assert ctypes.sizeof(kd.IndexLayout) == 272
    assert ctypes.sizeof(kd.MatmulSizes) == 32
    assert ctypes.sizeof(kd.ElementParameters) == 32


def test_no_device_reports_cleanly():
    backend = kd.Backend()
    if backend.lib.kd_available():
        pytest.skip("a device is present")
    p = ctypes.c_void_p()
    assert backend.lib.kd_malloc(ctypes.byref(p), 16) == -3
    assert "device" in backend.error()


def random_operands(rng):
    nd = int(rng.integers(0, 6))
    shape = tuple(int(rng.integers(1, 5)) for _ in range(nd))
    n_ops = int(rng.integers(2, 5))
    views = []
    for op in range(n_ops):
        if op == 0:
            s = shape
        else:
            r = int(rng.integers(0, nd + 1))
            s = tuple(1 if rng.random() < 0.3 else n for n in shape[nd - r:])
        perm = rng.permutation(len(s)) if rng.random() < 0.5 else np.arange(len(s))
        strides = [0] * len(s)
        acc = 1
        for d in reversed(perm.tolist()):
            strides[d] = acc * (2 if rng.random() < 0.2 else 1)
            acc *= s[d] * (2 if rng.random() < 0.2 else 1)
        views.append(type("V", (), {"shape": s, "strides": tuple(strides)}))
    return shape, views


def reference_layout(ref, shape, views, sizes):
    """Broadcast per reference shape.cpp:123-145, then kael::coalesce_dims."""
    nd = len(shape)
    strides = []
    for op, v in enumerate(views):
        full = [0] * nd
        off = nd - len(v.shape)
        for i, (n, st) in enumerate(zip(v.shape, v.strides)):
            if n == shape[i + off]:
                full[i + off] = st * sizes[op]
        strides.append(full)
    n_ops = len(views)
    shp = (ctypes.c_int64 * max(nd, 1))(*shape)
    st = (ctypes.c_int64 * max(nd * n_ops, 1))(*[s for row in strides for s in row])
    out_shape = (ctypes.c_int64 * 8)()
    out_st = (ctypes.c_int64 * 32)()
    n = ref.ref_coalesce(nd, n_ops, shp, st, out_shape, out_st)
    assert n >= 0
    if n == 0:  # prepare_loop's empty case, src/iterator.cpp:166-171
        return [1], [[0] for _ in range(n_ops)]
    return [out_shape[d] for d in range(n)], [[out_st[op * 8 + d] for d in range(n)] for op in range(n_ops)]


def test_layout_build_matches_kael_coalesce(refdev, oracle):
    lib = kd.Backend().lib
    rng = np.random.default_rng(0)
    for trial in range(400):
        shape, views = random_operands(rng)
        sizes = [int(rng.choice([1, 4, 8])) for _ in views]
        bases = [0x1000 * (i + 1) for i in range(len(views))]
        mine = layout_of(lib.kd_layout_build, views, sizes, bases)
        theirs = layout_of(oracle.oracle_layout_build, views, sizes, bases)
        want_shape, want_strides = reference_layout(refdev, shape, views, sizes)
        for lay in (mine, theirs):
            assert lay.dims == len(want_shape), (trial, shape)
            assert [lay.shape[d] for d in range(lay.dims)] == want_shape
            for op in range(len(views)):
                assert [lay.strides[op][d] for d in range(lay.dims)] == want_strides[op]
            assert lay.count == int(np.prod(shape)) if shape else lay.count == 1
            assert [lay.base[op] for op in range(len(views))] == bases


def test_layout_build_rejects_bad_broadcast():
    lib = kd.Backend().lib
    views = [type("V", (), {"shape": (3, 4), "strides": (4, 1)}), type("V", (), {"shape": (2, 4), "strides": (4, 1)})]
    with pytest.raises(RuntimeError):
        layout_of(lib.kd_layout_build, views, [4, 4], [0, 0])


def test_c2_layouts():
    """The layouts the C2 config produces: a[4096,4096] + b[4096,1]."""
    lib = kd.Backend().lib
    V = lambda s, st: type("V", (), {"shape": s, "strides": st})  # noqa: E731
    lay = layout_of(lib.kd_layout_build, [V((4096, 4096), (4096, 1)), V((4096, 4096), (4096, 1)), V((4096, 1), (1, 1))],
                    [4, 4, 4], [0, 0, 0])
    assert lay.dims == 2 and list(lay.strides[2])[:2] == [4, 0] and list(lay.strides[1])[:2] == [16384, 4]
    lay = layout_of(lib.kd_layout_build, [V((4096, 4096), (4096, 1)), V((4096, 4096), (1, 4096)), V((4096, 1), (1, 1))],
                    [4, 4, 4], [0, 0, 0])
    assert list(lay.strides[1])[:2] == [4, 16384]
    lay = layout_of(lib.kd_layout_build, [V((4096, 4096), (4096, 1)), V((4096, 4096), (4096, 1))], [4, 4], [0, 0])
    assert lay.dims == 1 and lay.shape[0] == 4096 * 4096

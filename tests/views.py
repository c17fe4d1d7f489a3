"""Strided operand views over flat storages, run through the backend and the oracle.

An operand is (shape, element strides, element offset) into its own flat storage. The same
storages are used on the host (oracle) and on the device (backend); the whole output storage
is compared afterwards, so writes outside the view are caught as well.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

import kd
import support


@dataclass
class View:
    shape: tuple
    strides: tuple
    offset: int = 0

    @property
    def storage_len(self) -> int:
        if any(s == 0 for s in self.shape):
            return self.offset + 1
        return self.offset + 1 + sum((n - 1) * st for n, st in zip(self.shape, self.strides))


def contiguous(shape) -> View:
    strides, acc = [], 1
    for n in reversed(shape):
        strides.append(acc)
        acc *= max(n, 1)
    return View(tuple(shape), tuple(reversed(strides)))


def transposed(shape) -> View:
    """A view of `shape` that is the transpose (last two dims swapped) of a contiguous tensor."""
    base = list(shape)
    base[-1], base[-2] = base[-2], base[-1]
    v = contiguous(base)
    st = list(v.strides)
    st[-1], st[-2] = st[-2], st[-1]
    return View(tuple(shape), tuple(st))


def stepped(shape, step=2, offset=1) -> View:
    """Every `step`-th element along the last dim of a wider contiguous tensor, plus an offset."""
    wide = list(shape)
    wide[-1] = shape[-1] * step
    v = contiguous(wide)
    st = list(v.strides)
    st[-1] *= step
    return View(tuple(shape), tuple(st), offset)


def layout_of(build_fn, views, element_sizes, bases) -> kd.ElementLayout:
    n = len(views)
    ranks = (ctypes.c_int * n)(*[len(v.shape) for v in views])
    shapes = (ctypes.c_int64 * (8 * n))()
    strides = (ctypes.c_int64 * (8 * n))()
    for i, v in enumerate(views):
        for d, (s, st) in enumerate(zip(v.shape, v.strides)):
            shapes[8 * i + d] = s
            strides[8 * i + d] = st
    sizes = (ctypes.c_int * n)(*element_sizes)
    bptr = (ctypes.c_void_p * n)(*bases)
    lay = kd.ElementLayout()
    rc = build_fn(ctypes.byref(lay), n, ranks, shapes, strides, sizes, bptr)
    if rc != 0:
        raise RuntimeError(f"layout build failed ({rc})")
    return lay


def random_values(rng, dtype, n, op=None):
    dt = np.dtype(dtype)
    if dt == np.uint8:
        return rng.integers(0, 2, n).astype(np.uint8)
    if dt == np.int64:
        if op == kd.OP["POWER"]:
            return rng.integers(-3, 6, n).astype(np.int64)
        v = rng.integers(-50, 51, n).astype(np.int64)
        big = rng.random(n) < 0.05
        v[big] = rng.integers(-(2**62), 2**62, int(big.sum()))
        return v
    v = rng.normal(0, 2, n).astype(dt)
    special = rng.random(n) < 0.03
    picks = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0], dt)
    v[special] = rng.choice(picks, int(special.sum()))
    return v


def run_both(kdb, oracle, views, in_dtype, out_dtype, call_kd, call_oracle, rng, op=None, inputs=None):
    """views[0] is the output. Returns (device output storage, oracle output storage). `inputs`
    (optional) gives the input storages instead of values drawn from `rng`."""
    in_np = kd.NUMPY_DTYPE[in_dtype]
    out_np = kd.NUMPY_DTYPE[out_dtype]
    storages = []
    for i, v in enumerate(views):
        if i == 0:
            s = np.full(v.storage_len, 7, out_np) if out_np != np.float32 else np.full(v.storage_len, -7.5, out_np)
        elif inputs is not None:
            s = np.ascontiguousarray(inputs[i - 1], in_np).reshape(-1)
            assert s.size == v.storage_len
        else:
            s = random_values(rng, in_np, v.storage_len, op)
            if op == kd.OP["POWER"] and i == 2 and in_np != np.int64:
                with np.errstate(invalid="ignore"):  # infinite draws become NaN exponents, kept as such
                    s = np.abs(s) % 4
        storages.append(s)
    host = [s.copy() for s in storages]
    sizes = [np.dtype(out_np).itemsize] + [np.dtype(in_np).itemsize] * (len(views) - 1)
    hbases = [h.ctypes.data + v.offset * sz for h, v, sz in zip(host, views, sizes)]
    lay_h = layout_of(oracle.oracle_layout_build, views, sizes, hbases)
    rc = call_oracle(lay_h)
    assert rc == 0, support_error(oracle)
    dev = [kdb.to_device(s) for s in storages]
    dbases = [d.ptr + v.offset * sz for d, v, sz in zip(dev, views, sizes)]
    lay_d = layout_of(kdb.lib.kd_layout_build, views, sizes, dbases)
    call_kd(lay_d)
    return dev[0].numpy(), host[0]


def support_error(oracle) -> str:
    m = oracle.oracle_last_error()
    return m.decode() if m else ""


def assert_same(got, want, exact: bool, rtol=1e-5, atol=1e-6, what=""):
    if exact or got.dtype in (np.int64, np.uint8):
        if got.dtype.kind == "f":
            same = (got == want) | (np.isnan(got) & np.isnan(want))
            if not same.all():
                i = int(np.argmax(~same))
                raise AssertionError(f"{what}: not bit-exact at {i}: {got[i]!r} vs {want[i]!r} ({(~same).sum()} differ)")
        else:
            if not np.array_equal(got, want):
                i = int(np.argmax(got != want))
                raise AssertionError(f"{what}: mismatch at {i}: {got[i]!r} vs {want[i]!r}")
        return
    ok, msg = support.golden_close(got, want, rtol, atol)
    assert ok, f"{what}: {msg}"

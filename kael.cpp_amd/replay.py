"""Replays a recorded sequence of kael device calls against the C ABI (libkd.so).

A trace is one JSON object per line, as the oracle backend's call trace writes it (KD_ORACLE_TRACE,
oracle/oracle_backend.cpp): every `kael::device` call of a kael run with its arguments, device
pointers as [allocation id, byte offset], host-to-device copies with their bytes when the recording
kept them, and "mark" records at the start of each training step. Replaying it issues exactly the
backend calls that kael's host code made, in the same order, without kael itself: bench.py times a
C3 / C4 training step this way.

Before any device work the whole trace is validated on the host: every operand's byte extent, from
the record's sizes, strides and dtypes, must lie inside its live allocation. Every allocation of
the trace gets its own device buffer, zero-filled first; copies whose bytes were not recorded
upload zeros (or bytes the caller supplies). The first run of the records checks every call that
reads indices
(gather, scatter_add, cross-entropy targets) against the bytes of what it indexes, reading the
indices back, so that no replayed kernel can address memory outside its buffers; `run(checked=False)`
then replays the same records without those reads.
"""
from __future__ import annotations

import gzip
import json
from ctypes import byref, c_int64, c_void_p
from pathlib import Path

import numpy as np

import kd

ELEMENT_BYTES = {kd.F32: 4, kd.F64: 8, kd.I64: 8, kd.BOOL: 1}


class ReplayError(RuntimeError):
    pass


def load(path) -> list[dict]:
    opener = gzip.open if str(path).endswith(".gz") else open
    with opener(path, "rt") as f:
        return [json.loads(line) for line in f if line.strip()]


def split_steps(records: list[dict]) -> tuple[list[dict], list[list[dict]]]:
    """(the records before the first step mark, the records of each step)."""
    setup: list[dict] = []
    steps: list[list[dict]] = []
    for r in records:
        if r["op"] == "mark":
            if r.get("name") == "step":
                steps.append([])
            continue
        if r["op"] != "result":
            (steps[-1] if steps else setup).append(r)
    return setup, steps


def traced_losses(records: list[dict]) -> list[float]:
    """kael's loss of each traced step (the trace's "result" record), if recorded."""
    for r in records:
        if r["op"] == "result":
            return list(r["losses"])
    return []


def matmul_flops(records: list[dict]) -> int:
    return sum(2 * r["sizes"][0] * r["sizes"][1] * r["sizes"][2] * r["sizes"][3]
               for r in records if r["op"] in ("matmul", "matmul_strided", "matmul_strided_heads", "matmul_strided_bias"))


# pointer fields of each record kind (the layout bases of convert / elementwise are checked apart)
POINTERS = {
    "h2d": ("t",), "d2h": ("s",), "d2d": ("t", "s"), "fill": ("t",), "convert": (), "elementwise": (),
    "reduce": ("results", "data"), "reduce_columns": ("results", "data"), "arg_reduce": ("results", "data"),
    "cumsum": ("out", "data"),
    "matmul": ("a", "b", "c"), "matmul_strided": ("a", "b", "c"), "matmul_strided_heads": ("a", "b", "c"),
    "matmul_strided_bias": ("a", "b", "c", "bias"),
    "gather": ("out", "data", "indices"),
    "scatter_add": ("data", "indices", "source"), "index_bounds": ("indices",),
    "causal_attention": ("out", "lse", "qkv"), "causal_attention_backward": ("dqkv", "dout", "qkv", "out", "lse"),
    "softmax_rows": ("out", "x"), "standardize_rows": ("out", "x"),
    "cross_entropy_rows": ("losses", "logits", "targets"), "cross_entropy_grad": ("out", "logits", "targets", "weights"),
    "softmax_rows_backward": ("out", "y", "grad"), "standardize_rows_backward": ("out", "x", "y", "grad"),
    "adam_step": ("p", "g", "m", "v"), "sgd_step": ("p", "g"), "adam_step_many": (),
    "layer_norm_rows": ("out", "y", "x", "w", "b"), "layer_norm_rows_backward": ("gx", "gw", "gb", "x", "y", "grad", "w"),
}


ELEMENT_SIZE = {kd.F32: 4, kd.F64: 8, kd.I64: 8, kd.BOOL: 1}
COMPARE_OPS = {kd.OP[n] for n in ("EQUAL", "NOT_EQUAL", "LESS", "LESS_EQUAL", "GREATER", "GREATER_EQUAL",
                                  "LOGICAL_AND", "LOGICAL_OR", "LOGICAL_XOR", "IS_ZERO")}


def strided_span(shape, strides) -> tuple[int, int]:
    """(lowest, highest + 1) offset, in the strides' own unit, of the elements a strided view of
    `shape` addresses from its base; (0, 0) when it has none."""
    if any(n <= 0 for n in shape):
        return 0, 0
    lo = sum(min(0, (n - 1) * st) for n, st in zip(shape, strides))
    hi = sum(max(0, (n - 1) * st) for n, st in zip(shape, strides))
    return lo, hi + 1


def operand_extents(r: dict) -> dict:
    """For a kernel record: pointer field -> (lowest, one past the highest) byte offset the call
    touches from it, derived from the record's sizes, strides and dtypes. Index-addressed data
    (gather's data, scatter_add's target) is absent: its reach depends on the index values, which
    the replay reads back and checks before the launch."""
    op = r["op"]
    e = ELEMENT_SIZE.get(r.get("dtype", kd.F32), 4)

    def dense(n, es=None):
        es = e if es is None else es
        return (0, n * es) if n > 0 else (0, 0)

    def strided(shape, strides, es=None):
        es = e if es is None else es
        lo, hi = strided_span(shape, strides)
        return (lo * es, (hi - 1) * es + es) if hi > 0 else (0, 0)

    if op == "fill":
        return {"t": dense(r["count"])}
    if op in ("convert", "elementwise"):
        lay = r["layout"]
        out_es = 1 if op == "elementwise" and r["eop"] in COMPARE_OPS else ELEMENT_SIZE[r["out"]]
        ext = {}
        for o in range(lay["operands"]):
            es = out_es if o == 0 else ELEMENT_SIZE[r["in"]]
            lo, hi = strided_span(lay["shape"][:lay["dims"]], lay["strides"][o][:lay["dims"]])
            ext[f"base{o}"] = (lo, hi - 1 + es) if hi > 0 and lay["count"] > 0 else (0, 0)
        return ext
    if op == "reduce":
        out_es = 8 if r["in"] in (kd.I64, kd.BOOL) and r["rop"] == kd.REDUCE_SUM else ELEMENT_SIZE[r["in"]]
        return {"data": dense(r["chunk"] * r["rows"], ELEMENT_SIZE[r["in"]]), "results": dense(r["rows"], out_es)}
    if op == "reduce_columns":
        out_es = 8 if r["in"] in (kd.I64, kd.BOOL) and r["rop"] == kd.REDUCE_SUM else ELEMENT_SIZE[r["in"]]
        return {"data": dense(r["outer"] * r["inner"], ELEMENT_SIZE[r["in"]]), "results": dense(r["inner"], out_es)}
    if op == "arg_reduce":
        return {"data": dense(r["chunk"] * r["rows"], ELEMENT_SIZE[r["in"]]), "results": dense(r["rows"], 8)}
    if op == "cumsum":
        n = r["size"] * r["rows"]
        return {"data": dense(n, ELEMENT_SIZE[r["in"]]), "out": dense(n, 8 if r["in"] in (kd.I64, kd.BOOL) else
                                                                      ELEMENT_SIZE[r["in"]])}
    if op == "matmul":
        bt, m, k, n = r["sizes"]
        return {"a": dense(bt * m * k), "b": dense(bt * k * n), "c": dense(bt * m * n)}
    if op in ("matmul_strided", "matmul_strided_bias", "matmul_strided_heads"):
        bt, m, k, n = r["sizes"]
        if op == "matmul_strided_heads":
            heads, ha, hb, hc = r["heads"]
            outer = bt // heads if heads > 0 else 0
            a = strided([outer, heads, m, k], [r["sa"][0], ha, r["sa"][1], r["sa"][2]])
            b = strided([outer, heads, k, n], [r["sb"][0], hb, r["sb"][1], r["sb"][2]])
            c = strided([outer, heads, m, n], [r["sc"][0], hc, r["sc"][1], r["sc"][2]])
        else:
            a = strided([bt, m, k], r["sa"])
            b = strided([bt, k, n], r["sb"])
            c = strided([bt, m, n], r["sc"])
        ext = {"a": a, "b": b, "c": c}
        if op == "matmul_strided_bias" and r.get("bias") is not None:
            ext["bias"] = dense(n)
        return ext
    if op == "gather":
        lay = r["layout"]
        return {"out": dense(lay["count"]),
                "indices": strided(lay["shape"][:lay["dims"]], lay["index_strides"][:lay["dims"]], 8)}
    if op == "scatter_add":
        lay = r["layout"]
        return {"source": strided(lay["shape"][:lay["dims"]], lay["source_strides"][:lay["dims"]]),
                "indices": strided(lay["shape"][:lay["dims"]], lay["index_strides"][:lay["dims"]], 8)}
    if op == "index_bounds":
        return {"indices": strided([r["count"]], [r["stride"]], 8)}
    if op in ("causal_attention", "causal_attention_backward"):
        bt, t, h, d = r["batch"], r["length"], r["heads"], r["head_dim"]
        qkv, rows, lse = dense(bt * t * 3 * h * d), dense(bt * t * h * d), dense(bt * h * t)
        if op == "causal_attention":
            return {"out": rows, "lse": lse, "qkv": qkv}
        return {"dqkv": qkv, "dout": rows, "qkv": qkv, "out": rows, "lse": lse}
    rc = r.get("rows", 0) * r.get("cols", 0)
    if op in ("softmax_rows", "standardize_rows"):
        return {"out": dense(rc), "x": dense(rc)}
    if op == "cross_entropy_rows":
        return {"losses": dense(r["rows"]), "logits": dense(rc), "targets": dense(r["rows"], 8)}
    if op == "cross_entropy_grad":
        ext = {"out": dense(rc), "logits": dense(rc), "targets": dense(r["rows"], 8)}
        if r.get("weights") is not None:
            ext["weights"] = dense(r["rows"])
        return ext
    if op == "softmax_rows_backward":
        return {"out": dense(rc), "y": dense(rc), "grad": dense(rc)}
    if op == "standardize_rows_backward":
        return {"out": dense(rc), "x": dense(rc), "y": dense(rc), "grad": dense(rc)}
    if op == "layer_norm_rows":
        return {"out": dense(rc), "y": dense(rc), "x": dense(rc), "w": dense(r["cols"]), "b": dense(r["cols"])}
    if op == "layer_norm_rows_backward":
        ext = {"gx": dense(rc), "x": dense(rc), "y": dense(rc), "grad": dense(rc), "w": dense(r["cols"])}
        for key in ("gw", "gb"):
            if r.get(key) is not None:
                ext[key] = dense(r["cols"])
        return ext
    if op == "adam_step":
        return {key: dense(r["count"]) for key in ("p", "g", "m", "v")}
    if op == "sgd_step":
        return {key: dense(r["count"]) for key in ("p", "g")}
    return {}


def validate(records: list[dict]) -> None:
    """Checks a trace without a device: known record kinds, every device pointer inside an
    allocation that is live at that record (allocated before, not yet freed), and every byte each
    call reads or writes through it (its extent from the record's sizes, strides and dtypes; copies
    by their byte counts) inside that allocation. Index-addressed data is checked by the replay
    against the index values before its launch."""
    size: dict[int, int] = {}
    live: set[int] = set()

    def check(p, what, need=0, low=0):
        if p is None:
            return
        i, off = p
        if i not in live:
            raise ReplayError(f"{what}: allocation {i} is not live")
        if off + low < 0 or off + need > size[i]:
            raise ReplayError(f"{what}: [{off + low}, {off + need}) outside allocation {i} ({size[i]} bytes)")

    for n, r in enumerate(records):
        op = r["op"]
        if op == "alloc":
            size[r["id"]] = r["bytes"]
            live.add(r["id"])
        elif op == "free":
            live.discard(r["id"])
        elif op in ("mark", "result"):
            continue
        elif op not in POINTERS:
            raise ReplayError(f"record {n}: unknown kind {op!r}")
        else:
            ext = operand_extents(r)
            for key in POINTERS[op]:
                if r.get(key) is None and key in ("weights", "bias", "gw", "gb"):
                    continue
                low, need = (0, r["bytes"]) if op in ("h2d", "d2h", "d2d") else ext.get(key, (0, 0))
                check(r[key], f"record {n} {op}.{key}", need, low)
            if op in ("convert", "elementwise"):
                for o, p in enumerate(r["layout"]["base"]):
                    low, need = ext.get(f"base{o}", (0, 0))
                    check(p, f"record {n} {op}.base[{o}]", need, low)
            if op == "adam_step_many":
                esize = 4 if r["dtype"] == kd.F32 else 8
                for t, x in enumerate(r["tensors"]):
                    for key in ("p", "g", "m", "v"):
                        check(x[key], f"record {n} {op}.tensors[{t}].{key}", x["count"] * esize)
            if op == "h2d" and "data" in r and len(r["data"]) != 2 * r["bytes"]:
                raise ReplayError(f"record {n}: h2d payload of {len(r['data']) // 2} bytes for {r['bytes']}")


def element_layout(j: dict, resolve) -> kd.ElementLayout:
    out = kd.ElementLayout()
    out.dims, out.operands, out.count = j["dims"], j["operands"], j["count"]
    for d, v in enumerate(j["shape"]):
        out.shape[d] = v
    for o, row in enumerate(j["strides"]):
        for d, v in enumerate(row):
            out.strides[o][d] = v
    for o, p in enumerate(j["base"]):
        out.base[o] = resolve(p)
    return out


def index_layout(j: dict) -> kd.IndexLayout:
    out = kd.IndexLayout()
    out.dims, out.axis, out.count = j["dims"], j["axis"], j["count"]
    for name in ("shape", "data_strides", "index_strides", "source_strides"):
        arr = getattr(out, name)
        for d, v in enumerate(j[name]):
            arr[d] = v
    return out


def index_span(layout: dict, skip_axis: bool) -> int:
    """Largest element offset the non-indexed dims of an index layout reach in the indexed tensor."""
    return sum((n - 1) * abs(s) for d, (n, s) in enumerate(zip(layout["shape"], layout["data_strides"]))
               if not (skip_axis and d == layout["axis"]) and n > 0)


class Replay:
    """The calls of one trace bound to device buffers of their allocations."""

    def __init__(self, backend: kd.Backend, records: list[dict], uploads: dict | None = None):
        """`uploads` maps the ordinal of a host-to-device copy among the trace's copies to the bytes it
        uploads instead of the recorded ones (or zeros): it must have the copy's size and, where the
        trace recorded the bytes, equal them."""
        validate(records)  # every operand's extent inside its allocation, before any launch
        self.b = backend
        self.records = records
        self.uploads = dict(uploads or {})
        self._h2d = 0
        sizes = {r["id"]: r["bytes"] for r in records if r["op"] == "alloc"}
        self.buffers = {i: backend.empty((max(n, 1),), np.uint8) for i, n in sizes.items()}
        zero = np.zeros(1, np.uint8)
        for buf in self.buffers.values():
            backend.check(backend.lib.kd_fill(kd.BOOL, c_void_p(buf.ptr), buf.nbytes, zero.ctypes.data_as(c_void_p)),
                          "kd_fill")
        backend.synchronize()
        self.bound = [self._bind(r) for r in records]
        if self.uploads:
            raise ReplayError(f"uploads {sorted(self.uploads)} name no host-to-device copy of the trace")
        self.losses: list[float] = []  # f32 scalars the replay read back (kael's loss.item())

    # -- pointers --
    def ptr(self, p):
        if p is None:
            return None
        i, off = p
        if i not in self.buffers:
            raise ReplayError(f"pointer into allocation {i}, which the trace never made")
        if not 0 <= off <= self.buffers[i].nbytes:
            raise ReplayError(f"offset {off} outside allocation {i} ({self.buffers[i].nbytes} bytes)")
        return self.buffers[i].ptr + off

    def room(self, p) -> int:
        """Bytes from pointer p to the end of its allocation."""
        i, off = p
        return self.buffers[i].nbytes - off

    def read_i64(self, p, count: int) -> np.ndarray:
        if count * 8 > self.room(p):
            raise ReplayError("index array runs past its allocation")
        out = np.empty(count, np.int64)
        if count:
            self.b.check(self.b.lib.kd_copy_d2h(out.ctypes.data_as(c_void_p), c_void_p(self.ptr(p)), count * 8),
                         "kd_copy_d2h")
        return out

    # -- binding --
    def _bind(self, r: dict):
        """(call, check): `call()` issues the record's backend call; `check()` (or None) validates its
        index operands first."""
        lib, chk, P = self.b.lib, self.b.check, self.ptr
        op = r["op"]
        if op in ("alloc", "free", "mark", "result"):
            return None, None
        if op == "h2d":
            data = np.frombuffer(bytes.fromhex(r["data"]), np.uint8).copy() if "data" in r else np.zeros(r["bytes"], np.uint8)
            given = self.uploads.pop(self._h2d, None)
            self._h2d += 1
            if given is not None:
                given = np.ascontiguousarray(given).view(np.uint8).ravel()
                if given.size != r["bytes"]:
                    raise ReplayError(f"upload {self._h2d - 1}: {given.size} bytes given for a copy of {r['bytes']}")
                if "data" in r and not np.array_equal(given, data):
                    raise ReplayError(f"upload {self._h2d - 1}: the given bytes differ from the recorded ones")
                data = given.copy()
            t, n = c_void_p(P(r["t"])), r["bytes"]
            return (lambda: chk(lib.kd_copy_h2d(t, data.ctypes.data_as(c_void_p), n), "kd_copy_h2d")), None
        if op == "d2h":
            host = np.empty(max(r["bytes"], 1), np.uint8)
            s, n = c_void_p(P(r["s"])), r["bytes"]

            def d2h():
                chk(lib.kd_copy_d2h(host.ctypes.data_as(c_void_p), s, n), "kd_copy_d2h")
                if n == 4:
                    self.losses.append(float(host[:4].view(np.float32)[0]))
            return d2h, None
        if op == "d2d":
            t, s, n = c_void_p(P(r["t"])), c_void_p(P(r["s"])), r["bytes"]
            return (lambda: chk(lib.kd_copy_d2d(t, s, n), "kd_copy_d2d")), None
        if op == "fill":
            value = np.frombuffer(bytes.fromhex(r["value"]), np.uint8).copy()
            t = c_void_p(P(r["t"]))
            return (lambda: chk(lib.kd_fill(r["dtype"], t, r["count"], value.ctypes.data_as(c_void_p)), "kd_fill")), None
        if op == "convert":
            lay = element_layout(r["layout"], P)
            return (lambda: chk(lib.kd_convert(r["out"], r["in"], byref(lay)), "kd_convert")), None
        if op == "elementwise":
            lay = element_layout(r["layout"], P)
            par = kd.params(r["reals"], r["ints"])
            return (lambda: chk(lib.kd_elementwise(r["eop"], r["out"], r["in"], byref(lay), par), "kd_elementwise")), None
        if op == "reduce":
            a = (r["rop"], r["out"], r["in"], c_void_p(P(r["results"])), c_void_p(P(r["data"])), r["chunk"], r["rows"])
            return (lambda: chk(lib.kd_reduce(*a), "kd_reduce")), None
        if op == "reduce_columns":
            a = (r["rop"], r["out"], r["in"], c_void_p(P(r["results"])), c_void_p(P(r["data"])), r["outer"], r["inner"])
            return (lambda: chk(lib.kd_reduce_columns(*a), "kd_reduce_columns")), None
        if op in ("causal_attention", "causal_attention_backward"):
            shape = (r["batch"], r["length"], r["heads"], r["head_dim"])
            if op == "causal_attention":
                a = (r["dtype"], c_void_p(P(r["out"])), c_void_p(P(r["lse"])), c_void_p(P(r["qkv"]))) + shape
                return (lambda: chk(lib.kd_causal_attention(*a), "kd_causal_attention")), None
            a = (r["dtype"], c_void_p(P(r["dqkv"])), c_void_p(P(r["dout"])), c_void_p(P(r["qkv"])), c_void_p(P(r["out"])),
                 c_void_p(P(r["lse"]))) + shape
            return (lambda: chk(lib.kd_causal_attention_backward(*a), "kd_causal_attention_backward")), None
        if op == "index_bounds":
            pair = (c_int64 * 2)()
            a = (c_void_p(P(r["indices"])), r["count"], r["stride"], pair)
            return (lambda: chk(lib.kd_index_bounds(*a), "kd_index_bounds")), None
        if op == "arg_reduce":
            a = (r["largest"], r["in"], c_void_p(P(r["results"])), c_void_p(P(r["data"])), r["chunk"], r["rows"])
            return (lambda: chk(lib.kd_arg_reduce(*a), "kd_arg_reduce")), None
        if op == "cumsum":
            a = (r["in"], c_void_p(P(r["out"])), c_void_p(P(r["data"])), r["size"], r["rows"])
            return (lambda: chk(lib.kd_cumsum(*a), "kd_cumsum")), None
        if op in ("matmul", "matmul_strided", "matmul_strided_heads", "matmul_strided_bias"):
            sizes = kd.MatmulSizes(*r["sizes"])
            a, b, c = c_void_p(P(r["a"])), c_void_p(P(r["b"])), c_void_p(P(r["c"]))
            if op == "matmul":
                return (lambda: chk(lib.kd_matmul(r["dtype"], a, b, c, byref(sizes)), "kd_matmul")), None
            st = kd.MatmulStrides()
            for i in range(3):
                st.a[i], st.b[i], st.out[i] = r["sa"][i], r["sb"][i], r["sc"][i]
            if op == "matmul_strided_bias":
                bias = c_void_p(P(r["bias"]))
                return (lambda: chk(lib.kd_matmul_strided_bias(r["dtype"], a, b, c, byref(sizes), byref(st), bias),
                                    "kd_matmul_strided_bias")), None
            if op == "matmul_strided_heads":
                h = kd.MatmulHeads(*r["heads"])
                return (lambda: chk(lib.kd_matmul_strided_heads(r["dtype"], a, b, c, byref(sizes), byref(st), byref(h)),
                                    "kd_matmul_strided_heads")), None
            return (lambda: chk(lib.kd_matmul_strided(r["dtype"], a, b, c, byref(sizes), byref(st)),
                                "kd_matmul_strided")), None
        if op in ("gather", "scatter_add"):
            lay = index_layout(r["layout"])
            es = ELEMENT_BYTES[r["dtype"]]
            idx_count = r["layout"]["count"]
            target = r["data"]  # the tensor the indices address

            def check_indices():
                # every index of the iteration (the index tensor's own strides, as the kernel reads
                # it) must keep the addressed element inside the data allocation
                L = r["layout"]
                reach = 1 + sum((n - 1) * abs(s) for n, s in zip(L["shape"], L["index_strides"]) if n > 0)
                ids = self.read_i64(r["indices"], reach) if idx_count else np.zeros(0, np.int64)
                if ids.size == 0:
                    return
                axis_stride = abs(L["data_strides"][L["axis"]])
                last = index_span(L, skip_axis=True) + int(ids.max()) * axis_stride
                if ids.min() < 0 or (last + 1) * es > self.room(target):
                    raise ReplayError(f"{op}: indices [{ids.min()}, {ids.max()}] leave the indexed allocation")
            if op == "gather":
                a = (r["dtype"], c_void_p(P(r["out"])), c_void_p(P(r["data"])), c_void_p(P(r["indices"])), byref(lay))
                return (lambda: chk(lib.kd_gather(*a), "kd_gather")), check_indices
            a = (r["dtype"], c_void_p(P(r["data"])), c_void_p(P(r["indices"])), c_void_p(P(r["source"])), byref(lay))
            return (lambda: chk(lib.kd_scatter_add(*a), "kd_scatter_add")), check_indices
        if op == "softmax_rows":
            a = (r["dtype"], c_void_p(P(r["out"])), c_void_p(P(r["x"])), r["rows"], r["cols"], r["log"])
            return (lambda: chk(lib.kd_softmax_rows(*a), "kd_softmax_rows")), None
        if op == "standardize_rows":
            a = (r["dtype"], c_void_p(P(r["out"])), c_void_p(P(r["x"])), r["rows"], r["cols"], r["eps"], None, None)
            return (lambda: chk(lib.kd_standardize_rows(*a), "kd_standardize_rows")), None
        if op in ("cross_entropy_rows", "cross_entropy_grad"):
            def check_targets():
                t = self.read_i64(r["targets"], r["rows"])
                if t.size and (t.min() < 0 or t.max() >= r["cols"]):
                    raise ReplayError(f"{op}: targets [{t.min()}, {t.max()}] outside [0, {r['cols']})")
            if op == "cross_entropy_rows":
                a = (r["dtype"], c_void_p(P(r["losses"])), c_void_p(P(r["logits"])), c_void_p(P(r["targets"])),
                     r["rows"], r["cols"])
                return (lambda: chk(lib.kd_cross_entropy_rows(*a), "kd_cross_entropy_rows")), check_targets
            a = (r["dtype"], c_void_p(P(r["out"])), c_void_p(P(r["logits"])), c_void_p(P(r["targets"])),
                 c_void_p(P(r["weights"])), r["rows"], r["cols"])
            return (lambda: chk(lib.kd_cross_entropy_grad(*a), "kd_cross_entropy_grad")), check_targets
        if op == "softmax_rows_backward":
            a = (r["dtype"], c_void_p(P(r["out"])), c_void_p(P(r["y"])), c_void_p(P(r["grad"])), r["rows"], r["cols"],
                 r["log"])
            return (lambda: chk(lib.kd_softmax_rows_backward(*a), "kd_softmax_rows_backward")), None
        if op == "standardize_rows_backward":
            a = (r["dtype"], c_void_p(P(r["out"])), c_void_p(P(r["x"])), c_void_p(P(r["y"])), c_void_p(P(r["grad"])),
                 r["rows"], r["cols"], r["eps"])
            return (lambda: chk(lib.kd_standardize_rows_backward(*a), "kd_standardize_rows_backward")), None
        if op == "layer_norm_rows":
            a = (r["dtype"], c_void_p(P(r["out"])), c_void_p(P(r["y"])), c_void_p(P(r["x"])), r["rows"], r["cols"],
                 r["eps"], c_void_p(P(r["w"])), c_void_p(P(r["b"])))
            return (lambda: chk(lib.kd_layer_norm_rows(*a), "kd_layer_norm_rows")), None
        if op == "layer_norm_rows_backward":
            a = (r["dtype"], c_void_p(P(r["gx"])), c_void_p(P(r["gw"])), c_void_p(P(r["gb"])), c_void_p(P(r["x"])),
                 c_void_p(P(r["y"])), c_void_p(P(r["grad"])), c_void_p(P(r["w"])), r["rows"], r["cols"], r["eps"])
            return (lambda: chk(lib.kd_layer_norm_rows_backward(*a), "kd_layer_norm_rows_backward")), None
        if op == "adam_step":
            a = (r["dtype"], c_void_p(P(r["p"])), c_void_p(P(r["g"])), c_void_p(P(r["m"])), c_void_p(P(r["v"])),
                 r["count"], r["lr"], r["b1"], r["b2"], r["eps"], r["wd"], r["decoupled"], r["step"])
            return (lambda: chk(lib.kd_adam_step(*a), "kd_adam_step")), None
        if op == "adam_step_many":
            table = (kd.AdamTensor * max(1, len(r["tensors"])))()
            for t, x in enumerate(r["tensors"]):
                table[t] = kd.AdamTensor(P(x["p"]), P(x["g"]), P(x["m"]), P(x["v"]), x["count"], x["step"])
            a = (r["dtype"], table, len(r["tensors"]), r["lr"], r["b1"], r["b2"], r["eps"], r["wd"], r["decoupled"])
            return (lambda: chk(lib.kd_adam_step_many(*a), "kd_adam_step_many")), None
        if op == "sgd_step":
            a = (r["dtype"], c_void_p(P(r["p"])), c_void_p(P(r["g"])), r["count"], r["lr"], r["wd"])
            return (lambda: chk(lib.kd_sgd_step(*a), "kd_sgd_step")), None
        raise ReplayError(f"unknown trace record {op!r}")

    def run(self, records: list[dict] | None = None, checked: bool = True, on_call=None) -> None:
        """Issues the calls of `records` (a slice of the trace this replay was built from, by
        identity; all of it by default). `on_call(record, call)` may wrap each call (timing)."""
        index = {id(r): i for i, r in enumerate(self.records)}
        for r in self.records if records is None else records:
            call, check = self.bound[index[id(r)]]
            if call is None:
                continue
            if checked and check is not None:
                self.b.synchronize()
                check()
            if on_call is None:
                call()
            else:
                on_call(r, call)

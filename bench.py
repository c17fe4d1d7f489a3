"""Benchmark of the MI355X kael backend; prints ONE JSON line.

Headline (BASELINE.json metric): f32 matmul TFLOP/s as a fraction of FP32 MFMA peak, on the
north-star size 4096^3 (C = A.B, A and B contiguous row-major, uniform[-1,1]); a "step" is one
kd_matmul call over inputs already resident in HBM. Secondary figures in "extra": the C1 shape
(512^3), the C2 elementwise/reduction ops in GB/s, the fused row kernels, the index and
optimizer kernels at GPT-2-small scale, a C3 and a C4 training step (replayed from the recorded
device calls of kael's own loop, see bench_replay), and GPT-2-small decode tokens/s. Each
section carries kael's CPU path on the same workload as its cpu_baseline.

Timing: W untimed warm-up steps, then K steps bracketed by kd_synchronize(); the kernel time comes
from HIP events recorded on the backend stream (the stream every kd_* launch uses). The GPU's
clocks ramp up from idle over tens of milliseconds (the 4096^3 matmul measures ~127 TFLOP/s after
5 warm-up steps and ~140 after 50), so W defaults to 50 for the headline; the secondary sections,
whose steps take microseconds, warm up for at least MIN_WARMUP_S of steps.
The CPU baseline is kael's own CPU matmul (oracle/_ref, built from the reference sources,
threaded over the host cores) on a bounded sample, reported beside the GPU figure.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--only matmul|c1|f64|c2|rows|attention|train|c3|c4|gpt2|refdev|copy]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "kael.cpp_amd"))

import kd  # noqa: E402

FP32_MFMA_PEAK_TFLOPS = 157.3   # MI355X dense FP32 matrix (AMD spec)
FP64_MFMA_PEAK_TFLOPS = 78.6    # MI355X dense FP64 matrix (AMD spec)
HBM_PEAK_GBPS = 8000.0          # MI355X HBM3E
# HBM bytes one 4096^3 launch of the headline kernel (mfma_f32_trans_kernel<false,false>) moves,
# from rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE (198 999 KiB and 65 536 KiB per dispatch), scaled
# by the factors a plain 256 MiB copy gives the same counters (x2.0 fetch, x1.0 write). The PMC
# runs and commands are kept in profiles/.
MATMUL_4096_TRAFFIC_BYTES = (2 * 198999 + 65536) * 1024


class Timer:
    """HIP events on the backend stream around a region."""

    def __init__(self, backend: kd.Backend):
        self.b = backend
        self.start, self.stop = ctypes.c_void_p(), ctypes.c_void_p()
        backend.check(backend.lib.kd_event_create(ctypes.byref(self.start)), "event")
        backend.check(backend.lib.kd_event_create(ctypes.byref(self.stop)), "event")

    def __enter__(self):
        self.b.check(self.b.lib.kd_event_record(self.start), "record")
        return self

    def __exit__(self, *exc):
        self.b.check(self.b.lib.kd_event_record(self.stop), "record")
        ms = ctypes.c_float()
        self.b.check(self.b.lib.kd_event_elapsed_ms(ctypes.byref(ms), self.start, self.stop), "elapsed")
        self.ms = ms.value


MIN_WARMUP_S = 0.05
HEADLINE_WARMUP_S = 0.1


def time_steps(backend, step, steps, warmup, min_warmup_s=0.0):
    """W warm-up steps, then (when `min_warmup_s` is given) more steps until that much wall time
    has passed, then K timed steps. The wall-time window opens after the first W steps have
    finished, so a first launch that loads the kernel's code object does not use it up."""
    for i in range(warmup):
        step(i)
    backend.synchronize()
    if min_warmup_s > 0:
        t_start = time.perf_counter()
        done = 0
        while time.perf_counter() - t_start < min_warmup_s:
            step(done)
            done += 1
            if done % 64 == 0:
                backend.synchronize()
        backend.synchronize()
    t0 = time.perf_counter()
    with Timer(backend) as t:
        for i in range(steps):
            step(i)
    backend.synchronize()
    wall = time.perf_counter() - t0
    return t.ms / steps, wall


def bench_matmul(backend, n, steps, warmup, seed=0, min_warmup_s=0.0, dtype=kd.F32):
    rng = np.random.default_rng(seed)
    npd = kd.NUMPY_DTYPE[dtype]
    a = rng.uniform(-1, 1, (n, n)).astype(npd)
    b = rng.uniform(-1, 1, (n, n)).astype(npd)
    da, db, dc = backend.to_device(a), backend.to_device(b), backend.empty((n, n), npd)
    sizes = kd.MatmulSizes(1, n, n, n)
    fn = backend.lib.kd_matmul

    def step(_):
        rc = fn(dtype, da.ptr, db.ptr, dc.ptr, sizes)
        if rc:
            backend.check(rc, "kd_matmul")

    ms, wall = time_steps(backend, step, steps, warmup, min_warmup_s)
    flops = 2.0 * n ** 3
    return {"ms": ms, "tflops": flops / (ms * 1e-3) / 1e12, "wall_s": wall, "flops_per_launch": flops}


def bench_c2(backend, steps, warmup):
    """C2 ops with 4 rotating buffer sets (>256 MB) so the last-level cache cannot serve them."""
    rows = cols = 4096
    rng = np.random.default_rng(1)
    sets = 4
    a = [backend.to_device(rng.uniform(-1, 1, (rows, cols)).astype(np.float32)) for _ in range(sets)]
    o = [backend.empty((rows, cols), np.float32) for _ in range(sets)]
    b = backend.to_device(rng.uniform(-1, 1, (rows, 1)).astype(np.float32))
    red = [backend.empty((rows,), np.float32) for _ in range(sets)]
    out = {}
    algo_bytes = {"add": 2 * rows * cols * 4 + rows * 4, "mul": 2 * rows * cols * 4 + rows * 4,
                  "transposed_add": 2 * rows * cols * 4 + rows * 4, "sum_dim1": rows * cols * 4 + rows * 4,
                  "max_all": rows * cols * 4 + 4}
    lays = {}
    for name in ("add", "mul"):
        lays[name] = [kd.element_layout((rows, cols), [(cols * 4, 4), (cols * 4, 4), (4, 0)], [o[i].ptr, a[i].ptr, b.ptr])
                      for i in range(sets)]
    lays["transposed_add"] = [kd.element_layout((rows, cols), [(cols * 4, 4), (4, cols * 4), (4, 0)],
                                                [o[i].ptr, a[i].ptr, b.ptr]) for i in range(sets)]
    p = kd.params()
    ew = backend.lib.kd_elementwise
    rd = backend.lib.kd_reduce
    for name, op in (("add", kd.OP["PLUS"]), ("mul", kd.OP["TIMES"]), ("transposed_add", kd.OP["PLUS"])):
        ls = lays[name]
        ms, _ = time_steps(backend, lambda i: ew(op, kd.F32, kd.F32, ctypes.byref(ls[i % sets]), p), steps, warmup,
                           MIN_WARMUP_S)
        out[name] = {"us": ms * 1e3, "gbps": algo_bytes[name] / (ms * 1e-3) / 1e9}
    ms, _ = time_steps(backend, lambda i: rd(kd.REDUCE_SUM, kd.F32, kd.F32, red[i % sets].ptr, a[i % sets].ptr, cols, rows),
                       steps, warmup, MIN_WARMUP_S)
    out["sum_dim1"] = {"us": ms * 1e3, "gbps": algo_bytes["sum_dim1"] / (ms * 1e-3) / 1e9}
    ms, _ = time_steps(backend, lambda i: rd(kd.REDUCE_MAX, kd.F32, kd.F32, red[i % sets].ptr, a[i % sets].ptr,
                                             rows * cols, 1), steps, warmup, MIN_WARMUP_S)
    out["max_all"] = {"us": ms * 1e3, "gbps": algo_bytes["max_all"] / (ms * 1e-3) / 1e9}
    # Reductions kael runs on the host, on the same matrix: argmax along dim 1 and cumsum along dim 1.
    idx = [backend.empty((rows,), np.int64) for _ in range(sets)]
    ms, _ = time_steps(backend, lambda i: backend.lib.kd_arg_reduce(1, kd.F32, idx[i % sets].ptr, a[i % sets].ptr,
                                                                    cols, rows), steps, warmup, MIN_WARMUP_S)
    out["argmax_dim1"] = {"us": ms * 1e3, "gbps": (rows * cols * 4 + rows * 8) / (ms * 1e-3) / 1e9}
    ms, _ = time_steps(backend, lambda i: backend.lib.kd_cumsum(kd.F32, o[i % sets].ptr, a[i % sets].ptr, cols, rows),
                       steps, warmup, MIN_WARMUP_S)
    out["cumsum_dim1"] = {"us": ms * 1e3, "gbps": 2 * rows * cols * 4 / (ms * 1e-3) / 1e9}
    for v in out.values():
        v["frac_hbm"] = v["gbps"] / HBM_PEAK_GBPS
    return out


def bench_rows(backend, steps, warmup):
    """Fused row kernels and GELU on [32768, 1024] f32 (128 MiB in, 128 MiB out), 2 rotating sets."""
    rows, cols = 32768, 1024
    rng = np.random.default_rng(2)
    sets = 2
    x = [backend.to_device(rng.normal(size=(rows, cols)).astype(np.float32)) for _ in range(sets)]
    y = [backend.empty((rows, cols), np.float32) for _ in range(sets)]
    w = backend.to_device(np.ones(cols, np.float32))
    bb = backend.to_device(np.zeros(cols, np.float32))
    nbytes = 2 * rows * cols * 4
    out = {}
    sm = backend.lib.kd_softmax_rows
    ms, _ = time_steps(backend, lambda i: sm(kd.F32, y[i % sets].ptr, x[i % sets].ptr, rows, cols, 0), steps, warmup,
                       MIN_WARMUP_S)
    out["softmax_1024"] = {"us": ms * 1e3, "gbps": nbytes / (ms * 1e-3) / 1e9}
    st = backend.lib.kd_standardize_rows
    ms, _ = time_steps(backend, lambda i: st(kd.F32, y[i % sets].ptr, x[i % sets].ptr, rows, cols, 1e-5, w.ptr, bb.ptr),
                       steps, warmup, MIN_WARMUP_S)
    out["layernorm_1024"] = {"us": ms * 1e3, "gbps": (nbytes + 2 * cols * 4) / (ms * 1e-3) / 1e9}
    # GELU (tanh form, GPT-2's default) over the same rows: an element op on the vector path.
    gl = [kd.element_layout((rows * cols,), [(4,), (4,)], [y[i].ptr, x[i].ptr]) for i in range(sets)]
    ew, gp, gelu = backend.lib.kd_elementwise, kd.params(), kd.OP["GELU_TANH"]
    ms, _ = time_steps(backend, lambda i: ew(gelu, kd.F32, kd.F32, ctypes.byref(gl[i % sets]), gp), steps, warmup,
                       MIN_WARMUP_S)
    out["gelu_tanh_1024"] = {"us": ms * 1e3, "gbps": nbytes / (ms * 1e-3) / 1e9}
    for v in out.values():
        v["frac_hbm"] = v["gbps"] / HBM_PEAK_GBPS
    return out


def bench_attention(backend, steps, warmup):
    """kd_causal_attention (forward) and kd_causal_attention_backward on C4's attention (32 x 128
    tokens, 4 heads of 64) and a GPT-2-small-shaped one (8 x 1024 tokens, 12 heads). FLOPs are the
    products' over the unmasked (query, key) pairs, T (T + 1) / 2 per head: forward q . k^T and
    P . v (4 D each pair), backward the four products of kael's chain (8 D each pair; the kernels
    also recompute the scores and dP once more, not counted)."""
    out = {}
    for name, (b, t, h) in {"c4_32x128x4": (32, 128, 4), "gpt2_8x1024x12": (8, 1024, 12)}.items():
        rng = np.random.default_rng(b + t + h)
        qkv = backend.to_device(rng.uniform(-1, 1, (b, t, 3 * h * 64)).astype(np.float32))
        dout = backend.to_device(rng.uniform(-1, 1, (b, t, h * 64)).astype(np.float32))
        o = backend.empty((b, t, h * 64), np.float32)
        lse = backend.empty((b, h, t), np.float32)
        dq = backend.empty((b, t, 3 * h * 64), np.float32)
        fwd, bwd = backend.lib.kd_causal_attention, backend.lib.kd_causal_attention_backward
        pairs = b * h * t * (t + 1) // 2
        ms_f, _ = time_steps(backend, lambda i: fwd(kd.F32, o.ptr, lse.ptr, qkv.ptr, b, t, h, 64), steps, warmup,
                             MIN_WARMUP_S)
        ms_b, _ = time_steps(backend, lambda i: bwd(kd.F32, dq.ptr, dout.ptr, qkv.ptr, o.ptr, lse.ptr, b, t, h, 64),
                             steps, warmup, MIN_WARMUP_S)
        out[name] = {"forward_us": ms_f * 1e3, "forward_tflops": 4 * 64 * pairs / (ms_f * 1e-3) / 1e12,
                     "backward_us": ms_b * 1e3, "backward_tflops": 8 * 64 * pairs / (ms_b * 1e-3) / 1e12}
        out[name]["frac_fp32_mfma"] = (out[name]["forward_tflops"] * ms_f + out[name]["backward_tflops"] * ms_b) / \
            (ms_f + ms_b) / FP32_MFMA_PEAK_TFLOPS
    return out


def bench_train(backend, steps, warmup):
    """The index and optimizer kernels at GPT-2-small scale (HBM-bound sizes; C4's own tensors are
    latency-bound): embedding-row gather and scatter_add of 65 536 token ids against the
    [50257, 768] table, and one fused Adam / SGD step over 124 439 808 f32 parameters (GPT-2
    small). Algorithmic bytes: gather reads and writes each row once (+ 8 B per id); scatter_add
    reads the source once and reads and writes each distinct target row once (+ 8 B per id); Adam
    reads p, g, m, v and writes p, m, v (28 B per parameter); SGD reads p, g and writes p (12 B)."""
    rng = np.random.default_rng(5)
    vocab, dim, tokens = 50257, 768, 65536
    table = backend.to_device(rng.normal(0, 0.02, (vocab, dim)).astype(np.float32))
    ids_host = rng.integers(0, vocab, tokens).astype(np.int64)
    ids = backend.to_device(ids_host)
    rows = backend.empty((tokens, dim), np.float32)
    lay = kd.index_layout((tokens, dim), 0, (dim, 1), (1, 0), (dim, 1))
    out = {}
    g = backend.lib.kd_gather
    ms, _ = time_steps(backend, lambda i: g(kd.F32, rows.ptr, table.ptr, ids.ptr, ctypes.byref(lay)), steps, warmup,
                       MIN_WARMUP_S)
    out["gather_65536x768"] = {"us": ms * 1e3, "gbps": (2 * tokens * dim * 4 + tokens * 8) / (ms * 1e-3) / 1e9}
    sa = backend.lib.kd_scatter_add
    distinct = len(np.unique(ids_host))
    ms, _ = time_steps(backend, lambda i: sa(kd.F32, table.ptr, ids.ptr, rows.ptr, ctypes.byref(lay)), steps, warmup,
                       MIN_WARMUP_S)
    out["scatter_add_65536x768"] = {"us": ms * 1e3, "distinct_rows": distinct,
                                    "gbps": (tokens * dim * 4 + 2 * distinct * dim * 4 + tokens * 8) / (ms * 1e-3) / 1e9}
    del rows, table
    n = 124439808
    p = backend.to_device(rng.uniform(-0.1, 0.1, n).astype(np.float32))
    gr = backend.to_device(rng.uniform(-1e-3, 1e-3, n).astype(np.float32))
    m = backend.to_device(np.zeros(n, np.float32))
    v = backend.to_device(np.zeros(n, np.float32))
    adam = backend.lib.kd_adam_step
    ms, _ = time_steps(backend, lambda i: adam(kd.F32, p.ptr, gr.ptr, m.ptr, v.ptr, n, 3e-4, 0.9, 0.999, 1e-8, 0.01, 1,
                                               i + 1), steps, warmup, MIN_WARMUP_S)
    out["adamw_step_124M"] = {"us": ms * 1e3, "gbps": 28 * n / (ms * 1e-3) / 1e9}
    sgd = backend.lib.kd_sgd_step
    ms, _ = time_steps(backend, lambda i: sgd(kd.F32, p.ptr, gr.ptr, n, 0.01, 0.0), steps, warmup, MIN_WARMUP_S)
    out["sgd_step_124M"] = {"us": ms * 1e3, "gbps": 12 * n / (ms * 1e-3) / 1e9}
    for v_ in out.values():
        v_["frac_hbm"] = v_["gbps"] / HBM_PEAK_GBPS
    return out


def bench_copy(backend, steps, warmup, mib=256):
    """Plain contiguous f32 copy (kd_convert f32->f32) of `mib` MiB: the calibration kernel for
    HBM byte counters (it must read and write exactly `mib` MiB each)."""
    n = mib * (1 << 20) // 4
    src = backend.to_device(np.ones(n, np.float32))
    dst = backend.empty((n,), np.float32)
    lay = kd.element_layout((n,), [(4,), (4,)], [dst.ptr, src.ptr])
    fn = backend.lib.kd_convert
    ms, _ = time_steps(backend, lambda i: fn(kd.F32, kd.F32, ctypes.byref(lay)), steps, warmup, MIN_WARMUP_S)
    return {"us": ms * 1e3, "bytes_per_launch": 2 * n * 4, "gbps": 2 * n * 4 / (ms * 1e-3) / 1e9}


def synced_call_s(backend, fn, iters):
    """Median wall seconds of one call followed by kd_synchronize, the way the reference's device
    benchmarks time an iteration (benchmarks/bench_cuda.cpp:11-21); 3 untimed calls first."""
    for _ in range(3):
        fn()
        backend.synchronize()
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        backend.synchronize()
        times.append(time.perf_counter() - t0)
    return float(np.median(times))


def bench_reference_device(backend, steps, warmup):
    """The reference's own device benchmarks (benchmarks/bench_cuda.cpp:23-52) at their shapes,
    f32 uniform [0, 1) inputs, through the C ABI: BM_DeviceAdd (a + b, contiguous) and BM_DeviceSum
    (the global sum) at 2^20 and 2^24 elements, BM_DeviceMatmul at 512, 1024 and 2048. Each is timed
    two ways: `kernel_*` from HIP events over K back-to-back calls, and `synced_*` as bench_cuda.cpp
    times an iteration, one call then kd_synchronize, the median of K wall times (outputs
    preallocated, as kael's caching allocator hands them out in a steady loop). Units are the
    reference's: elements/s for add and sum, FLOP/s for matmul. Also kael's dropout of C4's
    activation size (32 x 128 x 256, p 0.1) with the mask drawn on the device (kd_dropout, which
    returns the advanced generator state, so every call is synchronous)."""
    rng = np.random.default_rng(0)
    iters = max(steps, 20)
    out = {}
    for n in (1 << 20, 1 << 24):
        a = backend.to_device(rng.random(n, dtype=np.float32))
        b = backend.to_device(rng.random(n, dtype=np.float32))
        o = backend.empty((n,), np.float32)
        lay = kd.element_layout((n,), [(4,), (4,), (4,)], [o.ptr, a.ptr, b.ptr])
        p = kd.params()
        add = lambda i=0: backend.lib.kd_elementwise(kd.OP["PLUS"], kd.F32, kd.F32, ctypes.byref(lay), p)
        ms, _ = time_steps(backend, add, iters, warmup, MIN_WARMUP_S)
        sync_s = synced_call_s(backend, add, iters)
        out[f"BM_DeviceAdd/{n}"] = {"kernel_us": ms * 1e3, "kernel_items_per_s": n / (ms * 1e-3),
                                    "kernel_gbps": 12 * n / (ms * 1e-3) / 1e9, "synced_us": sync_s * 1e6,
                                    "synced_items_per_s": n / sync_s}
        r = backend.empty((1,), np.float32)
        total = lambda i=0: backend.lib.kd_reduce(kd.REDUCE_SUM, kd.F32, kd.F32, r.ptr, a.ptr, n, 1)
        ms, _ = time_steps(backend, total, iters, warmup, MIN_WARMUP_S)
        sync_s = synced_call_s(backend, total, iters)
        out[f"BM_DeviceSum/{n}"] = {"kernel_us": ms * 1e3, "kernel_items_per_s": n / (ms * 1e-3),
                                    "kernel_gbps": 4 * n / (ms * 1e-3) / 1e9, "synced_us": sync_s * 1e6,
                                    "synced_items_per_s": n / sync_s}
    for n in (512, 1024, 2048):
        a = backend.to_device(rng.random((n, n), dtype=np.float32))
        b = backend.to_device(rng.random((n, n), dtype=np.float32))
        c = backend.empty((n, n), np.float32)
        sizes = kd.MatmulSizes(1, n, n, n)
        mm = lambda i=0: backend.lib.kd_matmul(kd.F32, a.ptr, b.ptr, c.ptr, ctypes.byref(sizes))
        ms, _ = time_steps(backend, mm, iters, warmup, MIN_WARMUP_S)
        sync_s = synced_call_s(backend, mm, iters)
        flop = 2.0 * n ** 3
        out[f"BM_DeviceMatmul/{n}"] = {"kernel_us": ms * 1e3, "kernel_gflops": flop / (ms * 1e-3) / 1e9,
                                       "synced_us": sync_s * 1e6, "synced_gflops": flop / sync_s / 1e9}
    n = 32 * 128 * 256
    x = backend.to_device(rng.normal(0, 1, n).astype(np.float32))
    y, m = backend.empty((n,), np.float32), backend.empty((n,), np.float32)
    state = np.zeros(313, np.uint64)
    backend.lib.kd_mt19937_64_seed(state.ctypes.data_as(ctypes.c_void_p), 0)
    drop = lambda i=0: backend.check(backend.lib.kd_dropout(kd.F32, y.ptr, m.ptr, x.ptr, n, 0.9,
                                                            state.ctypes.data_as(ctypes.c_void_p)), "kd_dropout")
    sync_s = synced_call_s(backend, drop, iters)
    out["dropout_c4"] = {"elements": n, "synced_us": sync_s * 1e6, "synced_items_per_s": n / sync_s,
                         "note": "one launch: mt19937_64 draws, compare, x * mask / keep, mask stored; "
                                 "the generator state copied in and back"}
    return out


def cpu_reference_device_baseline(iters=5):
    """The same benchmark bodies on kael's CPU path (reference build, threaded), median of `iters`."""
    sys.path.insert(0, str(ROOT / "tests"))
    import support

    lib = support.load_ref("ref")
    threads = int(os.environ.get("KAEL_NUM_THREADS", "0") or 0) or min(os.cpu_count() or 1, 16)
    lib.ref_set_threads(threads)
    out = {}
    for which, name, sizes in ((0, "BM_DeviceAdd", (1 << 20, 1 << 24)), (1, "BM_DeviceSum", (1 << 20, 1 << 24)),
                               (2, "BM_DeviceMatmul", (512, 1024, 2048)), (3, "dropout_c4", (32 * 128 * 256,))):
        for n in sizes:
            t = ctypes.c_double()
            if lib.ref_time_device_bench(which, n, iters, ctypes.byref(t)) != 0:
                raise RuntimeError(support.ref_error(lib))
            key = name if which == 3 else f"{name}/{n}"
            out[key] = ({"us": t.value * 1e6, "gflops": 2.0 * n ** 3 / t.value / 1e9} if which == 2
                        else {"us": t.value * 1e6, "items_per_s": n / t.value})
    return {"ops": out, "cores": threads, "kind": "reference",
            "sample": f"kael CPU path, the same benchmark bodies (kael::rand inputs), median of {iters} calls each"}


def gpt2_weights(seed=4):
    """Config C5's model: kael's GPT-2 small after manual_seed(4) (N(0, 0.02) weights, residual
    projections N(0, 0.02/sqrt(2*layers)), LayerNorm gain 1 / bias 0, Linear biases 0; reference
    src/nn/transformer.cpp:167-207), drawn on the host by kd_gpt_kael_init as kael draws it."""
    return kd.kael_gpt_parameters(kd.load(), seed)


def bench_gpt2(backend, prompt_len=64, new_tokens=256, repeats=3, eager=False):
    """C5: greedy decode with the KV cache. Prefill = the prompt's forward producing token 1;
    decode = the new_tokens - 1 single-token steps that follow. `eager` launches each step's
    kernels directly instead of replaying the captured graph (for kernel-level profiling)."""
    g = kd.Gpt(backend, eager=eager)
    weights = gpt2_weights()
    for name, a in weights:
        g.load(name, a)
    params = sum(a.size for _, a in weights)
    prompt = np.random.default_rng(4).integers(0, 50257, prompt_len)
    g.prefill(prompt)  # warm-up (graph instantiation)
    g.decode(8)
    best = None
    for _ in range(repeats):
        t0 = time.perf_counter()
        g.prefill(prompt)
        g.decode(0)
        t1 = time.perf_counter()
        g.decode(new_tokens - 1)
        t2 = time.perf_counter()
        run = {"prefill_ms": (t1 - t0) * 1e3, "decode_s": t2 - t1}
        if best is None or run["decode_s"] < best["decode_s"]:
            best = run
    steps = new_tokens - 1
    ms_tok = best["decode_s"] / steps * 1e3
    greedy_head = g.sequence()[prompt_len:prompt_len + 8].tolist()
    # The same decode with the device sampler (kael's sample_next at the reference example's
    # defaults, temperature 0.8 and top-k 40), uniforms from a seeded generator.
    # Then GenerateOptions' defaults (temperature 1, no top-k: every entry kept, the softmax and
    # multinomial sums over the whole vocabulary in index order).
    draws = np.random.default_rng(5).uniform(0, 1, new_tokens)

    def sampled_decode_s(temperature, top_k):
        g.set_sampling(temperature, top_k)
        best_s = None
        for _ in range(repeats):
            g.set_uniforms(draws)
            g.prefill(prompt)
            t1 = time.perf_counter()
            g.decode(new_tokens - 1)
            t2 = time.perf_counter()
            best_s = t2 - t1 if best_s is None else min(best_s, t2 - t1)
        return best_s

    sampled_s = sampled_decode_s(0.8, 40)
    default_s = sampled_decode_s(1.0, 0)
    g.set_sampling(0.0)
    # Per decode step: every weight except the position table is read once (the head reuses the
    # token table), plus the KV cache read by attention (mean over the decode steps).
    weight_bytes = 4 * (params - 1024 * 768)
    mean_ctx = prompt_len + steps / 2
    kv_bytes = 2 * 12 * 4 * 768 * mean_ctx
    return {"prefill_ms": best["prefill_ms"], "decode_tok_s": steps / best["decode_s"], "ms_per_token": ms_tok,
            "sampled_decode_tok_s": steps / sampled_s, "sampled_no_top_k_decode_tok_s": steps / default_s,
            "bytes_per_token": weight_bytes + kv_bytes,
            "achieved_gbps": (weight_bytes + kv_bytes) / (ms_tok * 1e-3) / 1e9,
            "frac_hbm": (weight_bytes + kv_bytes) / (ms_tok * 1e-3) / 1e9 / HBM_PEAK_GBPS,
            "config": f"GPT-2 small f32, prompt {prompt_len}, {new_tokens} new tokens, batch 1, greedy, KV cache; "
                      "wall clock around kd_gpt_decode (one HIP graph per token)",
            "sequence_head": greedy_head}


def bench_replay(backend, name, steps):
    """Configs C3 / C4: one training step of kael on this backend. bench.py does not run kael (its
    host code is built only from the reference sources, under oracle/, for the tests); instead it
    replays the step's recorded device calls (tests/golden/<name>_step_calls.jsonl.gz, written by
    tests/golden/make_step_traces.py from kael's own training loop with the optional device
    branches) against the C ABI: the same calls, shapes, strides and order as kael issues them,
    including the blocking loss read. C3 records every upload; C4 records its token ids and targets,
    and its parameters are drawn as kael draws them (kd_gpt_kael_init, seed 3). Both replays
    reproduce kael's losses.

    step_ms: HIP-event time per replayed step (K repetitions of the last traced step, Python issuing
    the calls); kernel_ms: the sum of per-call event times, one pass with events around every call;
    matmul: the step's products and their FLOPs; ms sums each product's own time (its call
    repeated back to back on the step's operands), in_step_ms the event pairs around the products
    inside the step pass (which include the GPU's wait for Python to issue each call)."""
    import replay

    recs = replay.load(ROOT / "tests" / "golden" / f"{name}_step_calls.jsonl.gz")
    setup, step_recs = replay.split_steps(recs)
    uploads = {}
    if name == "c4":
        # The trace keeps the token ids and targets (uploads 0 and 1); the 52 parameter uploads that
        # follow get config C4's model, kael's GPT after manual_seed(3) (kd_gpt_kael_init).
        params = kd.kael_gpt_parameters(backend, 3, 96, 128, 4, 4, 256)
        uploads = {2 + i: a for i, (_, a) in enumerate(params)}
    rp = replay.Replay(backend, recs, uploads)
    rp.run(setup)
    for s in step_recs:
        rp.run(s)  # the traced steps, with their index operands checked
    backend.synchronize()
    # kael's loss of each traced step is the last f32 scalar the step reads back
    per_step = len(rp.losses) // len(step_recs)
    losses = [rp.losses[(i + 1) * per_step - 1] for i in range(len(step_recs))]
    kael_losses = replay.traced_losses(recs)
    if kael_losses and not np.allclose(losses, kael_losses, rtol=1e-4):
        raise RuntimeError(f"{name} replay losses {losses} differ from kael's {kael_losses}")
    last = step_recs[-1]
    for _ in range(3):
        rp.run(last, checked=False)
    backend.synchronize()
    t0 = time.perf_counter()
    with Timer(backend) as t:
        for _ in range(steps):
            rp.run(last, checked=False)
    backend.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    step_ms = t.ms / steps
    # one pass with an event pair around every call
    lib = backend.lib
    pairs = []

    def timed(r, call):
        e0, e1 = ctypes.c_void_p(), ctypes.c_void_p()
        backend.check(lib.kd_event_create(ctypes.byref(e0)), "event")
        backend.check(lib.kd_event_create(ctypes.byref(e1)), "event")
        backend.check(lib.kd_event_record(e0), "record")
        call()
        backend.check(lib.kd_event_record(e1), "record")
        pairs.append((r, e0, e1))

    rp.run(last, checked=False, on_call=timed)
    backend.synchronize()
    per_call = []
    for r, e0, e1 in pairs:
        ms = ctypes.c_float()
        backend.check(lib.kd_event_elapsed_ms(ctypes.byref(ms), e0, e1), "elapsed")
        per_call.append((r, ms.value))
        lib.kd_event_destroy(e0)
        lib.kd_event_destroy(e1)
    products = ("matmul", "matmul_strided", "matmul_strided_heads", "matmul_strided_bias")
    mm = [(r, ms) for r, ms in per_call if r["op"] in products]
    in_step_ms = sum(ms for _, ms in mm)
    # The pair around a call in the step also spans the time the GPU waits for Python to issue
    # that call (the step blocks at its index checks and loss read, so the host never runs far
    # ahead). Each product is therefore also timed alone: its own call, on the step's operands,
    # `repeat` times back to back between one event pair, after one untimed call.
    bound = []
    rp.run(last, checked=False, on_call=lambda r, call: (call(), bound.append((r, call))))
    repeat = 10
    mm_ms = 0.0
    for r, call in bound:
        if r["op"] not in products:
            continue
        call()
        with Timer(backend) as t:
            for _ in range(repeat):
                call()
        mm_ms += t.ms / repeat
    backend.synchronize()
    # row kernels: algorithmic bytes = the row arrays each one reads and writes once
    arrays = {"softmax_rows": 2, "standardize_rows": 2, "softmax_rows_backward": 3, "standardize_rows_backward": 4,
              "cross_entropy_rows": 1, "cross_entropy_grad": 2, "layer_norm_rows": 3, "layer_norm_rows_backward": 4}
    rows = [(r, ms) for r, ms in per_call if r["op"] in arrays]
    row_bytes = sum(arrays[r["op"]] * r["rows"] * r["cols"] * (4 if r["dtype"] == 0 else 8) for r, _ in rows)
    row_ms = sum(ms for _, ms in rows)
    flops = replay.matmul_flops(last)
    counts = {}
    for r in last:
        counts[r["op"]] = counts.get(r["op"], 0) + 1
    return {"step_ms": step_ms, "wall_ms": wall_ms, "kernel_ms": sum(ms for _, ms in per_call),
            "calls_per_step": len(last), "calls": counts,
            "matmul": {"count": len(mm), "ms": mm_ms, "in_step_ms": in_step_ms, "gflop": flops / 1e9,
                       "tflops": flops / (mm_ms * 1e-3) / 1e12 if mm_ms else None,
                       "frac_peak": flops / (mm_ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS if mm_ms else None},
            "row_kernels": {"count": len(rows), "ms": row_ms, "gbytes": row_bytes / 1e9,
                            "tb_s": row_bytes / (row_ms * 1e-3) / 1e12 if row_ms else None},
            "replay_losses": losses, "kael_losses": kael_losses,
            "data": "C3: kael's recorded inputs and initial parameters; C4: recorded token ids and targets, "
                    "kael's seed-3 parameters (kd_gpt_kael_init)"}


def cpu_train_baseline(name):
    """kael's own training step on the CPU path (reference build, threaded), same config and loop
    as the traced one: C3 100 SGD steps, C4 3 Adam steps (each ~0.7 s); seconds per step."""
    sys.path.insert(0, str(ROOT / "tests"))
    import support

    lib = support.load_ref("ref")
    threads = int(os.environ.get("KAEL_NUM_THREADS", "0") or 0) or min(os.cpu_count() or 1, 16)
    lib.ref_set_threads(threads)
    secs = ctypes.c_double()
    if name == "c3":
        steps = 100
        losses = np.zeros(steps, np.float32)
        rc = lib.ref_train_mlp(0, steps, losses.ctypes.data_as(ctypes.c_void_p), None, ctypes.byref(secs))
    else:
        steps = 3
        losses = np.zeros(steps, np.float32)
        rc = lib.ref_train_chargpt(0, steps, losses.ctypes.data_as(ctypes.c_void_p), ctypes.byref(secs))
    if rc != 0:
        raise RuntimeError(support.ref_error(lib))
    return {"value": secs.value / steps * 1e3, "unit": "ms/step", "cores": threads, "kind": "reference",
            "sample": f"kael {'ref_train_mlp' if name == 'c3' else 'ref_train_chargpt'} on the CPU path, {steps} steps "
                      f"(forward, cross-entropy, backward, {'SGD' if name == 'c3' else 'Adam'}, loss read)"}


def cpu_c2_baseline(iters=5):
    """kael's C2 ops on the CPU path (reference build, threaded): median of `iters` calls each."""
    sys.path.insert(0, str(ROOT / "tests"))
    import support

    lib = support.load_ref("ref")
    threads = int(os.environ.get("KAEL_NUM_THREADS", "0") or 0) or min(os.cpu_count() or 1, 16)
    lib.ref_set_threads(threads)
    rows = cols = 4096
    algo_bytes = {"add": 2 * rows * cols * 4 + rows * 4, "mul": 2 * rows * cols * 4 + rows * 4,
                  "transposed_add": 2 * rows * cols * 4 + rows * 4, "sum_dim1": rows * cols * 4 + rows * 4,
                  "max_all": rows * cols * 4 + 4}
    out = {}
    for which, op in enumerate(("add", "mul", "transposed_add", "sum_dim1", "max_all")):
        t = ctypes.c_double()
        if lib.ref_time_c2(which, rows, cols, iters, ctypes.byref(t)) != 0:
            raise RuntimeError(support.ref_error(lib))
        out[op] = {"us": t.value * 1e6, "gbps": algo_bytes[op] / t.value / 1e9}
    return {"ops": out, "unit": "GB/s", "cores": threads, "kind": "reference",
            "sample": f"kael CPU path, [4096,4096] f32 (manual_seed(1) inputs), median of {iters} calls per op"}


def cpu_gpt2_baseline(new_tokens=8, context=192):
    """kael's own nn::generate on the CPU path (reference build), GPT-2 small, seed 4: decode
    tokens/s from two runs (1 and 1 + new_tokens new tokens) so prefill cancels out. The prompt
    is `context` tokens long so that the sampled steps attend over the mean context of the GPU
    run (a 64-token prompt and 255 new tokens: positions 65-319, mean ~192)."""
    sys.path.insert(0, str(ROOT / "tests"))
    import support

    lib = support.load_ref("ref")
    threads = int(os.environ.get("KAEL_NUM_THREADS", "0") or 0) or min(os.cpu_count() or 1, 16)
    lib.ref_set_threads(threads)
    h = lib.ref_gpt_create(50257, 1024, 12, 12, 768, 4, 1)
    prompt = np.ascontiguousarray(np.random.default_rng(4).integers(0, 50257, context), np.int64)
    out = np.zeros(context + 1 + new_tokens, np.int64)
    t1, t2 = ctypes.c_double(), ctypes.c_double()
    try:
        if lib.ref_gpt_generate(h, prompt.ctypes.data_as(ctypes.c_void_p), context, 1, out.ctypes.data_as(ctypes.c_void_p),
                                ctypes.byref(t1)):
            raise RuntimeError(support.ref_error(lib))
        if lib.ref_gpt_generate(h, prompt.ctypes.data_as(ctypes.c_void_p), context, 1 + new_tokens,
                                out.ctypes.data_as(ctypes.c_void_p), ctypes.byref(t2)):
            raise RuntimeError(support.ref_error(lib))
    finally:
        lib.ref_gpt_destroy(h)
    rate = new_tokens / max(t2.value - t1.value, 1e-9)
    return {"value": rate, "unit": "tokens/s", "cores": threads, "kind": "reference",
            "sample": f"kael nn::generate GPT-2 small f32 (seed 4), prompt {context} (the GPU run's mean context), "
                      f"decode rate from {new_tokens} extra tokens, prefill {t1.value:.2f} s", "prefill_s": t1.value}


def cpu_baseline(n, budget_s=20.0):
    """kael's CPU matmul (reference build, threaded) on a bounded sample of the same workload."""
    sys.path.insert(0, str(ROOT / "tests"))
    import support

    lib = support.load_ref("ref")
    threads = int(os.environ.get("KAEL_NUM_THREADS", "0") or 0) or min(os.cpu_count() or 1, 16)
    lib.ref_set_threads(threads)
    t = ctypes.c_double()
    # one probe call sizes the sample to about `budget_s` seconds
    if lib.ref_time_matmul(n, n, n, 1, ctypes.byref(t)) != 0:
        raise RuntimeError(support.ref_error(lib))
    iters = max(1, min(10, int(budget_s / max(t.value, 1e-3)) - 1))
    if lib.ref_time_matmul(n, n, n, iters, ctypes.byref(t)) != 0:
        raise RuntimeError(support.ref_error(lib))
    tflops = 2.0 * n ** 3 / t.value / 1e12
    return {"value": tflops, "unit": "TFLOP/s", "cores": threads, "kind": "reference",
            "sample": f"kael::matmul f32 {n}^3 (CPU path, matmul_versions v6), median of {iters} calls after 2 warm-up calls, "
                      f"KAEL_NUM_THREADS={threads}", "median_s": t.value}


def guarded_cpu(fn, *args):
    """A CPU-baseline leg: its result, or the error it raised (a baseline is reported, never required)."""
    try:
        return fn(*args)
    except Exception as e:
        return {"error": str(e)}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--gpt-eager", action="store_true", help="GPT-2 steps without graph replay (profiling)")
    ap.add_argument("--gpt-tokens", type=int, default=256, help="GPT-2 new tokens per run (shorter profiling runs)")
    ap.add_argument("--gpt-repeats", type=int, default=3, help="GPT-2 timed runs (the best is reported)")
    ap.add_argument("--only", default="", choices=["", "all", "matmul", "c1", "f64", "copy", "c2", "rows", "attention",
                                                  "train", "c3", "c4", "gpt2", "refdev"],
                    help="run one group only (profiling runs); the JSON line is printed either way")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this backend drives one GPU; multi-GPU runs are out of scope (bench.py --gpus 1)"}))
        return 2
    backend = kd.load()
    if not backend.lib.kd_available():
        raise SystemExit(f"no usable gfx950 device: {backend.error()}")
    info = backend.device_info()
    n = 4096
    extra = {"device": info}
    if args.only == "copy":
        extra["copy"] = bench_copy(backend, args.steps, args.warmup)
        print(json.dumps({"metric": "copy calibration", "extra": extra}))
        return 0
    if args.only == "gpt2":
        extra["gpt2_decode"] = bench_gpt2(backend, new_tokens=args.gpt_tokens, repeats=args.gpt_repeats,
                                          eager=args.gpt_eager)
        print(json.dumps({"metric": "GPT-2-small decode tok/s", "extra": extra}))
        return 0
    if args.only == "f64":
        f64 = bench_matmul(backend, n, max(args.steps, 10), args.warmup, min_warmup_s=MIN_WARMUP_S, dtype=kd.F64)
        f64["frac_of_fp64_matrix_peak"] = f64["tflops"] / FP64_MFMA_PEAK_TFLOPS
        extra[f"matmul_f64_{n}"] = f64
        print(json.dumps({"metric": "f64 matmul 4096^3", "extra": extra}))
        return 0
    if args.only == "c1":
        extra["matmul_512"] = bench_matmul(backend, 512, max(args.steps, 50), args.warmup, min_warmup_s=MIN_WARMUP_S)
        if not args.no_cpu:
            extra["matmul_512"]["cpu_baseline"] = guarded_cpu(cpu_baseline, 512, 5.0)
        print(json.dumps({"metric": "C1 f32 matmul 512^3", "extra": extra}))
        return 0
    if args.only in ("c3", "c4"):
        extra[args.only] = bench_replay(backend, args.only, max(args.steps, 10))
        if not args.no_cpu:
            extra[args.only]["cpu_baseline"] = guarded_cpu(cpu_train_baseline, args.only)
        print(json.dumps({"metric": f"{args.only} training step (replayed kael device calls)", "extra": extra}))
        return 0
    if args.only == "refdev":
        extra["reference_device"] = bench_reference_device(backend, args.steps, args.warmup)
        if not args.no_cpu:
            extra["reference_device"]["cpu_baseline"] = guarded_cpu(cpu_reference_device_baseline)
        print(json.dumps({"metric": "reference device benchmarks", "extra": extra}))
        return 0
    if args.only == "attention":
        extra["attention"] = bench_attention(backend, max(args.steps, 20), args.warmup)
    if args.only in ("c2", "rows", "train"):
        fn = {"c2": bench_c2, "rows": bench_rows, "train": bench_train}[args.only]
        extra[args.only] = fn(backend, args.steps, args.warmup)
        if args.only == "c2" and not args.no_cpu:
            extra["c2"]["cpu_baseline"] = guarded_cpu(cpu_c2_baseline)
        print(json.dumps({"metric": f"{args.only} only", "extra": extra}))
        return 0
    # The headline warms up like every other section: W steps, then steps for at least
    # HEADLINE_WARMUP_S of wall time (~100 launches), so that a small W (the driver passes
    # --warmup 5) still times steady clocks.
    main_run = bench_matmul(backend, n, args.steps, args.warmup, min_warmup_s=HEADLINE_WARMUP_S)
    if args.only in ("", "all"):
        extra["matmul_512"] = bench_matmul(backend, 512, max(args.steps, 50), args.warmup, min_warmup_s=MIN_WARMUP_S)
        f64 = bench_matmul(backend, n, max(args.steps, 10), args.warmup, min_warmup_s=MIN_WARMUP_S, dtype=kd.F64)
        f64["frac_of_fp64_matrix_peak"] = f64["tflops"] / FP64_MFMA_PEAK_TFLOPS
        extra[f"matmul_f64_{n}"] = f64
        extra["c2"] = bench_c2(backend, max(args.steps, 50), args.warmup)
        extra["rows"] = bench_rows(backend, max(args.steps, 20), args.warmup)
        extra["attention"] = bench_attention(backend, max(args.steps, 20), args.warmup)
        extra["train"] = bench_train(backend, max(args.steps, 20), args.warmup)
        extra["c3"] = bench_replay(backend, "c3", max(args.steps, 20))
        extra["c4"] = bench_replay(backend, "c4", max(args.steps, 10))
        extra["gpt2_decode"] = bench_gpt2(backend)
        extra["reference_device"] = bench_reference_device(backend, args.steps, args.warmup)
    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(n)
        except Exception as e:  # the baseline is reported, never required
            cpu = {"error": str(e)}
        if "matmul_512" in extra:
            extra["matmul_512"]["cpu_baseline"] = guarded_cpu(cpu_baseline, 512, 5.0)
        if "c2" in extra:
            extra["c2"]["cpu_baseline"] = guarded_cpu(cpu_c2_baseline)
        for name in ("c3", "c4"):
            if name in extra:
                extra[name]["cpu_baseline"] = guarded_cpu(cpu_train_baseline, name)
        if "reference_device" in extra:
            extra["reference_device"]["cpu_baseline"] = guarded_cpu(cpu_reference_device_baseline)
        if "gpt2_decode" in extra:
            try:
                gcpu = cpu_gpt2_baseline()
                extra["gpt2_decode"]["cpu_baseline"] = gcpu
                extra["gpt2_decode"]["speedup_vs_cpu"] = extra["gpt2_decode"]["decode_tok_s"] / gcpu["value"]
            except Exception as e:
                extra["gpt2_decode"]["cpu_baseline"] = {"error": str(e)}
    achieved = main_run["tflops"]
    line = {
        "metric": "f32 matmul TFLOP/s (% FP32 MFMA peak)",
        "value": round(achieved, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_run["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic uniform[-1,1] (numpy seed 0), resident in HBM",
        "config": {"workload": "f32 matmul C=A.B, M=N=K=4096, contiguous row-major (BASELINE C1 recipe at the north-star size)",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / FP32_MFMA_PEAK_TFLOPS, 4),
                     "traffic": MATMUL_4096_TRAFFIC_BYTES if n == 4096 else None},
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

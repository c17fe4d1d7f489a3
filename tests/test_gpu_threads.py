"""Backend calls from several host threads at once.

kael may call its device backend from more than one host thread (reference
docs/08-cpu-performance.md:191: the Python/server thread beside the main thread), and the
reference backend takes no lock (src/cuda/backend.cu). This backend shares one scratch buffer
per device between the split reductions, the split cumsum and the split-K products, growing it
on demand; these tests drive those paths from four threads at once, with workspace sizes that
grow while the threads run, and require every result to equal, bit for bit, the same call made
alone afterwards (each of these kernels reduces in a fixed order). The fourth thread also takes
the index range checks' pinned host slots (one per call in flight) and the attention backward's
workspace; two more threads run kd_reduce_noalloc at once, whose split path shares one static
buffer per device.

The check runs in a child process so that the workspace starts empty and its growths happen
during the concurrent phase, whatever earlier tests allocated.
"""
import ctypes
import os
import subprocess
import sys
import threading
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent
sys.path.insert(0, str(ROOT / "kael.cpp_amd"))

import kd  # noqa: E402

ROUNDS = 6


def _reduce_jobs(backend, rng):
    """Few long rows: kd_reduce takes the split + combine path, kd_cumsum the segmented scan."""
    jobs = []
    for rows, chunk in ((3, 1 << 20), (2, 3 << 19), (1, 1 << 22)):
        x = backend.to_device(rng.uniform(-1, 1, (rows, chunk)).astype(np.float32))
        for op in (kd.REDUCE_SUM, kd.REDUCE_MAX):
            def run(x=x, rows=rows, chunk=chunk, op=op):
                out = backend.empty((rows,), np.float32)
                backend.call("reduce", op, kd.F32, kd.F32, out.ptr, x.ptr, chunk, rows)
                return out.numpy()
            jobs.append((f"reduce op {op} {rows}x{chunk}", run))

        def scan(x=x, rows=rows, chunk=chunk):
            out = backend.empty((rows, chunk), np.float32)
            backend.call("cumsum", kd.F32, out.ptr, x.ptr, chunk, rows)
            return out.numpy()
        jobs.append((f"cumsum {rows}x{chunk}", scan))
    return jobs


def _matmul_jobs(backend, rng):
    """Row-major products with too few tiles for the device (split K into the workspace), in
    increasing workspace size: 1, 4 and 16 MiB of partials."""
    jobs = []
    for m, k, n in ((128, 1024, 128), (128, 4096, 128), (128, 16384, 128), (256, 16384, 256)):
        a = backend.to_device(rng.uniform(-1, 1, (m, k)).astype(np.float32))
        b = backend.to_device(rng.uniform(-1, 1, (k, n)).astype(np.float32))

        def run(a=a, b=b, m=m, k=k, n=n):
            out = backend.empty((m, n), np.float32)
            backend.call("matmul", kd.F32, a.ptr, b.ptr, out.ptr, kd.MatmulSizes(1, m, k, n))
            return out.numpy()
        jobs.append((f"matmul {m}x{k}x{n}", run))
    return jobs


def _skinny_jobs(backend, rng):
    """Decode-shaped products (M <= 16) whose K is split across workgroups into the workspace."""
    jobs = []
    for m, k, n in ((1, 3072, 768), (4, 65536, 256), (16, 8192, 512)):
        a = backend.to_device(rng.uniform(-1, 1, (m, k)).astype(np.float32))
        b = backend.to_device(rng.uniform(-1, 1, (k, n)).astype(np.float32))

        def run(a=a, b=b, m=m, k=k, n=n):
            out = backend.empty((m, n), np.float32)
            backend.call("matmul", kd.F32, a.ptr, b.ptr, out.ptr, kd.MatmulSizes(1, m, k, n))
            return out.numpy()
        jobs.append((f"skinny {m}x{k}x{n}", run))
    return jobs


def _bounds_and_attention_jobs(backend, rng):
    """Index range checks (each holds a pinned host slot from its launch to its read; the larger
    ones also a workspace for the workgroups' pairs) and the attention backward (its delta rows in
    the workspace)."""
    jobs = []
    for count in (4096, 1 << 20, 3_000_001):
        ids = backend.to_device(rng.integers(-(1 << 40), 1 << 40, count).astype(np.int64))

        def bounds(ids=ids, count=count):
            pair = np.zeros(2, np.int64)
            backend.call("index_bounds", ids.ptr, count, 1, pair.ctypes.data_as(ctypes.c_void_p))
            return pair
        jobs.append((f"index_bounds {count}", bounds))
    b, t, h = 4, 128, 4
    qkv = backend.to_device(rng.uniform(-1, 1, (b, t, 3 * h * 64)).astype(np.float32))
    dout = backend.to_device(rng.uniform(-1, 1, (b, t, h * 64)).astype(np.float32))

    def attention():
        out, lse = backend.empty((b, t, h * 64), np.float32), backend.empty((b, h, t), np.float32)
        dq = backend.empty((b, t, 3 * h * 64), np.float32)
        backend.call("causal_attention", kd.F32, out.ptr, lse.ptr, qkv.ptr, b, t, h, 64)
        backend.call("causal_attention_backward", kd.F32, dq.ptr, dout.ptr, qkv.ptr, out.ptr, lse.ptr, b, t, h, 64)
        return dq.numpy()
    jobs.append(("causal_attention 4x128x4", attention))
    return jobs


def _noalloc_jobs(backend, rng, shapes):
    """kd_reduce_noalloc on its split path (few long rows): the segment partials in the one static
    buffer per device that every call shares; two threads run these at once."""
    jobs = []
    for rows, chunk in shapes:
        x = backend.to_device(rng.uniform(-1, 1, (rows, chunk)).astype(np.float32))

        def run(x=x, rows=rows, chunk=chunk):
            out = backend.empty((rows,), np.float32)
            backend.call("reduce_noalloc", kd.REDUCE_SUM, kd.F32, kd.F32, out.ptr, x.ptr, chunk, rows)
            return out.numpy()
        jobs.append((f"reduce_noalloc {rows}x{chunk}", run))
    return jobs


def child() -> int:
    backend = kd.load()
    if not backend.lib.kd_available():
        print(f"no device: {backend.error()}", flush=True)
        return 2
    rng = np.random.default_rng(11)
    groups = [_reduce_jobs(backend, rng), _matmul_jobs(backend, rng), _skinny_jobs(backend, rng),
              _bounds_and_attention_jobs(backend, rng), _noalloc_jobs(backend, rng, ((3, 1 << 20), (1, 1 << 22))),
              _noalloc_jobs(backend, rng, ((2, 3 << 19), (4, 1 << 19)))]
    results = [[] for _ in groups]
    errors = []

    def worker(g):
        try:
            for _ in range(ROUNDS):
                for name, job in groups[g]:
                    results[g].append((name, job()))
        except Exception as e:  # reported by the parent thread
            errors.append(f"thread {g}: {e!r}")

    threads = [threading.Thread(target=worker, args=(g,)) for g in range(len(groups))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    if errors:
        print("\n".join(errors), flush=True)
        return 1
    # The same calls, one at a time.
    bad = 0
    for g, jobs in enumerate(groups):
        alone = {name: job() for name, job in jobs}
        for name, got in results[g]:
            if not np.array_equal(got, alone[name]):
                bad += 1
                print(f"{name}: concurrent result differs from the serial one "
                      f"(max |diff| {np.max(np.abs(got - alone[name]))})", flush=True)
    print(f"{sum(len(r) for r in results)} concurrent calls checked, {bad} differ", flush=True)
    return 1 if bad else 0


@pytest.mark.gpu
def test_concurrent_calls_share_the_workspace_safely():
    env = dict(os.environ)
    proc = subprocess.run([sys.executable, "-u", str(Path(__file__).resolve()), "--child"], env=env,
                          capture_output=True, text=True, timeout=110)
    print(proc.stdout, proc.stderr)
    assert proc.returncode == 0, proc.stdout + proc.stderr


if __name__ == "__main__" and "--child" in sys.argv:
    sys.exit(child())

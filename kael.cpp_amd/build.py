"""Builds the gfx950 backend library kael.cpp_amd/lib/libkd.so (and, on request, the test
oracles under oracle/).

Every HIP translation unit under csrc/ is compiled separately for --offload-arch=gfx950 and the
host-only sources under host/ are compiled as C++20; all objects are linked into one shared
library whose exported C symbols are declared in include/kd_api.h.

Usage: python kael.cpp_amd/build.py [--oracle] [--jobs N]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
BUILD = PKG / "_build"
LIB = PKG / "lib"
INCLUDE = ROOT / "include"
ORACLE = ROOT / "oracle"
REFERENCE = Path("/root/reference")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (packed FP32 has misbehaved on this pool).
HIP_FLAGS = [
    "-O3", "-std=c++20", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-I", str(INCLUDE), "-I", str(CSRC),
]
HOST_FLAGS = ["-O2", "-std=c++20", "-fPIC", "-Wall", "-I", str(INCLUDE)]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + proc.stdout + proc.stderr)
        raise RuntimeError(f"command failed ({proc.returncode}): {cmd[0]} ... {cmd[-1]}")


def build_library(jobs: int = 8) -> Path:
    """Compiles csrc/*.hip and host/*.cpp and links lib/libkd.so. Always recompiles."""
    BUILD.mkdir(exist_ok=True)
    LIB.mkdir(exist_ok=True)
    jobs_list = []
    objects = []
    for src in sorted(CSRC.glob("*.hip")):
        obj = BUILD / (src.stem + ".o")
        jobs_list.append([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(obj)])
        objects.append(obj)
    for src in sorted(HOST.glob("kd_*.cpp")):
        obj = BUILD / (src.stem + ".o")
        jobs_list.append([HIPCC, *HOST_FLAGS, "-c", str(src), "-o", str(obj)])
        objects.append(obj)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        for fut in [pool.submit(_run, cmd) for cmd in jobs_list]:
            fut.result()
    out = LIB / "libkd.so"
    tmp = LIB / "libkd.so.tmp"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objects)])
    os.replace(tmp, out)
    return out


def build_oracle(jobs: int = 8) -> None:
    """Builds oracle/build/liboracle.so and, when the reference sources are present,
    oracle/_ref/libkael_ref-v{3,4}.so (test infrastructure only)."""
    make = shutil.which("make") or "make"
    _run([make, "-C", str(ORACLE), "-B", "build/liboracle.so"])
    if REFERENCE.is_dir():
        _run([make, "-C", str(ORACLE), f"-j{jobs}", "ref"])


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--oracle", action="store_true", help="also build the test oracles")
    ap.add_argument("--jobs", type=int, default=8)
    args = ap.parse_args()
    lib = build_library(args.jobs)
    print(f"built {lib}")
    if args.oracle:
        build_oracle(args.jobs)
        print("built oracle")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

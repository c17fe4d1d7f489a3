"""Writes the device-call traces of two training steps of configs C3 and C4 (test fixtures that
bench.py replays against the C ABI on the GPU).

Each trace is kael's own training loop (oracle/ref_shim.cpp: ref_train_mlp for C3,
ref_train_chargpt for C4) built with the optional device branches and the C oracle as its device
(oracle/_ref/libkael_oracle_fused.so), run on the CPU with KD_ORACLE_TRACE set: one JSON object
per device call, gzip-compressed, device pointers as [allocation id, byte offset], and a last
"result" record with kael's loss of each traced step. The calls
before the first "step" mark build the model and upload the data; each mark starts a step (zero
grad, forward, cross-entropy, backward, optimizer step, the loss read back).

    python tests/golden/make_step_traces.py [c3] [c4]   # writes c3_step_calls.jsonl.gz, c4_...

Needs the oracle builds (make -C oracle ref); C4's two steps on the C oracle take about 7 minutes.
"""
from __future__ import annotations

import ctypes
import gzip
import json
import os
import subprocess
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
CONFIGS = {"c3": "ref_train_mlp", "c4": "ref_train_chargpt"}
# Host-to-device bytes kept per copy: all of C3's (its inputs and parameters, 0.6 MB, so that a
# replay reproduces kael's losses); C4's token ids and targets only (its 13 MB of parameters upload
# as zeros in a replay).
PAYLOAD = {"c3": 1 << 20, "c4": 64 * 1024}
STEPS = 2


def run_one(name: str, raw: Path) -> None:
    """Runs config `name` for STEPS steps with the trace written to `raw` (in this process)."""
    os.environ["KD_ORACLE_TRACE"] = str(raw)
    os.environ["KD_ORACLE_TRACE_PAYLOAD"] = str(PAYLOAD[name])
    lib = ctypes.CDLL(str(ROOT / "oracle" / "_ref" / "libkael_oracle_fused.so"))
    losses = (ctypes.c_float * STEPS)()
    seconds = ctypes.c_double()
    if name == "c3":
        rc = lib.ref_train_mlp(1, ctypes.c_int64(STEPS), losses, None, ctypes.byref(seconds))
    else:
        rc = lib.ref_train_chargpt(1, ctypes.c_int64(STEPS), losses, ctypes.byref(seconds))
    if rc != 0:
        lib.ref_last_error.restype = ctypes.c_char_p
        raise SystemExit(f"{name}: {lib.ref_last_error().decode()}")
    print(f"{name}: losses {list(losses)}, {seconds.value:.1f} s", flush=True)
    Path(str(raw) + ".result").write_text(json.dumps({"op": "result", "losses": list(losses)}) + "\n")


def main() -> int:
    if len(sys.argv) == 3 and sys.argv[1] in CONFIGS:  # child: one config per process (the trace opens once)
        run_one(sys.argv[1], Path(sys.argv[2]))
        return 0
    for name in sys.argv[1:] or CONFIGS:
        with tempfile.TemporaryDirectory() as tmp:
            raw = Path(tmp) / "trace.jsonl"
            subprocess.run([sys.executable, __file__, name, str(raw)], check=True)
            # the trace, then a "result" record with kael's losses of the traced steps
            lines = raw.read_bytes() + Path(str(raw) + ".result").read_bytes()
            out = HERE / f"{name}_step_calls.jsonl.gz"
            with gzip.GzipFile(out, "wb", mtime=0) as f:
                f.write(lines)
            records = lines.count(b"\n")
            print(f"{out.name}: {records} records, {out.stat().st_size} bytes", flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

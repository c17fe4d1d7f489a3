"""Shared test helpers: library loading, golden-case runner and comparison rules.

Loads (never builds) the backend library and the test oracles:
  kael.cpp_amd/lib/libkd.so         the MI355X backend (the thing under test)
  oracle/build/liboracle.so         C restatement of the reference device semantics (checker)
  oracle/_ref/libkael_*.so          the reference kael core with one of three device backends
"""
from __future__ import annotations

import ctypes
import os
import sys
from ctypes import POINTER, c_char_p, c_double, c_int, c_int64, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "kael.cpp_amd"))

import kd  # noqa: E402  (the package directory name is not an identifier)

GOLDEN = ROOT / "tests" / "golden"
ORACLE_LIB = ROOT / "oracle" / "build" / "liboracle.so"
REF_DIR = ROOT / "oracle" / "_ref"


def cpu_has_avx512() -> bool:
    try:
        flags = Path("/proc/cpuinfo").read_text()
    except OSError:
        return False
    return " avx512f" in flags and " avx512bw" in flags and " avx512vl" in flags


def ref_path(variant: str) -> Path:
    """variant: 'ref' (reference emulation backend), 'oracle', 'hip'."""
    if variant == "ref":
        return REF_DIR / ("libkael_ref-v4.so" if cpu_has_avx512() else "libkael_ref-v3.so")
    return REF_DIR / f"libkael_{variant}.so"


ORACLE_SIGS = dict(kd.SIGNATURES)
ORACLE_SIGS["matmul"] = (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(kd.MatmulSizes), c_int])
ORACLE_SIGS["last_error"] = (c_char_p, [])
ORACLE_SIGS["mt19937_64_draws"] = (c_int, [c_void_p, c_int64, c_void_p])
ORACLE_SIGS["sample_topk"] = (c_int, [c_void_p, c_int64, c_double, c_int64, c_double, POINTER(c_int64)])


def load_oracle() -> ctypes.CDLL:
    lib = ctypes.CDLL(str(ORACLE_LIB))
    kd.bind(lib, "oracle_", ORACLE_SIGS)
    return lib


REF_SIGS = {
    "last_error": (c_char_p, []),
    "set_threads": (None, [c_int64]),
    "get_threads": (c_int64, []),
    "dev_fill": (c_int, [c_int, c_void_p, c_int64, c_void_p]),
    "dev_convert": (c_int, [c_int, c_int, POINTER(kd.ElementLayout)]),
    "dev_elementwise": (c_int, [c_int, c_int, c_int, POINTER(kd.ElementLayout), kd.ElementParameters]),
    "dev_reduce": (c_int, [c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int64]),
    "host_reduce": (c_int, [c_int, c_int, c_void_p, c_void_p, c_int64, c_int64]),
    "dev_matmul": (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(kd.MatmulSizes)]),
    "dev_gather": (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(kd.IndexLayout)]),
    "dev_scatter_add": (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(kd.IndexLayout)]),
    "coalesce": (c_int, [c_int, c_int, POINTER(c_int64), POINTER(c_int64), POINTER(c_int64), POINTER(c_int64)]),
    "matmul": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64]),
    "softmax": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_int]),
    "layer_norm": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_double, c_void_p, c_void_p]),
    "cross_entropy": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64]),
    "cross_entropy_grad": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64]),
    "gelu_backward": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int]),
    "uniform_pm1": (c_int, [ctypes.c_uint64, c_int64, c_void_p]),
    "time_matmul": (c_int, [c_int64, c_int64, c_int64, c_int, POINTER(c_double)]),
    "time_c2": (c_int, [c_int, c_int64, c_int64, c_int, POINTER(c_double)]),
    "gpt_create": (c_void_p, [c_int64, c_int64, c_int64, c_int64, c_int64, ctypes.c_uint64, c_int]),
    "gpt_destroy": (None, [c_void_p]),
    "gpt_param_count": (c_int64, [c_void_p]),
    "gpt_param": (c_int, [c_void_p, c_int64, c_char_p, c_int, POINTER(c_int64), POINTER(c_int), c_void_p]),
    "gpt_forward": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "gpt_cached_logits": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "gpt_generate": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_void_p, POINTER(c_double)]),
    "gpt_set_param": (c_int, [c_void_p, c_int64, c_void_p]),
    "gpt_generate_streamed": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_int64, c_int64, c_void_p,
                                      POINTER(c_int64), c_void_p, POINTER(c_int64)]),
    "golden": (c_int64, [c_char_p, c_char_p, c_int, POINTER(c_void_p), POINTER(c_int), POINTER(c_int),
                         POINTER(c_int64), POINTER(c_char_p), c_int, c_void_p, c_int64, POINTER(c_int),
                         POINTER(c_int), POINTER(c_int64)]),
    "device_available": (c_int, []),
    "train_mlp": (c_int, [c_int, c_int64, c_void_p, c_void_p, POINTER(c_double)]),
    "train_chargpt": (c_int, [c_int, c_int64, c_void_p, POINTER(c_double)]),
    "optim_steps": (c_int, [c_int, c_int, c_int, c_int64, c_int64, c_void_p, c_void_p, c_void_p, c_double, c_double,
                            c_double, c_double, c_double]),
    "train_gpt": (c_int, [c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p,
                          POINTER(c_double)]),
    "gpt_generate_on": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_int64, c_void_p, POINTER(c_double)]),
    "gpt_generate_sampled": (c_int, [c_void_p, c_int, c_void_p, c_int64, c_int64, c_int64, c_double, c_int64,
                                     ctypes.c_uint64, c_void_p, POINTER(c_double), POINTER(c_double)]),
    "train_gpt_params": (c_int, [c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p,
                                 c_void_p, POINTER(c_double)]),
    "gpt_param_total": (c_int64, [c_int64, c_int64, c_int64, c_int64, c_int64]),
    "mt_draws": (c_int, [ctypes.c_uint64, c_int64, c_int64, c_void_p, c_void_p]),
    "bernoulli": (c_int, [ctypes.c_uint64, c_int64, c_int, c_int64, c_double, c_void_p, c_void_p]),
    "dropout": (c_int, [c_int, ctypes.c_uint64, c_int64, c_int, c_void_p, c_int64, c_double, c_void_p, c_void_p,
                        c_void_p, c_void_p]),
    "time_device_bench": (c_int, [c_int, c_int64, c_int, POINTER(c_double)]),
    "gpt_grads": (c_int, [c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p, c_void_p]),
    "row_grad": (c_int, [c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int64, c_double, c_void_p, c_void_p]),
    "linear_grads": (c_int, [c_int, c_int64, c_int64, c_int64, c_int64, ctypes.c_uint64, c_void_p, c_void_p]),
    "head_grads": (c_int, [c_int, c_int64, c_int64, c_int64, c_int64, ctypes.c_uint64, c_void_p, c_void_p]),
    "select_grads": (c_int, [c_int, c_int, ctypes.c_uint64, c_void_p, c_void_p]),
    "attention_chain": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "attention_module": (c_int, [c_int, c_int64, c_int64, c_int64, c_int64, ctypes.c_uint64, c_void_p, c_void_p,
                                 c_void_p]),
    "sample_next": (c_int, [ctypes.c_uint64, c_int64, c_void_p, c_int64, c_double, c_int64, POINTER(c_int64)]),
    "cached_attention_module": (c_int, [c_int, c_int64, c_int64, c_int64, c_int64, c_int64, c_int64, ctypes.c_uint64,
                                        c_void_p, c_void_p]),
    "layer_norm_grads": (c_int, [c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_double,
                                 c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "suite_size": (c_int, []),
    "suite_name": (c_char_p, [c_int]),
    "suite_run": (c_int, [c_int]),
    "suite_message": (c_char_p, []),
    "suite_self_check": (c_int, []),
}


def load_ref(variant: str = "ref") -> ctypes.CDLL:
    path = ref_path(variant)
    lib = ctypes.CDLL(str(path), mode=os.RTLD_NOW | os.RTLD_LOCAL)
    kd.bind(lib, "ref_", REF_SIGS)
    return lib


def ref_error(lib) -> str:
    m = lib.ref_last_error()
    return m.decode() if m else ""


def suite_cases(lib) -> list[str]:
    """Names of the device-behaviour cases in oracle/device_suite.cpp."""
    return [lib.ref_suite_name(i).decode() for i in range(lib.ref_suite_size())]


def run_suite_case(lib, name: str) -> None:
    """Runs one device-behaviour case; fails or skips the calling test as the case does."""
    import pytest

    index = suite_cases(lib).index(name)
    status = lib.ref_suite_run(index)
    message = (lib.ref_suite_message() or b"").decode()
    if status == 2:
        pytest.skip(message)
    assert status == 0, f"{name}: {message}"


def ptr(a: np.ndarray) -> c_void_p:
    return a.ctypes.data_as(c_void_p)


# ---- golden manifest ----------------------------------------------------------------------

NPY_TO_CODE = {np.dtype(np.float32): kd.F32, np.dtype(np.float64): kd.F64,
               np.dtype(np.int64): kd.I64, np.dtype(np.bool_): kd.BOOL}


def golden_cases():
    cases = []
    for line in (GOLDEN / "manifest.txt").read_text().splitlines():
        if not line.strip():
            continue
        fields = dict(tok.split("=", 1) for tok in line.split())
        cases.append(fields)
    return cases


def run_golden(lib, case: dict, device: int):
    """Runs one golden case through kael's API in `lib`; returns (array, expected)."""
    op, name = case["op"], case["case"]
    inputs = case["inputs"].split(",")
    arrays = [np.load(GOLDEN / op / f"{name}_{i}.npy") for i in inputs]
    expected = np.load(GOLDEN / op / f"{name}_out.npy")
    views = [case[f"view_{i}"] for i in inputs]
    return run_op(lib, op, case["args"], arrays, views, device, expected.nbytes), expected


def run_op(lib, op: str, args: str, arrays, views, device: int, out_bytes: int):
    """Runs kael op `op` (the shim's golden op table, arguments as in the golden manifest) on
    `arrays` with the given input views ("none", "transpose", ...); returns the result array.
    `out_bytes` bounds the result size."""
    arrays = [np.require(a.astype(np.uint8) if a.dtype == np.bool_ else a, requirements="C") for a in arrays]
    n = len(arrays)
    datas = (c_void_p * n)(*[a.ctypes.data for a in arrays])
    dtypes = (c_int * n)(*[kd.DTYPE_OF[a.dtype] for a in arrays])
    ranks = (c_int * n)(*[a.ndim for a in arrays])
    shapes = (c_int64 * (8 * n))()
    for i, a in enumerate(arrays):
        for d, s in enumerate(a.shape):
            shapes[8 * i + d] = s
    views = (c_char_p * n)(*[v.encode() for v in views])
    capacity = max(1024, out_bytes * 8 + 1024)
    out = np.zeros(capacity, np.uint8)
    odt, orank = c_int(), c_int()
    oshape = (c_int64 * 8)()
    nbytes = lib.ref_golden(op.encode(), args.encode(), n, datas, dtypes, ranks, shapes, views, device,
                            ptr(out), capacity, ctypes.byref(odt), ctypes.byref(orank), oshape)
    if nbytes < 0:
        raise RuntimeError(f"{op} {args}: {ref_error(lib)}")
    dtype = kd.NUMPY_DTYPE[odt.value]
    shape = tuple(oshape[d] for d in range(orank.value))
    result = out[:nbytes].view(dtype).reshape(shape)
    if dtype == np.uint8:
        result = result.astype(np.bool_)
    return result


def apply_view(x: np.ndarray, view: str) -> np.ndarray:
    """numpy's counterpart of the shim's input views "none", "transpose:a:b" and "permute:..."."""
    name, *args = view.split(":")
    dims = [int(a) for a in args]
    if name == "none":
        return x
    if name == "transpose":
        return np.swapaxes(x, dims[0], dims[1])
    if name == "permute":
        return np.transpose(x, dims)
    raise ValueError(view)


def golden_close(actual: np.ndarray, expected: np.ndarray, rtol=None, atol=None) -> tuple[bool, str]:
    """The reference's allclose (tests/support/allclose.h:21-32) with equal_nan, default
    tolerances f32 1e-5/1e-6, f64 1e-12/1e-14, exact for int64/bool."""
    if actual.shape != expected.shape:
        return False, f"shape {actual.shape} != {expected.shape}"
    if actual.dtype != expected.dtype:
        return False, f"dtype {actual.dtype} != {expected.dtype}"
    if expected.dtype in (np.int64, np.bool_):
        ok = np.array_equal(actual, expected)
        return ok, "" if ok else "integer mismatch"
    if rtol is None:
        rtol, atol = (1e-5, 1e-6) if expected.dtype == np.float32 else (1e-12, 1e-14)
    a = actual.astype(np.float64)
    e = expected.astype(np.float64)
    nan = np.isnan(a) | np.isnan(e)
    both_nan = np.isnan(a) & np.isnan(e)
    inf = np.isinf(a) | np.isinf(e)
    ok = np.ones(a.shape, bool)
    ok[nan] = both_nan[nan]
    fin = ~nan & ~inf
    ok[inf & ~nan] = a[inf & ~nan] == e[inf & ~nan]
    ok[fin] = np.abs(a[fin] - e[fin]) <= atol + rtol * np.abs(e[fin])
    if ok.all():
        return True, ""
    idx = np.argwhere(~ok)[0]
    return False, f"first mismatch at {tuple(idx)}: {a[tuple(idx)]} vs {e[tuple(idx)]} ({(~ok).sum()} bad)"


def export_gpt_params(ref, handle):
    """kael's GPT parameters (GPT::named_parameters() order) as (name, f32 array) pairs."""
    n = ref.ref_gpt_param_count(handle)
    name = ctypes.create_string_buffer(256)
    shape = (c_int64 * 8)()
    rank = c_int()
    out = []
    for i in range(n):
        assert ref.ref_gpt_param(handle, i, name, 256, shape, ctypes.byref(rank), None) == 0
        dims = tuple(shape[d] for d in range(rank.value))
        data = np.empty(dims, np.float32)
        assert ref.ref_gpt_param(handle, i, name, 256, shape, ctypes.byref(rank), data.ctypes.data_as(c_void_p)) == 0
        out.append((name.value.decode(), data))
    return out


def hf_gpt2_tensors(params, prefix_blocks=True):
    """The same weights under Hugging Face GPT-2 names and layouts (Conv1D weights [in, out]),
    with the extra entries a checkpoint carries (the tied lm_head, attention mask buffers), as
    in reference tests/test_transformer.cpp:294-329."""
    own = dict(params)
    hf = {"wte.weight": own["token_embedding.weight"], "wpe.weight": own["position_embedding.weight"],
          "ln_f.weight": own["ln_final.weight"], "ln_f.bias": own["ln_final.bias"],
          "lm_head.weight": own["token_embedding.weight"]}
    layers = sum(1 for n in own if n.endswith(".ln1.weight"))
    for i in range(layers):
        h = ("transformer.h." if prefix_blocks else "h.") + f"{i}."
        b = f"blocks.{i}."
        hf[h + "ln_1.weight"], hf[h + "ln_1.bias"] = own[b + "ln1.weight"], own[b + "ln1.bias"]
        hf[h + "ln_2.weight"], hf[h + "ln_2.bias"] = own[b + "ln2.weight"], own[b + "ln2.bias"]
        for hname, kname in (("attn.c_attn", "attn.qkv"), ("attn.c_proj", "attn.proj"), ("mlp.c_fc", "mlp.fc1"),
                             ("mlp.c_proj", "mlp.fc2")):
            hf[h + hname + ".weight"] = np.ascontiguousarray(own[b + kname + ".weight"].T)
            hf[h + hname + ".bias"] = own[b + kname + ".bias"]
        hf[h + "attn.bias"] = np.zeros((1,), np.float32)
    return hf

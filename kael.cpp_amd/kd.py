"""ctypes binding of the gfx950 backend's C ABI (include/kd_api.h).

`load()` opens kael.cpp_amd/lib/libkd.so and returns a `Backend` whose methods raise
`KdError` on a non-zero status. There is no fallback: a missing library or device is an error.
The same structure classes describe layouts for the test oracle, whose entry points share
these signatures.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libkd.so"

MAX_DIMS = 8
MAX_OPERANDS = 4

F32, F64, I64, BOOL = 0, 1, 2, 3
NUMPY_DTYPE = {F32: np.float32, F64: np.float64, I64: np.int64, BOOL: np.uint8}
DTYPE_OF = {np.dtype(np.float32): F32, np.dtype(np.float64): F64, np.dtype(np.int64): I64,
            np.dtype(np.uint8): BOOL, np.dtype(np.bool_): BOOL}

OPS = [
    "PLUS", "MINUS", "TIMES", "DIVIDES", "POWER", "MAXIMUM", "MINIMUM", "EQUAL", "NOT_EQUAL",
    "LESS", "LESS_EQUAL", "GREATER", "GREATER_EQUAL", "LOGICAL_AND", "LOGICAL_OR",
    "LOGICAL_XOR", "IS_ZERO", "NEGATE", "ABSOLUTE", "SIGN", "EXP", "LOG", "LOG1P", "EXPM1",
    "SQRT", "RSQRT", "SIN", "COS", "TANH", "SIGMOID", "RELU", "GELU_EXACT", "GELU_TANH",
    "CLAMP", "WHERE", "MASKED_FILL",
]
OP = {name: i for i, name in enumerate(OPS)}
OP["GELU_EXACT_BACKWARD"] = 64
OP["GELU_TANH_BACKWARD"] = 65
COMPARE_OPS = {OP[n] for n in ("EQUAL", "NOT_EQUAL", "LESS", "LESS_EQUAL", "GREATER",
                               "GREATER_EQUAL", "LOGICAL_AND", "LOGICAL_OR", "LOGICAL_XOR")}
FLOATING_OPS = {OP[n] for n in ("EXP", "LOG", "LOG1P", "EXPM1", "SQRT", "RSQRT", "SIN", "COS",
                                "TANH", "SIGMOID", "GELU_EXACT", "GELU_TANH",
                                "GELU_EXACT_BACKWARD", "GELU_TANH_BACKWARD")}
REDUCE_SUM, REDUCE_MAX, REDUCE_MIN = 0, 1, 2
REDUCE_PROD, REDUCE_ALL, REDUCE_ANY = 16, 17, 18  # extensions (kael computes these on the host)


def op_inputs(op: int) -> int:
    if op <= OP["LOGICAL_XOR"]:
        return 2
    if op == OP["WHERE"]:
        return 3
    if op in (OP["MASKED_FILL"], OP["GELU_EXACT_BACKWARD"], OP["GELU_TANH_BACKWARD"]):
        return 2
    return 1


class KdError(RuntimeError):
    pass


class ElementParameters(Structure):
    _fields_ = [("reals", c_double * 2), ("integers", c_int64 * 2)]


class ElementLayout(Structure):
    _fields_ = [("dims", c_int32), ("operands", c_int32), ("count", c_int64),
                ("shape", c_int64 * MAX_DIMS), ("strides", (c_int64 * MAX_DIMS) * MAX_OPERANDS),
                ("base", c_void_p * MAX_OPERANDS)]


class IndexLayout(Structure):
    _fields_ = [("dims", c_int32), ("axis", c_int32), ("count", c_int64),
                ("shape", c_int64 * MAX_DIMS), ("data_strides", c_int64 * MAX_DIMS),
                ("index_strides", c_int64 * MAX_DIMS), ("source_strides", c_int64 * MAX_DIMS)]


class MatmulSizes(Structure):
    _fields_ = [("batches", c_int64), ("rows", c_int64), ("inner", c_int64), ("columns", c_int64)]


class MatmulStrides(Structure):
    _fields_ = [("a", c_int64 * 3), ("b", c_int64 * 3), ("out", c_int64 * 3)]


class MatmulHeads(Structure):
    _fields_ = [("heads", c_int64), ("a", c_int64), ("b", c_int64), ("out", c_int64)]


class AdamTensor(Structure):
    _fields_ = [("param", c_void_p), ("grad", c_void_p), ("first", c_void_p), ("second", c_void_p),
                ("count", c_int64), ("step", c_int64)]


class GptConfig(Structure):
    _fields_ = [("vocab_size", c_int64), ("max_positions", c_int64), ("layers", c_int64), ("heads", c_int64),
                ("dimension", c_int64), ("tanh_gelu", c_int32), ("flags", c_int32)]


assert ctypes.sizeof(ElementLayout) == 368
assert ctypes.sizeof(IndexLayout) == 272


def params(reals=(0.0, 0.0), integers=(0, 0)) -> ElementParameters:
    p = ElementParameters()
    p.reals[0], p.reals[1] = float(reals[0]), float(reals[1])
    p.integers[0], p.integers[1] = int(integers[0]), int(integers[1])
    return p


# name -> (restype, argtypes); shared by the backend (prefix kd_) and the oracle (oracle_).
SIGNATURES = {
    "fill": (c_int, [c_int, c_void_p, c_int64, c_void_p]),
    "convert": (c_int, [c_int, c_int, POINTER(ElementLayout)]),
    "elementwise": (c_int, [c_int, c_int, c_int, POINTER(ElementLayout), ElementParameters]),
    "reduce": (c_int, [c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int64]),
    "reduce_columns": (c_int, [c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int64]),
    "arg_reduce": (c_int, [c_int, c_int, c_void_p, c_void_p, c_int64, c_int64]),
    "cumsum": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64]),
    "mt19937_64_seed": (None, [c_void_p, ctypes.c_uint64]),
    "bernoulli": (c_int, [c_int, c_void_p, c_int64, c_double, c_void_p]),
    "dropout": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_double, c_void_p]),
    "gather": (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(IndexLayout)]),
    "scatter_add": (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(IndexLayout)]),
    "index_bounds": (c_int, [c_void_p, c_int64, c_int64, c_void_p]),
    "causal_attention": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64]),
    "causal_attention_backward": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
                                          c_int64, c_int64]),
    "cached_attention": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                 c_int64, c_int64, c_int64, c_int64]),
    "softmax_rows": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_int]),
    "standardize_rows": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_int64, c_double, c_void_p, c_void_p]),
    "cross_entropy_rows": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64]),
    "cross_entropy_grad": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64]),
    "softmax_rows_backward": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int]),
    "standardize_rows_backward": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64,
                                          c_double]),
    "layer_norm_rows": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_double, c_void_p, c_void_p]),
    "layer_norm_rows_backward": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                         c_int64, c_int64, c_double]),
    "adam_step": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_double, c_double, c_double,
                          c_double, c_double, c_int, c_int64]),
    "adam_step_many": (c_int, [c_int, POINTER(AdamTensor), c_int64, c_double, c_double, c_double, c_double, c_double,
                               c_int]),
    "sgd_step": (c_int, [c_int, c_void_p, c_void_p, c_int64, c_double, c_double]),
    "matmul_strided": (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(MatmulSizes), POINTER(MatmulStrides)]),
    "matmul_strided_bias": (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(MatmulSizes), POINTER(MatmulStrides),
                                    c_void_p]),
    "matmul_strided_heads": (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(MatmulSizes), POINTER(MatmulStrides),
                                     POINTER(MatmulHeads)]),
    "layout_build": (c_int, [POINTER(ElementLayout), c_int, POINTER(c_int), POINTER(c_int64),
                             POINTER(c_int64), POINTER(c_int), POINTER(c_void_p)]),
}
BACKEND_ONLY = {
    "last_error": (c_char_p, []),
    "available": (c_int, []),
    "synchronize": (c_int, []),
    "set_stream": (c_int, [c_void_p]),
    "get_stream": (c_void_p, []),
    "malloc": (c_int, [POINTER(c_void_p), c_int64]),
    "free": (None, [c_void_p]),
    "copy_h2d": (c_int, [c_void_p, c_void_p, c_int64]),
    "copy_d2h": (c_int, [c_void_p, c_void_p, c_int64]),
    "copy_d2d": (c_int, [c_void_p, c_void_p, c_int64]),
    "matmul": (c_int, [c_int, c_void_p, c_void_p, c_void_p, POINTER(MatmulSizes)]),
    "reduce_noalloc": (c_int, [c_int, c_int, c_int, c_void_p, c_void_p, c_int64, c_int64]),
    "event_create": (c_int, [POINTER(c_void_p)]),
    "event_destroy": (c_int, [c_void_p]),
    "event_record": (c_int, [c_void_p]),
    "event_elapsed_ms": (c_int, [POINTER(c_float), c_void_p, c_void_p]),
    "device_info": (c_int, [POINTER(c_int), POINTER(c_int), ctypes.c_char_p, c_int]),
    "gpt_create": (c_int, [POINTER(c_void_p), POINTER(GptConfig)]),
    "gpt_destroy": (None, [c_void_p]),
    "gpt_load_parameter": (c_int, [c_void_p, ctypes.c_char_p, c_void_p, c_int64]),
    "gpt_load_parameter_device": (c_int, [c_void_p, ctypes.c_char_p, c_void_p, c_int64]),
    "gpt_load_safetensors": (c_int, [c_void_p, ctypes.c_char_p]),
    "safetensors_tensor": (c_int, [ctypes.c_char_p, ctypes.c_char_p, c_void_p, c_int64, POINTER(c_int64),
                                   POINTER(c_int32)]),
    "gpt_supported": (c_int, [POINTER(GptConfig)]),
    "gpt_kael_init": (c_int, [POINTER(GptConfig), ctypes.c_uint64, c_void_p, c_int64, POINTER(c_int64)]),
    "gpt_prefill": (c_int, [c_void_p, c_void_p, c_int64]),
    "gpt_decode": (c_int, [c_void_p, c_int64, c_void_p]),
    "gpt_forward_logits": (c_int, [c_void_p, c_void_p, c_int64, c_void_p]),
    "gpt_sequence": (c_int, [c_void_p, c_void_p, c_int64, POINTER(c_int64)]),
    "gpt_logits": (c_int, [c_void_p, c_void_p]),
    "gpt_set_sampling": (c_int, [c_void_p, c_double, c_int64]),
    "gpt_set_uniforms": (c_int, [c_void_p, c_void_p, c_int64]),
    "gpt_draws_used": (c_int, [c_void_p, POINTER(c_int64)]),
}

# Every symbol include/kd_api.h declares.
EXPORTED = sorted({"kd_" + n for n in SIGNATURES} | {"kd_" + n for n in BACKEND_ONLY})


def bind(lib: ctypes.CDLL, prefix: str, names: dict) -> None:
    for name, (restype, argtypes) in names.items():
        fn = getattr(lib, prefix + name)
        fn.restype = restype
        fn.argtypes = argtypes


class Backend:
    """The loaded library plus thin checked wrappers."""

    def __init__(self, path: Path = LIB_PATH):
        if not Path(path).is_file():
            raise KdError(f"{path} is missing: build it with `python kael.cpp_amd/build.py`")
        self.lib = ctypes.CDLL(str(path), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
        bind(self.lib, "kd_", SIGNATURES)
        bind(self.lib, "kd_", BACKEND_ONLY)
        self.path = Path(path)

    def error(self) -> str:
        msg = self.lib.kd_last_error()
        return msg.decode() if msg else ""

    def check(self, rc: int, what: str = "") -> None:
        if rc != 0:
            raise KdError(f"{what} failed ({rc}): {self.error()}")

    def call(self, name: str, *args) -> None:
        self.check(getattr(self.lib, "kd_" + name)(*args), "kd_" + name)

    # -- memory --
    def malloc(self, nbytes: int) -> int:
        p = c_void_p()
        self.check(self.lib.kd_malloc(ctypes.byref(p), int(nbytes)), "kd_malloc")
        return p.value or 0

    def free(self, ptr: int) -> None:
        self.lib.kd_free(c_void_p(ptr))

    def to_device(self, arr: np.ndarray) -> "DeviceArray":
        arr = np.ascontiguousarray(arr)
        buf = DeviceArray(self, arr.shape, arr.dtype)
        self.check(self.lib.kd_copy_h2d(c_void_p(buf.ptr), arr.ctypes.data_as(c_void_p), arr.nbytes), "kd_copy_h2d")
        return buf

    def empty(self, shape, dtype) -> "DeviceArray":
        return DeviceArray(self, tuple(shape), np.dtype(dtype))

    def synchronize(self) -> None:
        self.check(self.lib.kd_synchronize(), "kd_synchronize")

    def device_info(self) -> dict:
        cus, clk = c_int(), c_int()
        arch = ctypes.create_string_buffer(64)
        self.check(self.lib.kd_device_info(ctypes.byref(cus), ctypes.byref(clk), arch, 64), "kd_device_info")
        return {"compute_units": cus.value, "clock_khz": clk.value, "arch": arch.value.decode()}


class DeviceArray:
    """A device allocation with a numpy-like shape/dtype; freed when collected."""

    def __init__(self, backend: Backend, shape, dtype):
        self.backend = backend
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        self.ptr = backend.malloc(max(self.nbytes, 1))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            self.backend.check(self.backend.lib.kd_copy_d2h(out.ctypes.data_as(c_void_p), c_void_p(self.ptr), self.nbytes),
                               "kd_copy_d2h")
        return out

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        assert arr.nbytes == self.nbytes
        self.backend.check(self.backend.lib.kd_copy_h2d(c_void_p(self.ptr), arr.ctypes.data_as(c_void_p), arr.nbytes),
                           "kd_copy_h2d")

    def __del__(self):
        try:
            if self.ptr:
                self.backend.free(self.ptr)
                self.ptr = 0
        except Exception:
            pass


class Gpt:
    """The GPT-2 decode engine (kd_gpt_*): kael's parameter names and layout, greedy decoding."""

    EAGER = 1
    STEPWISE_PREFILL = 2

    def __init__(self, backend: Backend, vocab_size=50257, max_positions=1024, layers=12, heads=12, dimension=768,
                 tanh_gelu=True, eager=False, stepwise_prefill=False):
        self.b = backend
        flags = (self.EAGER if eager else 0) | (self.STEPWISE_PREFILL if stepwise_prefill else 0)
        self.config = GptConfig(vocab_size, max_positions, layers, heads, dimension, int(bool(tanh_gelu)), flags)
        h = c_void_p()
        backend.check(backend.lib.kd_gpt_create(ctypes.byref(h), ctypes.byref(self.config)), "kd_gpt_create")
        self.handle = h

    def load(self, name: str, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array, dtype=np.float32)
        self.b.check(self.b.lib.kd_gpt_load_parameter(self.handle, name.encode(), a.ctypes.data_as(c_void_p), a.size),
                     f"kd_gpt_load_parameter({name})")

    def load_gpt2_safetensors(self, path) -> None:
        """Loads a Hugging Face GPT-2 checkpoint (`model.safetensors`) through the library's own
        reader (kd_gpt_load_safetensors), as kael's load_gpt2_weights does (reference
        src/nn/transformer.cpp:297-308): the file memory-mapped and checked, names translated,
        Conv1D weights transposed, entries kael's GPT does not have ignored, a missing one an
        error."""
        self.b.check(self.b.lib.kd_gpt_load_safetensors(self.handle, os.fsencode(str(path))),
                     "kd_gpt_load_safetensors")

    def prefill(self, prompt) -> None:
        p = np.ascontiguousarray(prompt, dtype=np.int64)
        self.b.check(self.b.lib.kd_gpt_prefill(self.handle, p.ctypes.data_as(c_void_p), p.size), "kd_gpt_prefill")

    def decode(self, count: int) -> np.ndarray:
        out = np.zeros(max(count, 1), np.int64)
        self.b.check(self.b.lib.kd_gpt_decode(self.handle, count, out.ctypes.data_as(c_void_p)), "kd_gpt_decode")
        return out[:count]

    def forward_logits(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int64)
        out = np.empty((t.size, self.config.vocab_size), np.float32)
        self.b.check(self.b.lib.kd_gpt_forward_logits(self.handle, t.ctypes.data_as(c_void_p), t.size,
                                                      out.ctypes.data_as(c_void_p)), "kd_gpt_forward_logits")
        return out

    def set_sampling(self, temperature: float, top_k: int = 0) -> None:
        self.b.check(self.b.lib.kd_gpt_set_sampling(self.handle, float(temperature), int(top_k)), "kd_gpt_set_sampling")

    def set_uniforms(self, uniforms) -> None:
        u = np.ascontiguousarray(uniforms, dtype=np.float64)
        self.b.check(self.b.lib.kd_gpt_set_uniforms(self.handle, u.ctypes.data_as(c_void_p), u.size),
                     "kd_gpt_set_uniforms")

    def draws_used(self) -> int:
        n = c_int64()
        self.b.check(self.b.lib.kd_gpt_draws_used(self.handle, ctypes.byref(n)), "kd_gpt_draws_used")
        return n.value

    def logits(self) -> np.ndarray:
        """Logits of the most recent position (the prompt's last after prefill)."""
        out = np.empty(self.config.vocab_size, np.float32)
        self.b.check(self.b.lib.kd_gpt_logits(self.handle, out.ctypes.data_as(c_void_p)), "kd_gpt_logits")
        return out

    def sequence(self) -> np.ndarray:
        n = c_int64()
        self.b.check(self.b.lib.kd_gpt_sequence(self.handle, None, 0, ctypes.byref(n)), "kd_gpt_sequence")
        buf = np.zeros(max(n.value, 1), np.int64)
        self.b.check(self.b.lib.kd_gpt_sequence(self.handle, buf.ctypes.data_as(c_void_p), buf.size, ctypes.byref(n)),
                     "kd_gpt_sequence")
        return buf[:n.value]

    def __del__(self):
        try:
            if self.handle:
                self.b.lib.kd_gpt_destroy(self.handle)
                self.handle = None
        except Exception:
            pass


def gpt2_parameter_shapes(vocab_size=50257, max_positions=1024, layers=12, dimension=768):
    """kael's GPT parameter names and shapes in GPT::named_parameters() order."""
    d = dimension
    shapes = [("token_embedding.weight", (vocab_size, d)), ("position_embedding.weight", (max_positions, d))]
    for l in range(layers):
        b = f"blocks.{l}."
        shapes += [(b + "ln1.weight", (d,)), (b + "ln1.bias", (d,)), (b + "attn.qkv.weight", (3 * d, d)),
                   (b + "attn.qkv.bias", (3 * d,)), (b + "attn.proj.weight", (d, d)), (b + "attn.proj.bias", (d,)),
                   (b + "ln2.weight", (d,)), (b + "ln2.bias", (d,)), (b + "mlp.fc1.weight", (4 * d, d)),
                   (b + "mlp.fc1.bias", (4 * d,)), (b + "mlp.fc2.weight", (d, 4 * d)), (b + "mlp.fc2.bias", (d,))]
    shapes += [("ln_final.weight", (d,)), ("ln_final.bias", (d,))]
    return shapes


def kael_gpt_parameters(backend: "Backend", seed: int, vocab_size=50257, max_positions=1024, layers=12, heads=12,
                        dimension=768) -> list:
    """kael's GPT parameters after manual_seed(seed) (kd_gpt_kael_init, host only) as (name, f32 array)
    pairs in GPT::named_parameters() order; the arrays are views of one buffer."""
    cfg = GptConfig(vocab_size, max_positions, layers, heads, dimension, 1, 0)
    total = c_int64()
    backend.check(backend.lib.kd_gpt_kael_init(ctypes.byref(cfg), seed, None, 0, ctypes.byref(total)),
                  "kd_gpt_kael_init")
    flat = np.empty(total.value, np.float32)
    backend.check(backend.lib.kd_gpt_kael_init(ctypes.byref(cfg), seed, flat.ctypes.data_as(c_void_p), flat.size,
                                               ctypes.byref(total)), "kd_gpt_kael_init")
    out, at = [], 0
    for name, shape in gpt2_parameter_shapes(vocab_size, max_positions, layers, dimension):
        n = int(np.prod(shape))
        out.append((name, flat[at:at + n].reshape(shape)))
        at += n
    assert at == flat.size
    return out


_BACKEND: Backend | None = None


def load() -> Backend:
    global _BACKEND
    if _BACKEND is None:
        _BACKEND = Backend()
    return _BACKEND


def index_layout(shape, axis, data_strides, index_strides, source_strides) -> IndexLayout:
    """kd_index_layout for an iteration `shape` with the gathered / scattered `axis` and element
    strides of the data, index and source (or output) tensors per dim."""
    lay = IndexLayout()
    lay.dims = len(shape)
    lay.axis = axis
    lay.count = int(np.prod(shape)) if len(shape) else 1
    for d in range(len(shape)):
        lay.shape[d] = shape[d]
        lay.data_strides[d] = data_strides[d]
        lay.index_strides[d] = index_strides[d]
        lay.source_strides[d] = source_strides[d]
    return lay


def element_layout(shape, strides_bytes, bases) -> ElementLayout:
    """An ElementLayout from explicit dims: shape (d), per-operand byte strides [ops][d]."""
    lay = ElementLayout()
    lay.dims = len(shape)
    lay.operands = len(bases)
    lay.count = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    for d, s in enumerate(shape):
        lay.shape[d] = int(s)
    for op, st in enumerate(strides_bytes):
        for d, s in enumerate(st):
            lay.strides[op][d] = int(s)
    for op, b in enumerate(bases):
        lay.base[op] = b
    return lay


def safetensors_tensor(backend: Backend, path, name: str) -> np.ndarray:
    """One tensor of a safetensors file as float32, read by the library on the host
    (kd_safetensors_tensor): no device is needed."""
    dims = c_int32()
    shape = (c_int64 * MAX_DIMS)()
    p, n = os.fsencode(str(path)), name.encode()
    backend.check(backend.lib.kd_safetensors_tensor(p, n, None, 0, shape, ctypes.byref(dims)), "kd_safetensors_tensor")
    out = np.empty(tuple(shape[i] for i in range(dims.value)), np.float32)
    backend.check(backend.lib.kd_safetensors_tensor(p, n, out.ctypes.data_as(c_void_p), out.size, shape,
                                                    ctypes.byref(dims)), "kd_safetensors_tensor")
    return out

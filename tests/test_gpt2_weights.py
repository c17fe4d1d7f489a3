"""The library's own safetensors reader (kael.cpp_amd/host/kd_safetensors.cpp) behind
kd_safetensors_tensor and kd_gpt_load_safetensors, on the CPU.

Against the reference's reader (src/io/safetensors.cpp:64-133,258-318): kael's own GPT weights
written in Hugging Face layout read back bit for bit; F64 / I64 / BOOL convert as kael's copy_ into
an f32 tensor converts them (static_cast); F16 and BF16 widen exactly; every malformed file the
reference rejects is rejected (header too long for the file, JSON that is not an object or has
trailing text, entries without dtype / shape / two offsets, negative or non-integer dims,
offsets whose span is not numel x element size, entries that do not tile the data, bool bytes
above 1, non-string metadata, bad strings); an unknown dtype is KD_E_UNSUPPORTED. kael's GPT-2 name
translation and Conv1D transposes (reference src/nn/transformer.cpp:54-89 and its tests
tests/test_transformer.cpp:286-329) through a small C++ driver built from the same source. The
engine-side checks (missing or misshapen parameters, entries kael's GPT does not have) need a
device and are in tests/test_gpu_gpt2.py.
"""
import json
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import kd
import support

ROOT = Path(__file__).resolve().parents[1]
HOST = ROOT / "kael.cpp_amd" / "host"


@pytest.fixture(scope="module")
def lib():
    return kd.Backend()


def read(lib, path, name):
    return kd.safetensors_tensor(lib, path, name)


def status(lib, path, name="x"):
    dims = kd.c_int32()
    return lib.lib.kd_safetensors_tensor(str(path).encode(), name.encode(), None, 0, None, kd.ctypes.byref(dims))


def write_raw(path, header, data=b"", header_size=None):
    text = json.dumps(header).encode() if not isinstance(header, bytes) else header
    n = len(text) if header_size is None else header_size
    path.write_bytes(struct.pack("<Q", n) + text + data)
    return path


@pytest.fixture
def kael_params(refdev):
    h = refdev.ref_gpt_create(11, 16, 2, 2, 8, 5, 1)
    assert h, support.ref_error(refdev)
    try:
        yield support.export_gpt_params(refdev, h)
    finally:
        refdev.ref_gpt_destroy(h)


def test_kael_weights_round_trip(tmp_path, lib, kael_params):
    from safetensors.numpy import save_file

    hf = support.hf_gpt2_tensors(kael_params)
    path = tmp_path / "model.safetensors"
    save_file(hf, str(path), metadata={"format": "pt"})
    for name, array in hf.items():
        got = read(lib, path, name)
        assert got.shape == array.shape
        np.testing.assert_array_equal(got, array, err_msg=name)


def test_dtype_conversions(tmp_path, lib):
    rng = np.random.default_rng(0)
    f64 = rng.normal(0, 3, 7)
    i64 = np.array([0, 1, -5, 2 ** 40 + 1, -(2 ** 53) - 3], np.int64)
    boo = np.array([1, 0, 1, 1], np.uint8)
    f16 = np.array([0.0, -0.0, 1.5, 65504.0, 6.0e-8, -3.0e-5, np.inf, -np.inf], np.float16)
    bf16_bits = np.array([0x3F80, 0xC2F7, 0x0001, 0x7F80, 0x8000], np.uint16)  # 1, -123.5, subnormal, inf, -0
    parts = [("a_f64", "F64", f64.tobytes(), [7]), ("b_i64", "I64", i64.tobytes(), [5]),
             ("c_bool", "BOOL", boo.tobytes(), [2, 2]), ("d_f16", "F16", f16.tobytes(), [8]),
             ("e_bf16", "BF16", bf16_bits.tobytes(), [5])]
    header, data = {}, b""
    for name, dt, raw, shape in parts:
        header[name] = {"dtype": dt, "shape": shape, "data_offsets": [len(data), len(data) + len(raw)]}
        data += raw
    path = write_raw(tmp_path / "t.safetensors", header, data)
    np.testing.assert_array_equal(read(lib, path, "a_f64"), f64.astype(np.float32))
    np.testing.assert_array_equal(read(lib, path, "b_i64"), i64.astype(np.float32))
    np.testing.assert_array_equal(read(lib, path, "c_bool"), boo.reshape(2, 2).astype(np.float32))
    np.testing.assert_array_equal(read(lib, path, "d_f16"), f16.astype(np.float32))
    assert np.signbit(read(lib, path, "d_f16")[1])
    want = (bf16_bits.astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(read(lib, path, "e_bf16"), want)


def test_f16_nan_and_subnormals_widen_exactly(tmp_path, lib):
    bits = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16)  # every half value
    path = write_raw(tmp_path / "h.safetensors", {"h": {"dtype": "F16", "shape": [1 << 16],
                                                       "data_offsets": [0, 2 << 16]}}, bits.tobytes())
    got = read(lib, path, "h")
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(got[~nan], want[~nan])


def entry(dtype="F32", shape=(2,), begin=0, end=8):
    return {"dtype": dtype, "shape": list(shape), "data_offsets": [begin, end]}


@pytest.mark.parametrize("case", [
    "short_file", "header_past_end", "not_json", "trailing_text", "not_object", "no_dtype", "no_shape",
    "one_offset", "negative_dim", "float_dim", "span_mismatch", "gap", "overlap", "short_data", "bool_byte",
    "metadata_not_string", "control_char", "lone_surrogate", "bad_utf8", "missing_name",
])
def test_malformed_files_are_rejected(tmp_path, lib, case):
    p = tmp_path / "bad.safetensors"
    eight = np.ones(2, np.float32).tobytes()
    if case == "short_file":
        p.write_bytes(b"\x01\x00")
    elif case == "header_past_end":
        write_raw(p, {"x": entry()}, eight, header_size=10_000)
    elif case == "not_json":
        write_raw(p, b'{"x": ', eight)
    elif case == "trailing_text":
        write_raw(p, json.dumps({"x": entry()}).encode() + b" x", eight)
    elif case == "not_object":
        write_raw(p, b"[1, 2]", b"")
    elif case == "no_dtype":
        write_raw(p, {"x": {"shape": [2], "data_offsets": [0, 8]}}, eight)
    elif case == "no_shape":
        write_raw(p, {"x": {"dtype": "F32", "data_offsets": [0, 8]}}, eight)
    elif case == "one_offset":
        write_raw(p, {"x": {"dtype": "F32", "shape": [2], "data_offsets": [0]}}, eight)
    elif case == "negative_dim":
        write_raw(p, {"x": entry(shape=(-2,))}, eight)
    elif case == "float_dim":
        write_raw(p, {"x": entry(shape=(2.0,))}, eight)
    elif case == "span_mismatch":
        write_raw(p, {"x": entry(shape=(3,))}, eight)
    elif case == "gap":
        write_raw(p, {"x": entry(begin=4, end=12)}, b"\0" * 12)
    elif case == "overlap":
        write_raw(p, {"x": entry(), "y": entry(begin=4, end=12)}, b"\0" * 12)
    elif case == "short_data":
        write_raw(p, {"x": entry()}, eight[:4])
    elif case == "bool_byte":
        write_raw(p, {"x": entry(dtype="BOOL", shape=(2,), end=2)}, b"\x01\x02")
    elif case == "metadata_not_string":
        write_raw(p, {"__metadata__": {"k": 1}, "x": entry()}, eight)
    elif case == "control_char":
        write_raw(p, b'{"x\x01": ' + json.dumps(entry()).encode() + b"}", eight)
    elif case == "lone_surrogate":
        write_raw(p, b'{"x\\ud800": ' + json.dumps(entry()).encode() + b"}", eight)
    elif case == "bad_utf8":
        write_raw(p, b'{"x\xff": ' + json.dumps(entry()).encode() + b"}", eight)
    elif case == "missing_name":
        write_raw(p, {"y": entry()}, eight)
    assert status(lib, p) == -1  # KD_E_INVALID
    assert lib.error()


def test_unknown_dtype_is_unsupported(tmp_path, lib):
    p = write_raw(tmp_path / "u.safetensors", {"x": entry(dtype="F8_E4M3", end=2)}, b"\0\0")
    assert status(lib, p) == -4  # KD_E_UNSUPPORTED


def test_json_details(tmp_path, lib):
    """Escapes and unicode in names, whitespace and padding, a repeated name (its last
    description counts), empty tensors, and metadata are read as the reference's parser reads them."""
    eight = np.array([1.0, -2.0], np.float32).tobytes()
    text = ('{"__metadata__": {"a": "b"}, "x\\u00e9\\n\\ud83d\\ude00": {"dtype": "F32", "shape": [2], '
            '"data_offsets": [0, 8]}, "z": {"dtype": "F32", "shape": [0, 3], "data_offsets": [8, 8]}, '
            '"y": {"dtype": "F32", "shape": [9], "data_offsets": [0, 36]}, '
            '"y": {"dtype": "I64", "shape": [1], "data_offsets": [8, 16]}}').encode()
    text += b" " * (-len(text) % 8)
    p = write_raw(tmp_path / "j.safetensors", text, eight + struct.pack("<q", 7))
    np.testing.assert_array_equal(read(lib, p, "xé\n\U0001F600"), [1.0, -2.0])
    np.testing.assert_array_equal(read(lib, p, "y"), [7.0])
    assert read(lib, p, "z").shape == (0, 3)


def test_gpt2_names_follow_the_reference_translation(tmp_path):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("no g++")
    exe = tmp_path / "gpt2_names"
    subprocess.run([gxx, "-std=c++20", "-O1", f"-I{HOST}", str(ROOT / "tests" / "cpp" / "gpt2_names.cpp"),
                    str(HOST / "kd_safetensors.cpp"), "-o", str(exe)], check=True)
    cases = {
        "transformer.h.1.attn.c_attn.weight": ("blocks.1.attn.qkv.weight", 1),
        "transformer.h.1.attn.c_attn.bias": ("blocks.1.attn.qkv.bias", 0),
        "h.0.mlp.c_proj.bias": ("blocks.0.mlp.fc2.bias", 0),
        "h.0.mlp.c_proj.weight": ("blocks.0.mlp.fc2.weight", 1),
        "h.3.mlp.c_fc.weight": ("blocks.3.mlp.fc1.weight", 1),
        "h.2.attn.c_proj.weight": ("blocks.2.attn.proj.weight", 1),
        "h.10.ln_2.weight": ("blocks.10.ln2.weight", 0),
        "h.10.ln_1.bias": ("blocks.10.ln1.bias", 0),
        "wte.weight": ("token_embedding.weight", 0),
        "transformer.wpe.weight": ("position_embedding.weight", 0),
        "ln_f.bias": ("ln_final.bias", 0),
        "lm_head.weight": ("lm_head.weight", 0),
        "h.0.attn.bias": ("blocks.0.attn.bias", 0),
    }
    out = subprocess.run([str(exe), *cases], check=True, capture_output=True, text=True).stdout.split("\n")
    for (stored, (name, transposed)), line in zip(cases.items(), out):
        assert line == f"{name} {transposed}", stored


def test_reader_survives_mutated_files(tmp_path, lib):
    """Seeded mutations of a valid file (bytes of the header and its length field overwritten,
    bytes inserted or removed, the file truncated): every call returns a status (OK only when the
    tensor then reads back at its full size). Run against a library whose host code is built with
    AddressSanitizer and UndefinedBehaviorSanitizer, a stray access here fails the run."""
    from safetensors.numpy import save_file

    good = tmp_path / "good.safetensors"
    save_file({"x": np.arange(24, dtype=np.float32).reshape(4, 6), "y": np.ones(3, np.float64)}, str(good))
    base = bytearray(good.read_bytes())
    header_end = 8 + struct.unpack("<Q", bytes(base[:8]))[0]
    rng = np.random.default_rng(12)
    path = tmp_path / "m.safetensors"
    for trial in range(300):
        data = bytearray(base)
        kind = trial % 4
        if kind == 0:  # overwrite header bytes
            for _ in range(int(rng.integers(1, 6))):
                data[int(rng.integers(0, header_end))] = int(rng.integers(0, 256))
        elif kind == 1:  # insert bytes into the header
            at = int(rng.integers(8, header_end))
            data[at:at] = bytes(rng.integers(0, 256, int(rng.integers(1, 5))).astype(np.uint8))
        elif kind == 2:  # remove bytes
            at = int(rng.integers(0, len(data) - 1))
            del data[at:at + int(rng.integers(1, 9))]
        else:  # truncate
            data = data[:int(rng.integers(0, len(data)))]
        path.write_bytes(bytes(data))
        for name in ("x", "y"):
            rc = status(lib, path, name)
            assert rc in (0, -1, -4), (trial, name, rc)
            if rc == 0:
                shape = (kd.c_int64 * 8)()
                dims = kd.c_int32()
                assert lib.lib.kd_safetensors_tensor(str(path).encode(), name.encode(), None, 0, shape,
                                                     kd.ctypes.byref(dims)) == 0
                count = int(np.prod([shape[i] for i in range(dims.value)])) if dims.value else 1
                out = np.empty(max(count, 1), np.float32)
                assert lib.lib.kd_safetensors_tensor(str(path).encode(), name.encode(),
                                                     out.ctypes.data_as(kd.c_void_p), out.size, None,
                                                     kd.ctypes.byref(dims)) == 0

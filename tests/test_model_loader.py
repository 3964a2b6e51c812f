"""Checkpoint loader (host side, CPU only).

* Every malformed-header case fails with the same message as the reference's
  load_safetensors (src/io/safetensors.cpp:237-608, compiled into
  oracle/_ref), and every well-formed case loads the same tensors.
* Decoded values (BF16 / F16 / F32, incl. F16 subnormals, infinities, NaN
  payloads and -0) are bit-exact against numpy's own conversions and against
  the reference loader.
* load_linear_bf16_transposed matches the reference bit for bit.
The tool under test is build/bin/tool_model (tests/cpp/tool_model.cpp), or
the binary SKV_TOOL_MODEL names (tests/test_host_sanitizers.py runs this
module against the AddressSanitizer/UBSan build).
"""
import ctypes
import json
import os
import struct
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOOL = os.environ.get("SKV_TOOL_MODEL") or os.path.join(ROOT, "build", "bin", "tool_model")
REF = os.path.join(ROOT, "oracle", "_ref", "libstratakv_ref.so")


def tool(*args, timeout=120):
    if not os.path.exists(TOOL):
        pytest.fail(f"{TOOL} is missing: run __graft_entry__.build() first")
    p = subprocess.run([TOOL, *map(str, args)], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                       timeout=timeout)
    assert p.returncode == 0, p.stderr
    return json.loads(p.stdout.strip().splitlines()[-1])


@pytest.fixture(scope="module")
def ref():
    if not os.path.exists(REF):
        pytest.skip("oracle/_ref is not built (the StrataKV sources are absent)")
    lib = ctypes.CDLL(REF)
    lib.ref_load_tensor.restype = ctypes.c_int
    return lib


def ref_load(lib, path, require_mapped=False, name=None, n=0):
    out = np.zeros(max(n, 1), np.float32)
    got_n = ctypes.c_size_t(0)
    count = ctypes.c_int(0)
    err = ctypes.create_string_buffer(1024)
    rc = lib.ref_load_tensor(str(path).encode(), int(require_mapped), name.encode() if name else None,
                             out.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(n), ctypes.byref(got_n),
                             ctypes.byref(count), err, 1024)
    if rc == 0:
        return {"ok": True, "count": count.value}, out[: got_n.value]
    return {"ok": False, "error": err.value.decode()}, None


def write_raw(path, header: bytes, payload: bytes = b"", length=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header) if length is None else length))
        f.write(header)
        f.write(payload)


def t(dtype, shape, a, b):
    return {"dtype": dtype, "shape": shape, "data_offsets": [a, b]}


def J(obj):
    return json.dumps(obj).encode()


# (header bytes, payload bytes) cases; the expected outcome is whatever the
# reference does.
CASES = {
    "ok_one": (J({"a": t("F32", [2], 0, 8)}), b"\0" * 8),
    "ok_empty": (b"{}", b""),
    "ok_meta": (J({"__metadata__": {"k": "v", "x": "y"}, "w": t("BF16", [2, 2], 0, 8)}), b"\0" * 8),
    "ok_ws": (b'{ "a" : { "dtype" : "F16" , "shape" : [ 1 ] , "data_offsets" : [ 0 , 2 ] } }  ', b"\0\0"),
    "ok_bfloat16_name": (J({"a": t("bfloat16", [1], 0, 2)}), b"\0\0"),
    "ok_zero_dim": (J({"a": t("F32", [0, 5], 0, 0), "b": t("F32", [1], 0, 4)}), b"\0" * 4),
    "ok_escapes": (b'{"a\\u00e9\\ud83d\\ude00\\n\\t\\/":' + J(t("F32", [1], 0, 4)) + b"}", b"\0" * 4),
    "leading_ws": (b' {"a":' + J(t("F32", [1], 0, 4)) + b"}", b"\0" * 4),
    "bad_utf8": (b'{"\xff":1}', b""),
    "trunc_utf8": (b'{"a":1}\xc3', b""),
    "bad_cont": (b'{"\xc3\x28":1}', b""),
    "overlong": (b'{"\xe0\x80\x80":1}', b""),
    "surrogate_utf8": (b'{"\xed\xa0\x80":1}', b""),
    "too_big_cp": (b'{"\xf4\x90\x80\x80":1}', b""),
    "missing_low": (b'{"\\ud83d":1}', b""),
    "invalid_low": (b'{"\\ud83d\\u0041":1}', b""),
    "unpaired_low": (b'{"\\ude00":1}', b""),
    "bad_hex": (b'{"\\u00zz":1}', b""),
    "trunc_hex": (b'{"\\u00', b""),
    "bad_escape": (b'{"\\x":1}', b""),
    "trunc_escape": (b'{"\\', b""),
    "control_char": (b'{"a\x01":1}', b""),
    "unterminated": (b'{"abc', b""),
    "no_colon": (b'{"a" ' + J(t("F32", [1], 0, 4)) + b"}", b"\0" * 4),
    "leading_zero": (b'{"a":{"dtype":"F32","shape":[01],"data_offsets":[0,4]}}', b"\0" * 4),
    "negative": (b'{"a":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}', b"\0" * 4),
    "overflow_int": (b'{"a":{"dtype":"F32","shape":[99999999999999999999999],"data_offsets":[0,4]}}', b""),
    "float_num": (b'{"a":{"dtype":"F32","shape":[1.5],"data_offsets":[0,4]}}', b""),
    "rank_65": (J({"a": t("F32", [1] * 65, 0, 4)}), b"\0" * 4),
    "rank_64": (J({"a": t("F32", [1] * 64, 0, 4)}), b"\0" * 4),
    "offsets_3": (J({"a": t("F32", [1], 0, 4) | {"data_offsets": [0, 4, 8]}}), b"\0" * 4),
    "offsets_1": (J({"a": t("F32", [1], 0, 4) | {"data_offsets": [4]}}), b"\0" * 4),
    "unknown_field": (b'{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4],"x":"y"}}', b"\0" * 4),
    "dup_field": (b'{"a":{"dtype":"F32","dtype":"F32","shape":[1],"data_offsets":[0,4]}}', b"\0" * 4),
    "missing_field": (b'{"a":{"dtype":"F32","shape":[1]}}', b"\0" * 4),
    "empty_tensor": (b'{"a":{}}', b""),
    "dup_key": (b'{"a":' + J(t("F32", [1], 0, 4)) + b',"a":' + J(t("F32", [1], 4, 8)) + b"}", b"\0" * 8),
    "dup_meta": (b'{"__metadata__":{"k":"v","k":"w"}}', b""),
    "meta_nonstring": (b'{"__metadata__":{"k":1}}', b""),
    "dtype_i32": (J({"a": t("I32", [1], 0, 4)}), b"\0" * 4),
    "shape_overflow": (J({"a": t("F32", [2**62, 4], 0, 4)}), b"\0" * 4),
    "zero_then_big": (J({"a": t("F32", [0, 2**62], 0, 0)}), b""),
    "range_backwards": (J({"a": t("F32", [1], 4, 0)}), b"\0" * 4),
    "range_past_end": (J({"a": t("F32", [1], 4, 8)}), b"\0" * 4),
    "range_size": (J({"a": t("F32", [2], 0, 4)}), b"\0" * 4),
    "hole": (J({"a": t("F32", [1], 0, 4), "b": t("F32", [1], 8, 12)}), b"\0" * 12),
    "overlap": (J({"a": t("F32", [2], 0, 8), "b": t("F32", [1], 4, 8)}), b"\0" * 8),
    "unreferenced": (J({"a": t("F32", [1], 0, 4)}), b"\0" * 8),
    "trailing": (J({"a": t("F32", [1], 0, 4)}) + b" x", b"\0" * 4),
    "trailing_comma": (b'{"a":' + J(t("F32", [1], 0, 4)) + b",}", b"\0" * 4),
    "not_object": (b'[1,2]', b""),
}


@pytest.mark.parametrize("case", sorted(CASES))
def test_header_cases_match_reference(tmp_path, ref, case):
    header, payload = CASES[case]
    path = tmp_path / f"{case}.safetensors"
    write_raw(path, header, payload)
    got = tool("load-host", path)
    want, _ = ref_load(ref, path)
    if want["ok"]:
        assert got["ok"], got
        assert got["count"] == want["count"]
    else:
        assert not got["ok"], (got, want)
        assert got["error"] == want["error"]


@pytest.mark.parametrize("length", [0, 1, 100 * 1024 * 1024 + 1, 10**6])
def test_header_length_rules(tmp_path, ref, length):
    path = tmp_path / "len.safetensors"
    write_raw(path, b"{}", b"", length=length)
    got, (want, _) = tool("load-host", path), ref_load(ref, path)
    assert not got["ok"] and not want["ok"]
    assert got["error"] == want["error"]


def test_file_errors(tmp_path, ref):
    small = tmp_path / "small.safetensors"
    small.write_bytes(b"\x02\0\0")
    for path in (small, tmp_path / "missing.safetensors"):
        got, (want, _) = tool("load-host", path), ref_load(ref, path)
        assert not got["ok"] and not want["ok"]
        assert got["error"] == want["error"]


def special_halves():
    bits = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0200, 0x0400, 0x3C00, 0xC000, 0x7BFF,
                     0x7C00, 0xFC00, 0x7E00, 0x7C01, 0xFE55], np.uint16)
    rng = np.random.default_rng(5)
    return np.concatenate([bits, rng.integers(0, 0x10000, 4000, dtype=np.uint16)])


def mixed_checkpoint(path, aligned_norm=True):
    """BF16, F16 and F32 tensors with special values; returns name -> expected FP32 bits."""
    rng = np.random.default_rng(11)
    halves = special_halves()
    bf = np.concatenate([halves, rng.integers(0, 0x10000, 1000, dtype=np.uint16)])
    f32 = np.concatenate([rng.standard_normal(999).astype(np.float32),
                          np.array([np.inf, -np.inf, -0.0, 1e-45], np.float32)]).view(np.uint32)
    norm = rng.standard_normal(16).astype(np.float32).view(np.uint32)
    tensors = [("w.bf16", "BF16", [len(bf)], bf.astype("<u2").tobytes(), (bf.astype(np.uint32) << 16)),
               ("w.f16", "F16", [len(halves)], halves.astype("<u2").tobytes(),
                halves.view(np.float16).astype(np.float32).view(np.uint32)),
               ("w.f32", "F32", [len(f32)], f32.astype("<u4").tobytes(), f32),
               ("model.norm.weight", "F32", [16], norm.astype("<u4").tobytes(), norm)]
    header, off, payload = {}, 0, b""
    for name, dt, shape, raw, _ in tensors:
        header[name] = t(dt, shape, off, off + len(raw))
        off += len(raw)
        payload += raw
    hj = json.dumps(header).encode()
    # pad so the payload starts 64-byte aligned in the file (norm aliasing)
    pad = (-(8 + len(hj)) % 64) if aligned_norm else ((-(8 + len(hj)) % 64) + 4)
    hj += b" " * pad
    write_raw(path, hj, payload)
    return {name: exp for name, _, _, _, exp in tensors}


def test_values_match_numpy_and_reference(tmp_path, ref):
    path = tmp_path / "mixed.safetensors"
    expected = mixed_checkpoint(path)
    for name, exp in expected.items():
        out = tmp_path / "dump.bin"
        got = tool("load-host", path, "--dump", name, out)
        assert got["ok"], got
        bits = np.fromfile(out, np.uint32)
        # NaN payloads included: compare bit patterns
        np.testing.assert_array_equal(bits, exp, err_msg=name)
        _, vals = ref_load(ref, path, name=name, n=len(exp))
        np.testing.assert_array_equal(vals.view(np.uint32), exp, err_msg=name)


def test_require_mapped_f32(tmp_path, ref):
    aligned = tmp_path / "aligned.safetensors"
    mixed_checkpoint(aligned, aligned_norm=True)
    for path in (aligned,):
        got, (want, _) = tool("load-host", path, "--require-mapped"), ref_load(ref, path, True)
        assert got["ok"] == want["ok"]
        if not want["ok"]:
            assert got["error"] == want["error"]
    # Only a 64-byte-aligned F32 norm tensor can be mapped: a lone norm passes
    # when aligned and fails when the header shifts it by 4 bytes.
    for shift, name in ((0, "ok.safetensors"), (4, "shifted.safetensors")):
        norm = np.arange(16, dtype=np.float32).tobytes()
        hj = json.dumps({"model.norm.weight": t("F32", [16], 0, 64)}).encode()
        hj += b" " * ((-(8 + len(hj)) % 64) + shift)
        path = tmp_path / name
        write_raw(path, hj, norm)
        got, (want, _) = tool("load-host", path, "--require-mapped"), ref_load(ref, path, True)
        assert got["ok"] == want["ok"] == (shift == 0), (got, want)
        if not want["ok"]:
            assert got["error"] == want["error"]


@pytest.mark.parametrize("shape", [(1, 1), (37, 5), (64, 64), (65, 130), (300, 7)])
def test_linear_transpose_matches_reference(tmp_path, ref, shape):
    out_f, in_f = shape
    rng = np.random.default_rng(out_f * 1000 + in_f)
    src = rng.standard_normal((out_f, in_f)).astype(np.float32)
    src.tofile(tmp_path / "src.bin")
    p = subprocess.run([TOOL, "transpose", tmp_path / "src.bin", str(out_f), str(in_f), tmp_path / "dst.bin"],
                       capture_output=True, text=True)
    assert p.returncode == 0, p.stderr
    got = np.fromfile(tmp_path / "dst.bin", np.uint16).reshape(in_f, out_f)
    want = np.zeros(out_f * in_f, np.uint16)
    assert ref.ref_linear_bf16_transposed(src.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(out_f),
                                          ctypes.c_size_t(in_f), want.ctypes.data_as(ctypes.c_void_p)) == 0
    np.testing.assert_array_equal(got, want.reshape(in_f, out_f))
    # and the rule itself: the upper 16 bits of each FP32 value, transposed
    np.testing.assert_array_equal(got, (src.view(np.uint32) >> 16).astype(np.uint16).T)


def test_generated_checkpoint_loads(tmp_path, ref):
    """The test checkpoint writer produces files both loaders accept."""
    import sys
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import make_checkpoint

    path, _ = make_checkpoint.ensure("mini", str(tmp_path))
    got, (want, _) = tool("load-host", path), ref_load(ref, path)
    assert got["ok"] and want["ok"] and got["count"] == want["count"] == 2 + 9 * 2 + 1

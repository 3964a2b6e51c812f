"""stratakv_amd -- MI355X (gfx950) paged KV-cache hot path.

Python bindings (ctypes) over ``libstratakv_amd.so``, whose C ABI is declared
in ``include/stratakv_amd.h``.  The library holds hand-written HIP kernels for
the KV append and paged decode attention; there is no CPU fallback: every
entry point raises if the library or a GPU is missing.

bf16 data crosses this boundary as ``numpy.uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libstratakv_amd.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "stratakv_amd.h")
GEMM_LIB_PATH = os.path.join(_HERE, "libstratakv_amd_gemm.so")
GEMM_HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "stratakv_amd_gemm.h")

SKV_OK = 0
SKV_ERR_INVALID_ARGUMENT = 1
SKV_ERR_HIP = 2
SKV_ERR_WORKSPACE = 3
SKV_ERR_UNSUPPORTED = 4

DTYPE_BF16 = 0
DTYPE_FP32 = 1
DTYPE_F16 = 2

FLAG_NONFINITE_LOGITS = 1
FLAG_BAD_TOKEN = 2
FLAG_NONFINITE_SCALED = 4
FLAG_BAD_DISTRIBUTION = 8


class SkvError(RuntimeError):
    """A non-zero status from the C ABI (runtime_error in the reference)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class SkvInvalidArgument(SkvError, ValueError):
    """SKV_ERR_INVALID_ARGUMENT (std::invalid_argument in the reference)."""


_c = ctypes
_vp, _i32, _i64, _u64, _sz, _f32 = _c.c_void_p, _c.c_int, _c.c_int64, _c.c_uint64, _c.c_size_t, _c.c_float
_PROTOS = {
    "skv_last_error": (_c.c_char_p, []),
    "skv_abi_version": (_i32, []),
    "skv_device_count": (_i32, [_c.POINTER(_i32)]),
    "skv_set_device": (_i32, [_i32]),
    "skv_malloc": (_i32, [_c.POINTER(_vp), _sz]),
    "skv_free": (_i32, [_vp]),
    "skv_memcpy_h2d": (_i32, [_vp, _vp, _sz, _vp]),
    "skv_memcpy_d2h": (_i32, [_vp, _vp, _sz, _vp]),
    "skv_memcpy_d2d": (_i32, [_vp, _vp, _sz, _vp]),
    "skv_memset_d8": (_i32, [_vp, _i32, _sz, _vp]),
    "skv_stream_create": (_i32, [_c.POINTER(_vp)]),
    "skv_stream_destroy": (_i32, [_vp]),
    "skv_stream_synchronize": (_i32, [_vp]),
    "skv_device_synchronize": (_i32, []),
    "skv_event_create": (_i32, [_c.POINTER(_vp)]),
    "skv_event_destroy": (_i32, [_vp]),
    "skv_event_record": (_i32, [_vp, _vp]),
    "skv_event_synchronize": (_i32, [_vp]),
    "skv_event_elapsed_ms": (_i32, [_c.POINTER(_f32), _vp, _vp]),
    "skv_host_alloc": (_i32, [_c.POINTER(_vp), _sz]),
    "skv_host_free": (_i32, [_vp]),
    "skv_memcpy_h2d_async": (_i32, [_vp, _vp, _sz, _vp]),
    "skv_memcpy_d2h_async": (_i32, [_vp, _vp, _sz, _vp]),
    "skv_event_query": (_i32, [_vp, _c.POINTER(_i32)]),
    "skv_scatter_i32": (_i32, [_vp, _vp, _i32, _vp]),
    "skv_fill_normal_bf16": (_i32, [_vp, _sz, _u64, _u64, _vp]),
    "skv_fill_normal_scaled_bf16": (_i32, [_vp, _sz, _u64, _u64, _f32, _vp]),
    "skv_fill_u16": (_i32, [_vp, _sz, _c.c_uint16, _vp]),
    "skv_kv_append": (_i32, [_vp, _vp, _i32, _vp, _vp, _i64, _vp, _i32, _vp, _vp,
                             _i32, _i32, _i32, _i32, _i32, _vp]),
    "skv_kv_append_token": (_i32, [_vp, _vp, _i32, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32,
                                   _i32, _vp]),
    "skv_paged_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "skv_paged_decode": (_i32, [_vp, _i32, _vp, _vp, _i64, _vp, _i32, _vp, _i32, _i32, _i32,
                                _i32, _i32, _f32, _vp, _vp, _sz, _vp]),
    "skv_paged_decode_append": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _i64, _vp, _i32, _vp,
                                       _i32, _i32, _i32, _i32, _i32, _f32, _vp, _vp, _sz, _vp]),
    "skv_paged_decode_append_noalloc": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _vp, _i64, _vp, _i32,
                                               _vp, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _vp]),
    "skv_paged_attention_decode_append": (_i32, [_vp, _vp, _vp, _i32, _vp, _vp, _i64, _vp, _vp,
                                                 _i32, _i32, _i32, _i32, _i32, _f32, _vp, _sz,
                                                 _vp]),
    "skv_paged_prefill": (_i32, [_vp, _i32, _vp, _vp, _i64, _vp, _i32, _vp, _vp, _i32, _i32, _i32,
                                 _i32, _i32, _i32, _f32, _vp, _vp]),
    "skv_paged_attention_decode_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "skv_paged_attention_decode": (_i32, [_vp, _vp, _vp, _i64, _vp, _vp, _i32, _i32, _i32, _i32,
                                          _i32, _f32, _vp, _sz, _vp]),
    "skv_gather_blocks": (_i32, [_vp, _i64, _vp, _i32, _i64, _vp, _vp]),
    "skv_copy_chunks": (_i32, [_vp, _vp, _i32, _sz, _vp]),
    "skv_paged_block_checksum": (_i32, [_vp, _vp, _i64, _vp, _i32, _vp, _i32, _i32, _i32, _i32, _i32,
                                        _vp, _vp]),
    "skv_stream_read_checksum": (_i32, [_vp, _i64, _vp, _vp]),
    "skv_graph_begin_capture": (_i32, [_vp]),
    "skv_graph_end_capture": (_i32, [_vp, _c.POINTER(_vp)]),
    "skv_graph_abort_capture": (_i32, [_vp]),
    "skv_graph_launch": (_i32, [_vp, _vp]),
    "skv_graph_destroy": (_i32, [_vp]),
    "skv_rmsnorm_f32": (_i32, [_vp, _vp, _vp, _i32, _i32, _f32, _vp]),
    "skv_linear_f32": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp, _vp]),
    "skv_rope_f32": (_i32, [_vp, _i32, _i32, _i32, _vp]),
    "skv_swiglu_f32": (_i32, [_vp, _vp, _i32, _vp]),
    "skv_add_f32": (_i32, [_vp, _vp, _i32, _vp]),
    "skv_fused_qkv_f32": (_i32, [_vp, _vp, _f32, _vp, _vp, _vp, _i32, _i64, _c.POINTER(_c.c_int64),
                                 _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp]),
    "skv_fused_qkv_at_f32": (_i32, [_vp, _vp, _f32, _vp, _vp, _vp, _i32, _i64, _c.POINTER(_c.c_int64),
                                    _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp, _vp, _i32, _vp, _vp, _vp,
                                    _vp]),
    "skv_rope_cos_sin": (_i32, [_i32, _i32, _i32, _vp]),
    "skv_fused_gate_up_swiglu_f32": (_i32, [_vp, _vp, _f32, _vp, _vp, _i32, _i64, _i64, _i64, _vp,
                                            _vp, _i32, _i32, _vp, _vp]),
    "skv_linear_residual_f32": (_i32, [_vp, _vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp, _vp, _vp]),
    "skv_fused_qkv_rows_f32": (_i32, [_vp, _i32, _vp, _f32, _vp, _vp, _vp, _i32, _i64,
                                      _c.POINTER(_c.c_int64), _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                      _i32, _vp, _vp, _vp, _vp, _vp]),
    "skv_fused_gate_up_swiglu_rows_f32": (_i32, [_vp, _i32, _vp, _f32, _vp, _vp, _i32, _i64, _i64,
                                                 _i64, _vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "skv_linear_residual_rows_f32": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp,
                                            _vp, _vp]),
    "skv_fused_qkv_mm_f32": (_i32, [_vp, _i32, _vp, _f32, _vp, _vp, _vp, _i32, _i64,
                                    _c.POINTER(_c.c_int64), _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                    _i32, _vp, _vp, _vp, _vp, _vp]),
    "skv_fused_gate_up_swiglu_mm_f32": (_i32, [_vp, _i32, _vp, _f32, _vp, _vp, _i32, _i64, _i64,
                                               _i64, _vp, _vp, _i32, _i32, _vp, _vp, _vp]),
    "skv_linear_residual_mm_f32": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp,
                                          _vp, _vp]),
    "skv_rope_rows_f32": (_i32, [_vp, _i32, _i32, _i32, _i32, _vp]),
    "skv_write_i32": (_i32, [_vp, _c.POINTER(_c.c_int32), _i32, _vp]),
    "skv_convert_to_bf16": (_i32, [_vp, _i32, _sz, _vp, _vp, _vp]),
    "skv_convert_to_f32": (_i32, [_vp, _i32, _sz, _vp, _vp, _vp]),
    "skv_check_finite": (_i32, [_vp, _i32, _sz, _vp, _vp]),
    "skv_embedding_f32": (_i32, [_vp, _i32, _i32, _i32, _vp, _i32, _vp, _vp, _vp]),
    "skv_embedding_rows_f32": (_i32, [_vp, _i32, _i32, _i32, _vp, _i32, _i32, _vp, _vp, _vp]),
    "skv_argmax_f32": (_i32, [_vp, _i32, _vp, _i32, _vp, _vp]),
    "skv_embedding_at_f32": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp]),
    "skv_argmax_at_f32": (_i32, [_vp, _i32, _vp, _vp, _vp, _vp, _vp]),
    "skv_sample_f32": (_i32, [_vp, _i32, _f32, _i32, _f32, _c.c_double, _vp, _i32, _vp, _vp]),
}

# libstratakv_amd_gemm.so (include/stratakv_amd_gemm.h): the hipBLASLt
# projections of long prompt chunks, the only library linking hipBLASLt.
_GEMM_PROTOS = {
    "skv_prompt_gemm_workspace_bytes": (_sz, [_i32, _i32, _i32]),
    "skv_fused_qkv_gemm_f32": (_i32, [_vp, _i32, _vp, _f32, _vp, _vp, _vp, _i32, _i64,
                                      _c.POINTER(_c.c_int64), _vp, _vp, _vp, _i32, _i32, _i32, _i32,
                                      _i32, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "skv_fused_gate_up_swiglu_gemm_f32": (_i32, [_vp, _i32, _vp, _f32, _vp, _vp, _i32, _i64, _i64,
                                                 _i64, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "skv_linear_residual_gemm_f32": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i32, _i32, _vp, _vp,
                                            _vp, _vp, _sz, _vp]),
    "skv_ffn_swiglu_gemm_f32": (_i32, [_vp, _i32, _vp, _f32, _vp, _vp, _vp, _i32, _i64, _i64, _i64, _i64,
                                       _vp, _vp, _vp, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
}

_lib = None
_gemm_lib = None


def header_symbols(path: str = HEADER_PATH) -> list[str]:
    """Names of every function declared in the C ABI header."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(skv_\w+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    """Load the native library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run __graft_entry__.build() first")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _PROTOS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def gemm_lib() -> ctypes.CDLL:
    """Load libstratakv_amd_gemm.so (after libstratakv_amd.so, which it
    depends on and which holds skv_last_error; raises if either is missing)."""
    global _gemm_lib
    if _gemm_lib is None:
        lib()
        path = os.path.join(os.path.dirname(LIB_PATH), os.path.basename(GEMM_LIB_PATH))
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing: run __graft_entry__.build() first")
        handle = ctypes.CDLL(path)
        for name, (res, args) in _GEMM_PROTOS.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _gemm_lib = handle
    return _gemm_lib


def _check(rc: int) -> None:
    if rc != SKV_OK:
        msg = lib().skv_last_error().decode(errors="replace")
        if rc == SKV_ERR_INVALID_ARGUMENT:
            raise SkvInvalidArgument(rc, msg)
        raise SkvError(rc, msg)


def device_count() -> int:
    n = _c.c_int(0)
    _check(lib().skv_device_count(_c.byref(n)))
    return n.value


def require_gpu() -> None:
    if device_count() < 1:
        raise SkvError(SKV_ERR_HIP, "no HIP device is visible")


def synchronize() -> None:
    _check(lib().skv_device_synchronize())


class DeviceBuffer:
    """Owning device allocation (hipMalloc through the C ABI)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _c.c_void_p()
        _check(lib().skv_malloc(_c.byref(p), self.nbytes))
        self.ptr = p.value or 0

    @classmethod
    def from_numpy(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(max(arr.nbytes, 1))
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= self.nbytes, "upload past the end of the buffer"
        if arr.nbytes:
            _check(lib().skv_memcpy_h2d(self.ptr + offset, arr.ctypes.data, arr.nbytes, None))

    def download(self, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert offset + out.nbytes <= self.nbytes, "download past the end of the buffer"
        if out.nbytes:
            _check(lib().skv_memcpy_d2h(out.ctypes.data, self.ptr + offset, out.nbytes, None))
        return out

    def fill_u16(self, value: int, count: int | None = None, stream=None) -> None:
        n = self.nbytes // 2 if count is None else count
        _check(lib().skv_fill_u16(self.ptr, n, value, stream))

    def free(self) -> None:
        if self.ptr:
            _check(lib().skv_free(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.skv_free(self.ptr)
        except Exception:
            pass


def _ptr(x) -> int | None:
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr
    return int(x)


def fill_normal_bf16(dst, count: int, seed: int, first_index: int = 0, stream=None) -> None:
    _check(lib().skv_fill_normal_bf16(_ptr(dst), count, seed, first_index, stream))


def kv_append(k_new, v_new, src_dtype: int, k_pool, v_pool, total_blocks: int, block_tables,
              max_blocks_per_seq: int, positions, num_seqs: int, tokens_per_seq: int,
              num_kv_heads: int, head_dim: int, block_size: int, token_offsets=None,
              stream=None) -> None:
    _check(lib().skv_kv_append(_ptr(k_new), _ptr(v_new), src_dtype, _ptr(k_pool), _ptr(v_pool),
                               total_blocks, _ptr(block_tables), max_blocks_per_seq,
                               _ptr(positions), _ptr(token_offsets), num_seqs, tokens_per_seq,
                               num_kv_heads, head_dim, block_size, stream))


def decode_workspace_bytes(num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int) -> int:
    return int(lib().skv_paged_decode_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim))


def decode_workspace(num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                     stream=None) -> tuple["DeviceBuffer", int]:
    """A decode workspace for these arguments; returns (buffer, size in bytes)."""
    nbytes = decode_workspace_bytes(num_seqs, num_q_heads, num_kv_heads, head_dim)
    return DeviceBuffer(nbytes), nbytes


def single_decode_workspace(num_q_heads: int, num_kv_heads: int, head_dim: int,
                            stream=None) -> tuple["DeviceBuffer", int]:
    """The same for the single-sequence entry points (skv_paged_attention_decode*)."""
    nbytes = int(lib().skv_paged_attention_decode_workspace_bytes(num_q_heads, num_kv_heads, head_dim))
    return DeviceBuffer(nbytes), nbytes


def paged_decode(q, q_dtype: int, k_pool, v_pool, total_blocks: int, block_tables,
                 max_blocks_per_seq: int, context_lens, num_seqs: int, num_q_heads: int,
                 num_kv_heads: int, head_dim: int, block_size: int, scale: float, out,
                 workspace, workspace_bytes: int, stream=None) -> None:
    _check(lib().skv_paged_decode(_ptr(q), q_dtype, _ptr(k_pool), _ptr(v_pool), total_blocks,
                                  _ptr(block_tables), max_blocks_per_seq, _ptr(context_lens),
                                  num_seqs, num_q_heads, num_kv_heads, head_dim, block_size,
                                  scale, _ptr(out), _ptr(workspace), workspace_bytes, stream))


def paged_decode_append(q, q_dtype: int, k_new, v_new, kv_dtype: int, k_pool, v_pool,
                        total_blocks: int, block_tables, max_blocks_per_seq: int, context_lens,
                        num_seqs: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                        block_size: int, scale: float, out, workspace, workspace_bytes: int,
                        stream=None) -> None:
    """Append each sequence's new token at context_lens[b] - 1, then decode (one launch)."""
    _check(lib().skv_paged_decode_append(_ptr(q), q_dtype, _ptr(k_new), _ptr(v_new), kv_dtype,
                                         _ptr(k_pool), _ptr(v_pool), total_blocks,
                                         _ptr(block_tables), max_blocks_per_seq,
                                         _ptr(context_lens), num_seqs, num_q_heads, num_kv_heads,
                                         head_dim, block_size, scale, _ptr(out), _ptr(workspace),
                                         workspace_bytes, stream))


def paged_attention_decode_append(query, key_row, value_row, kv_dtype: int, key_cache,
                                  value_cache, total_blocks: int, block_table, output,
                                  context_len: int, block_size: int, num_q_heads: int,
                                  num_kv_heads: int, head_dim: int, scale: float, workspace,
                                  workspace_bytes: int, stream=None) -> None:
    _check(lib().skv_paged_attention_decode_append(
        _ptr(query), _ptr(key_row), _ptr(value_row), kv_dtype, _ptr(key_cache), _ptr(value_cache),
        total_blocks, _ptr(block_table), _ptr(output), context_len, block_size, num_q_heads,
        num_kv_heads, head_dim, scale, _ptr(workspace), workspace_bytes, stream))


def paged_prefill(q, q_dtype: int, k_pool, v_pool, total_blocks: int, block_tables,
                  max_blocks_per_seq: int, seq_offsets, context_lens, num_seqs: int,
                  num_tokens: int, num_q_heads: int, num_kv_heads: int, head_dim: int,
                  block_size: int, scale: float, out, stream=None) -> None:
    """Causal prefill attention of each sequence's chunk (rows seq_offsets[b]..)."""
    _check(lib().skv_paged_prefill(_ptr(q), q_dtype, _ptr(k_pool), _ptr(v_pool), total_blocks,
                                   _ptr(block_tables), max_blocks_per_seq, _ptr(seq_offsets),
                                   _ptr(context_lens), num_seqs, num_tokens, num_q_heads,
                                   num_kv_heads, head_dim, block_size, scale, _ptr(out), stream))


def paged_attention_decode(query, key_cache, value_cache, total_blocks: int, block_table, output,
                           context_len: int, block_size: int, num_q_heads: int, num_kv_heads: int,
                           head_dim: int, scale: float, workspace, workspace_bytes: int,
                           stream=None) -> None:
    _check(lib().skv_paged_attention_decode(_ptr(query), _ptr(key_cache), _ptr(value_cache),
                                            total_blocks, _ptr(block_table), _ptr(output),
                                            context_len, block_size, num_q_heads, num_kv_heads,
                                            head_dim, scale, _ptr(workspace), workspace_bytes,
                                            stream))


def gather_blocks(pool, total_blocks: int, table, num_blocks: int, block_elems: int, dst,
                  stream=None) -> None:
    _check(lib().skv_gather_blocks(_ptr(pool), total_blocks, _ptr(table), num_blocks, block_elems,
                                   _ptr(dst), stream))


def stream_read_checksum(data, nbytes: int, checksum, stream=None) -> None:
    """skv_stream_read_checksum: read `nbytes` of `data` once (plain streaming reads) and
    write the wrapping 32-bit sum of its 32-bit words to `checksum` (device uint32)."""
    _check(lib().skv_stream_read_checksum(_ptr(data), nbytes, _ptr(checksum), stream))


def paged_block_checksum(k_pool, v_pool, total_blocks: int, block_tables, max_blocks_per_seq: int,
                         context_lens, num_seqs: int, num_q_heads: int, num_kv_heads: int,
                         head_dim: int, block_size: int, checksums, stream=None) -> None:
    _check(lib().skv_paged_block_checksum(_ptr(k_pool), _ptr(v_pool), total_blocks, _ptr(block_tables),
                                          max_blocks_per_seq, _ptr(context_lens), num_seqs, num_q_heads,
                                          num_kv_heads, head_dim, block_size, _ptr(checksums), stream))


def convert_to_bf16(src, src_dtype: int, count: int, dst, nonfinite=None, stream=None) -> None:
    _check(lib().skv_convert_to_bf16(_ptr(src), src_dtype, count, _ptr(dst), _ptr(nonfinite), stream))


def convert_to_f32(src, src_dtype: int, count: int, dst, nonfinite=None, stream=None) -> None:
    _check(lib().skv_convert_to_f32(_ptr(src), src_dtype, count, _ptr(dst), _ptr(nonfinite), stream))


def check_finite(src, src_dtype: int, count: int, nonfinite, stream=None) -> None:
    _check(lib().skv_check_finite(_ptr(src), src_dtype, count, _ptr(nonfinite), stream))


def embedding(table, table_dtype: int, vocab: int, hidden: int, token_ids, index: int, out, flags=None,
              stream=None) -> None:
    _check(lib().skv_embedding_f32(_ptr(table), table_dtype, vocab, hidden, _ptr(token_ids), index, _ptr(out),
                                   _ptr(flags), stream))


def embedding_rows(table, table_dtype: int, vocab: int, hidden: int, token_ids, first_index: int, rows: int, out,
                   flags=None, stream=None) -> None:
    _check(lib().skv_embedding_rows_f32(_ptr(table), table_dtype, vocab, hidden, _ptr(token_ids), first_index, rows,
                                        _ptr(out), _ptr(flags), stream))


def argmax(logits, n: int, token_ids, index: int, flags=None, stream=None) -> None:
    _check(lib().skv_argmax_f32(_ptr(logits), n, _ptr(token_ids), index, _ptr(flags), stream))


def sample(logits, n: int, temperature: float, top_k: int, top_p: float, uniform: float, token_ids,
           index: int, flags=None, stream=None) -> None:
    """token_ids[index] = the reference Sampler's choice for the draw `uniform`."""
    _check(lib().skv_sample_f32(_ptr(logits), n, temperature, top_k, top_p, uniform, _ptr(token_ids), index,
                                _ptr(flags), stream))


class Event:
    def __init__(self):
        p = _c.c_void_p()
        _check(lib().skv_event_create(_c.byref(p)))
        self.ptr = p.value

    def record(self, stream=None) -> None:
        _check(lib().skv_event_record(self.ptr, stream))

    def elapsed_ms(self, later: "Event") -> float:
        ms = _c.c_float()
        _check(lib().skv_event_elapsed_ms(_c.byref(ms), self.ptr, later.ptr))
        return ms.value

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.skv_event_destroy(self.ptr)
        except Exception:
            pass


class Stream:
    """A non-blocking HIP stream at the default priority."""

    def __init__(self):
        p = _c.c_void_p()
        _check(lib().skv_stream_create(_c.byref(p)))
        self.ptr = p.value

    @property
    def handle(self):
        return self.ptr

    def synchronize(self) -> None:
        _check(lib().skv_stream_synchronize(self.ptr))

    def __del__(self):
        try:
            if self.ptr and _lib is not None:
                _lib.skv_stream_destroy(self.ptr)
        except Exception:
            pass


__all__ = [
    "LIB_PATH", "HEADER_PATH", "SkvError", "SkvInvalidArgument", "DTYPE_BF16", "DTYPE_FP32",
    "header_symbols", "lib", "device_count", "require_gpu", "synchronize", "DeviceBuffer",
    "fill_normal_bf16", "kv_append", "decode_workspace_bytes",
    "decode_workspace", "single_decode_workspace", "paged_decode",
    "paged_attention_decode", "gather_blocks", "paged_block_checksum", "stream_read_checksum", "Event", "Stream", "convert_to_bf16", "convert_to_f32",
    "check_finite", "embedding", "embedding_rows", "argmax", "sample",
]

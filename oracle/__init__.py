"""CPU oracle for the paged-KV hot path -- TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``oracle/liboracle.so`` (the C restatement of the
reference, ``oracle/oracle.c``) and, when it was built, over
``oracle/_ref/libstratakv_ref.so`` (the reference's own CPU classes compiled
from its sources, ``oracle/Makefile`` target ``ref``).  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg use this
module, as the checker or the timed CPU baseline; the product never does.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(_HERE, "liboracle.so")
REF_LIB = os.path.join(_HERE, "_ref", "libstratakv_ref.so")

OP_ALLOC_SEQ, OP_APPEND, OP_FREE_SEQ = 1, 2, 3
ST_OK, ST_OOM, ST_UNKNOWN, ST_EXISTS = 0, 1, 2, 3

_c = ctypes
_vp, _i32, _i64, _sz, _f32, _f64 = _c.c_void_p, _c.c_int, _c.c_int64, _c.c_size_t, _c.c_float, _c.c_double
_ATTN = [_vp, _vp, _vp, _i64, _vp, _i32, _vp, _i32, _i32, _i32, _i32, _i32]
_PROTOS = {
    "oracle_bf16_to_f32": (_f32, [_c.c_uint16]),
    "oracle_f32_to_bf16_rne": (_c.c_uint16, [_f32]),
    "oracle_f32_to_bf16_trunc": (_c.c_uint16, [_f32]),
    "oracle_bf16_to_f32_n": (None, [_vp, _vp, _sz]),
    "oracle_f32_to_bf16_rne_n": (None, [_vp, _vp, _sz]),
    "oracle_pool_trace": (_i32, [_i32, _i32, _vp, _i32, _i32, _vp, _vp, _vp, _i32, _vp]),
    "oracle_kv_append": (None, [_vp, _vp, _i32, _vp, _vp, _i64, _vp, _i32, _vp, _vp, _i32, _i32,
                                _i32, _i32, _i32]),
    "oracle_paged_decode_f32": (_i32, _ATTN + [_f32, _vp]),
    "oracle_paged_decode_f64": (_i32, _ATTN + [_f64, _vp]),
    "oracle_paged_decode_f32_mt": (_i32, _ATTN + [_f32, _vp, _i32]),
    "oracle_paged_decode_f32_fp32pool": (_i32, _ATTN + [_f32, _vp]),
}
_REF_PROTOS = {
    "ref_pool_trace": (_i32, [_i32, _i32, _vp, _i32, _i32, _vp, _vp, _vp, _i32, _vp]),
    "ref_bf16_rne_n": (_i32, [_vp, _vp, _sz]),
    "ref_attention_trace": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp,
                                   _vp, _vp]),
    "ref_prefill_trace": (_i32, [_i32, _i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp,
                                 _vp, _vp]),
}

_lib = None
_ref = None


def _load(path, protos):
    h = ctypes.CDLL(path)
    for name, (res, args) in protos.items():
        fn = getattr(h, name)
        fn.restype = res
        fn.argtypes = args
    return h


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_LIB):
            raise ImportError(f"{ORACLE_LIB} is missing: run __graft_entry__.build() first")
        _lib = _load(ORACLE_LIB, _PROTOS)
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_LIB)


def ref():
    global _ref
    if _ref is None:
        _ref = _load(REF_LIB, _REF_PROTOS)
    return _ref


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


# ---- bf16 ---------------------------------------------------------------------
def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_bf16_to_f32_n(_p(h), _p(out), h.size)
    return out


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().oracle_f32_to_bf16_rne_n(_p(x), _p(out), x.size)
    return out


# ---- pool trace ----------------------------------------------------------------
def pool_trace(total: int, block_size: int, ops, max_seqs: int, max_blocks_out: int,
               use_reference: bool = False):
    """Replay (opcode, seq_id) pairs; returns (results, lens, blocks, drain)."""
    ops = np.ascontiguousarray(np.asarray(ops, dtype=np.int32).reshape(-1, 2))
    n = ops.shape[0]
    results = np.zeros((n, 2), np.int32)
    lens = np.zeros(max_seqs, np.int32)
    blocks = np.zeros((max_seqs, max_blocks_out), np.int32)
    drain = np.zeros(total + n + 1, np.int32)
    fn = ref().ref_pool_trace if use_reference else lib().oracle_pool_trace
    k = fn(total, block_size, _p(ops), n, max_seqs, _p(results), _p(lens), _p(blocks),
           max_blocks_out, _p(drain))
    return results, lens, blocks, drain[:k].copy()


# ---- append ----------------------------------------------------------------------
def kv_append(k_new, v_new, k_pool, v_pool, tables, positions, num_seqs, tokens_per_seq,
              num_kv_heads, head_dim, block_size, offsets=None):
    """In-place scatter into uint16 pools; k_new/v_new are uint16 (bf16) or float32."""
    src_fp32 = 1 if k_new.dtype == np.float32 else 0
    tables = np.ascontiguousarray(tables, np.int32)
    positions = np.ascontiguousarray(positions, np.int32)
    offsets = None if offsets is None else np.ascontiguousarray(offsets, np.int32)
    total_blocks = k_pool.shape[0]
    lib().oracle_kv_append(_p(np.ascontiguousarray(k_new)), _p(np.ascontiguousarray(v_new)),
                           src_fp32, _p(k_pool), _p(v_pool), total_blocks, _p(tables),
                           tables.shape[1], _p(positions), _p(offsets), num_seqs, tokens_per_seq,
                           num_kv_heads, head_dim, block_size)


# ---- attention ---------------------------------------------------------------------
def paged_decode(q, k_pool, v_pool, tables, lens, num_kv_heads, block_size, scale,
                 precision: str = "f32", threads: int = 1):
    """q [B,Hq,hd] float32; pools [total, bs, Hkv, hd] uint16 (bf16) or float32.

    precision: "f32" (the reference's loops), "f64" (double-precision truth).
    """
    q = np.ascontiguousarray(q, np.float32)
    B, Hq, hd = q.shape
    tables = np.ascontiguousarray(tables, np.int32)
    lens = np.ascontiguousarray(lens, np.int32)
    k_pool = np.ascontiguousarray(k_pool)
    v_pool = np.ascontiguousarray(v_pool)
    total = k_pool.shape[0]
    args = [_p(q), _p(k_pool), _p(v_pool), total, _p(tables), tables.shape[1], _p(lens), B, Hq,
            num_kv_heads, hd, block_size]
    if precision == "f64":
        out = np.zeros((B, Hq, hd), np.float64)
        rc = lib().oracle_paged_decode_f64(*args, float(scale), _p(out))
    elif k_pool.dtype == np.float32:
        out = np.zeros((B, Hq, hd), np.float32)
        rc = lib().oracle_paged_decode_f32_fp32pool(*args, float(scale), _p(out))
    else:
        out = np.zeros((B, Hq, hd), np.float32)
        rc = lib().oracle_paged_decode_f32_mt(*args, float(scale), _p(out), int(threads))
    if rc != 0:
        raise RuntimeError(f"oracle paged decode failed with status {rc}")
    return out


def prefill_positions(seq_offsets, lens):
    """Per query token of a prefill batch: (sequence, position).  Sequence b
    owns tokens seq_offsets[b] .. seq_offsets[b+1]-1, the last n_b positions of
    its lens[b]-token context."""
    seq_offsets = np.asarray(seq_offsets, np.int64)
    lens = np.asarray(lens, np.int64)
    seqs, pos = [], []
    for b in range(len(lens)):
        n = int(seq_offsets[b + 1] - seq_offsets[b])
        seqs += [b] * n
        pos += list(range(int(lens[b]) - n, int(lens[b])))
    return np.array(seqs, np.int64), np.array(pos, np.int64)


def paged_prefill(q, k_pool, v_pool, tables, seq_offsets, lens, num_kv_heads, block_size, scale,
                  precision: str = "f32", threads: int = 1):
    """Causal chunked-prefill attention (src/layers/attention.cpp:263-337 per
    token): query token i of sequence b sits at position p = lens[b] - n_b + i
    and attends to positions 0..p of its sequence.  q [N, Hq, hd] float32 with
    N = seq_offsets[-1]; returns [N, Hq, hd].  Each token is the reference's
    decode loop at context p + 1, so this runs paged_decode with one row per
    token (its sequence's table, length p + 1); tokens with p < 0 give zeros."""
    seqs, pos = prefill_positions(seq_offsets, lens)
    tables = np.ascontiguousarray(tables, np.int32)
    tok_tables = np.ascontiguousarray(tables[seqs]) if len(seqs) else tables[:0]
    tok_lens = np.maximum(pos + 1, 0).astype(np.int32)
    q = np.ascontiguousarray(q, np.float32)
    if len(seqs) == 0:
        return np.zeros_like(q)
    return paged_decode(q, k_pool, v_pool, tok_tables, tok_lens, num_kv_heads, block_size, scale,
                        precision=precision, threads=threads)


def ref_prefill_trace(hidden: int, heads: int, kv_heads: int, total_blocks: int, block_size: int,
                      x: np.ndarray, chunk_lens):
    """Run tokens x [T, hidden] through the reference's PagedAttention::forward
    in chunks (sum(chunk_lens) == T)."""
    x = np.ascontiguousarray(x, np.float32)
    chunks = np.ascontiguousarray(chunk_lens, np.int32)
    T = x.shape[0]
    assert int(chunks.sum()) == T
    hd = hidden // heads
    kv_dim = kv_heads * hd
    out = np.zeros((T, hidden), np.float32)
    q = np.zeros((T, hidden), np.float32)
    k = np.zeros((T, kv_dim), np.float32)
    v = np.zeros((T, kv_dim), np.float32)
    table = np.zeros(total_blocks, np.int32)
    nb = ctypes.c_int(0)
    rc = ref().ref_prefill_trace(hidden, heads, kv_heads, total_blocks, block_size, len(chunks),
                                 _p(chunks), _p(x), _p(out), _p(q), _p(k), _p(v), _p(table),
                                 ctypes.byref(nb))
    if rc != 0:
        raise RuntimeError("reference prefill trace failed")
    return out, q, k, v, table[: nb.value].copy()


def ref_attention_trace(hidden: int, heads: int, kv_heads: int, total_blocks: int, block_size: int,
                        x: np.ndarray):
    """Run tokens x [T, hidden] through the reference's PagedAttention::forward."""
    x = np.ascontiguousarray(x, np.float32)
    T = x.shape[0]
    hd = hidden // heads
    kv_dim = kv_heads * hd
    out = np.zeros((T, hidden), np.float32)
    q = np.zeros((T, hidden), np.float32)
    k = np.zeros((T, kv_dim), np.float32)
    v = np.zeros((T, kv_dim), np.float32)
    table = np.zeros(total_blocks, np.int32)
    nb = ctypes.c_int(0)
    rc = ref().ref_attention_trace(hidden, heads, kv_heads, total_blocks, block_size, T, _p(x),
                                   _p(out), _p(q), _p(k), _p(v), _p(table), ctypes.byref(nb))
    if rc != 0:
        raise RuntimeError("reference attention trace failed")
    return out, q, k, v, table[: nb.value].copy()


def ref_decode_timing(hidden: int, heads: int, kv_heads: int, block_size: int, context: int, reps: int = 5):
    """Median ms of the reference's single-token PagedAttention::forward at a
    context of `context` tokens and at a context of 1 (identity projections)."""
    a, b = ctypes.c_double(0.0), ctypes.c_double(0.0)
    rc = ref().ref_decode_timing(hidden, heads, kv_heads, block_size, context, reps, ctypes.byref(a),
                                 ctypes.byref(b))
    if rc != 0:
        raise RuntimeError("reference decode timing failed")
    return a.value, b.value


def ref_bf16_rne(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    if ref().ref_bf16_rne_n(_p(x), _p(out), x.size) != 0:
        raise RuntimeError("reference bf16 conversion failed")
    return out

"""The C ABI library on the CPU: it loads, exports every symbol the header
declares, sizes workspaces, and rejects invalid arguments with the
reference's invalid_argument semantics (src/cuda/gemm_cuda.cu:920-928) before
touching a device.  No kernel runs here."""
import ctypes
import math
import shutil
import subprocess

import pytest

import stratakv_amd as skv


def test_library_exports_every_header_symbol():
    names = skv.header_symbols()
    assert len(names) >= 20
    lib = ctypes.CDLL(skv.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"
    assert skv.lib().skv_abi_version() >= 1


def test_gemm_library_exports_every_header_symbol():
    names = skv.header_symbols(skv.GEMM_HEADER_PATH)
    assert len(names) == 5
    assert not set(names) & set(skv.header_symbols()), "declared in both headers"
    glib = skv.gemm_lib()
    missing = [n for n in names if not hasattr(glib, n)]
    assert not missing, f"declared but not exported: {missing}"


def _needed(path):
    out = subprocess.run(["readelf", "-d", path], stdout=subprocess.PIPE, text=True, check=True).stdout
    return [line.split("[")[1].split("]")[0] for line in out.splitlines() if "(NEEDED)" in line]


@pytest.mark.skipif(shutil.which("readelf") is None, reason="readelf not installed")
def test_only_the_gemm_library_links_hipblaslt():
    """libstratakv_amd.so (append, decode, layer kernels, host layer) loads
    without hipBLASLt; libstratakv_amd_gemm.so links it and the main library."""
    main = _needed(skv.LIB_PATH)
    assert not [n for n in main if "hipblaslt" in n], main
    gemm = _needed(skv.GEMM_LIB_PATH)
    assert any("hipblaslt" in n for n in gemm) and "libstratakv_amd.so" in gemm, gemm


def test_workspace_sizes_are_positive_and_bounded():
    small = skv.decode_workspace_bytes(1, 32, 4, 64)
    big = skv.decode_workspace_bytes(128, 32, 8, 128)
    assert 0 < small and 0 < big
    # partial slots do not depend on the batch; larger heads need more room
    assert skv.decode_workspace_bytes(64, 32, 8, 128) < skv.decode_workspace_bytes(64, 32, 8, 256)
    assert big < 256 << 20
    assert skv.decode_workspace_bytes(0, 32, 8, 128) == 0
    single = skv.lib().skv_paged_attention_decode_workspace_bytes(32, 4, 64)
    assert single == small


FAKE = 0x1000  # never dereferenced: validation rejects before any device work


@pytest.mark.parametrize("kw,msg", [
    (dict(context_len=0), "context"),
    (dict(num_q_heads=6, num_kv_heads=4), "multiple"),
    (dict(scale=0.0), "scale"),
    (dict(scale=math.inf), "scale"),
    (dict(scale=math.nan), "scale"),
    (dict(block_size=0), "dimensions"),
    (dict(query=None), "pointers"),
])
def test_single_decode_rejects_invalid_arguments(kw, msg):
    args = dict(query=FAKE, key_cache=FAKE, value_cache=FAKE, total_blocks=4, block_table=FAKE,
                output=FAKE, context_len=5, block_size=16, num_q_heads=8, num_kv_heads=4,
                head_dim=64, scale=0.125, workspace=FAKE, workspace_bytes=1 << 20)
    args.update(kw)
    with pytest.raises(skv.SkvInvalidArgument):
        skv.paged_attention_decode(**args)


def test_batched_decode_rejects_invalid_arguments():
    base = dict(q=FAKE, q_dtype=skv.DTYPE_BF16, k_pool=FAKE, v_pool=FAKE, total_blocks=4,
                block_tables=FAKE, max_blocks_per_seq=2, context_lens=FAKE, num_seqs=2,
                num_q_heads=8, num_kv_heads=4, head_dim=64, block_size=16, scale=0.125, out=FAKE,
                workspace=FAKE, workspace_bytes=1 << 30)
    for bad in (dict(q_dtype=7), dict(num_seqs=0), dict(num_kv_heads=3), dict(total_blocks=0),
                dict(context_lens=None)):
        with pytest.raises(skv.SkvInvalidArgument):
            skv.paged_decode(**dict(base, **bad))


def test_append_rejects_invalid_arguments():
    base = dict(k_new=FAKE, v_new=FAKE, src_dtype=skv.DTYPE_BF16, k_pool=FAKE, v_pool=FAKE,
                total_blocks=4, block_tables=FAKE, max_blocks_per_seq=2, positions=FAKE,
                num_seqs=1, tokens_per_seq=1, num_kv_heads=4, head_dim=64, block_size=16)
    for bad in (dict(src_dtype=9), dict(block_size=0), dict(k_pool=None), dict(num_seqs=-1)):
        with pytest.raises(skv.SkvInvalidArgument):
            skv.kv_append(**dict(base, **bad))
    skv.kv_append(**dict(base, num_seqs=0))  # empty batch is a no-op


def test_fused_decode_append_rejects_invalid_arguments():
    base = dict(q=FAKE, q_dtype=skv.DTYPE_BF16, k_new=FAKE, v_new=FAKE, kv_dtype=skv.DTYPE_BF16,
                k_pool=FAKE, v_pool=FAKE, total_blocks=4, block_tables=FAKE, max_blocks_per_seq=2,
                context_lens=FAKE, num_seqs=2, num_q_heads=8, num_kv_heads=4, head_dim=64,
                block_size=16, scale=0.125, out=FAKE, workspace=FAKE, workspace_bytes=1 << 30)
    for bad in (dict(kv_dtype=5), dict(q_dtype=7), dict(k_new=None), dict(num_seqs=0),
                dict(num_kv_heads=3), dict(scale=float("nan"))):
        with pytest.raises(skv.SkvInvalidArgument):
            skv.paged_decode_append(**dict(base, **bad))
    single = dict(query=FAKE, key_row=FAKE, value_row=FAKE, kv_dtype=skv.DTYPE_FP32,
                  key_cache=FAKE, value_cache=FAKE, total_blocks=4, block_table=FAKE, output=FAKE,
                  context_len=5, block_size=16, num_q_heads=8, num_kv_heads=4, head_dim=64,
                  scale=0.125, workspace=FAKE, workspace_bytes=1 << 20)
    for bad in (dict(context_len=0), dict(key_row=None), dict(kv_dtype=3), dict(num_q_heads=6)):
        with pytest.raises(skv.SkvInvalidArgument):
            skv.paged_attention_decode_append(**dict(single, **bad))


def test_multi_token_entry_points_reject_invalid_arguments():
    """The *_rows_f32 projections, skv_rope_rows_f32 and skv_write_i32 validate
    before any device work (INVALID_ARGUMENT), and refuse shapes the register
    tiling does not cover with UNSUPPORTED."""
    lib = skv.lib()
    eps = ctypes.c_float(1e-5)
    strides = (ctypes.c_int64 * 3)(2048, 2048, 2048)
    qkv = lambda rows, gamma, K, hd, normalized: lib.skv_fused_qkv_rows_f32(
        FAKE, rows, gamma, eps, FAKE, FAKE, FAKE, skv.DTYPE_BF16, 1, strides, None, None, None, K, 32, 4, hd,
        0, FAKE, FAKE, FAKE, normalized, None)
    assert qkv(0, FAKE, 2048, 64, FAKE) == skv.SKV_ERR_INVALID_ARGUMENT        # no rows
    assert qkv(4, FAKE, 2048, 63, FAKE) == skv.SKV_ERR_INVALID_ARGUMENT        # odd head_dim
    assert qkv(4, FAKE, 2048, 64, None) == skv.SKV_ERR_INVALID_ARGUMENT        # gamma without scratch
    assert "scratch" in skv.lib().skv_last_error().decode()
    assert qkv(4, FAKE, 2000, 64, FAKE) == skv.SKV_ERR_UNSUPPORTED             # K not a multiple of 512
    gate_up = lambda rows, K: lib.skv_fused_gate_up_swiglu_rows_f32(
        FAKE, rows, FAKE, eps, FAKE, FAKE, skv.DTYPE_BF16, 1, K, K, None, None, K, 5632, FAKE, FAKE, None)
    assert gate_up(0, 2048) == skv.SKV_ERR_INVALID_ARGUMENT
    assert gate_up(3, 8192) == skv.SKV_ERR_UNSUPPORTED                         # rows too long for registers
    res = lambda rows, dt, K: lib.skv_linear_residual_rows_f32(FAKE, rows, FAKE, dt, 1, K, K, 2048, None, FAKE,
                                                               FAKE, None)
    assert res(-1, skv.DTYPE_BF16, 2048) == skv.SKV_ERR_INVALID_ARGUMENT
    assert res(2, 9, 2048) == skv.SKV_ERR_INVALID_ARGUMENT                     # unknown dtype
    assert res(2, skv.DTYPE_FP32, 4096) == skv.SKV_ERR_UNSUPPORTED
    assert lib.skv_rope_rows_f32(FAKE, 3, 4, 63, 0, None) == skv.SKV_ERR_INVALID_ARGUMENT
    assert lib.skv_rope_rows_f32(FAKE, 3, 4, 1026, 0, None) == skv.SKV_ERR_INVALID_ARGUMENT
    assert lib.skv_rope_rows_f32(FAKE, 3, 4, 64, -1, None) == skv.SKV_ERR_INVALID_ARGUMENT
    vals = (ctypes.c_int32 * 17)(*range(17))
    assert lib.skv_write_i32(FAKE, vals, 17, None) == skv.SKV_ERR_INVALID_ARGUMENT
    assert lib.skv_write_i32(None, vals, 2, None) == skv.SKV_ERR_INVALID_ARGUMENT
    assert lib.skv_write_i32(FAKE, vals, 0, None) == skv.SKV_OK             # nothing to write


def test_matrix_core_projections_and_prompt_embedding_reject_invalid_arguments():
    """The *_mm_f32 projections and skv_embedding_rows_f32 validate before any
    device work: INVALID_ARGUMENT for bad sizes or a missing scratch,
    UNSUPPORTED (nothing launched) for shapes the matrix-core kernel does not
    take: fp32 weights, in_dim not a multiple of 128, an output count not a
    multiple of 32 (16 for gate/up), a rotated head_dim not a multiple of 32."""
    lib = skv.lib()
    eps = ctypes.c_float(1e-5)
    strides = (ctypes.c_int64 * 3)(2048, 2048, 2048)
    qkv = lambda rows, gamma, dt, K, hd, position, normalized: lib.skv_fused_qkv_mm_f32(
        FAKE, rows, gamma, eps, FAKE, FAKE, FAKE, dt, 1, strides, None, None, None, K, 32, 4, hd, position,
        FAKE, FAKE, FAKE, normalized, None)
    B = skv.DTYPE_BF16
    assert qkv(0, FAKE, B, 2048, 64, 0, FAKE) == skv.SKV_ERR_INVALID_ARGUMENT       # no rows
    assert qkv(4, FAKE, B, 2048, 64, 0, None) == skv.SKV_ERR_INVALID_ARGUMENT       # gamma without scratch
    assert qkv(4, FAKE, skv.DTYPE_FP32, 2048, 64, 0, FAKE) == skv.SKV_ERR_UNSUPPORTED
    assert qkv(4, FAKE, B, 2000, 64, 0, FAKE) == skv.SKV_ERR_UNSUPPORTED            # K not a multiple of 128
    assert qkv(4, FAKE, B, 2048, 48, 0, FAKE) == skv.SKV_ERR_UNSUPPORTED            # rotated head_dim 48
    gate_up = lambda rows, K, out: lib.skv_fused_gate_up_swiglu_mm_f32(
        FAKE, rows, FAKE, eps, FAKE, FAKE, B, 1, K, K, None, None, K, out, FAKE, FAKE, None)
    assert gate_up(0, 2048, 5632) == skv.SKV_ERR_INVALID_ARGUMENT
    assert gate_up(3, 2048, 5640) == skv.SKV_ERR_UNSUPPORTED                        # out_dim not a multiple of 16
    res = lambda rows, K, out: lib.skv_linear_residual_mm_f32(FAKE, rows, FAKE, B, 1, K, K, out, None, FAKE, FAKE,
                                                             None)
    assert res(-1, 2048, 2048) == skv.SKV_ERR_INVALID_ARGUMENT
    assert res(2, 2048, 2050) == skv.SKV_ERR_UNSUPPORTED                            # out_dim not a multiple of 32
    emb = lambda table, first, rows: lib.skv_embedding_rows_f32(table, B, 32000, 2048, FAKE, first, rows, FAKE,
                                                                None, None)
    assert emb(FAKE, 0, 0) == skv.SKV_ERR_INVALID_ARGUMENT                          # no rows
    assert emb(FAKE, 0, 65536) == skv.SKV_ERR_INVALID_ARGUMENT                      # more than one launch takes
    assert emb(FAKE, -1, 4) == skv.SKV_ERR_INVALID_ARGUMENT
    assert emb(None, 0, 4) == skv.SKV_ERR_INVALID_ARGUMENT


def test_library_gemm_projections_reject_invalid_arguments():
    """The *_gemm_f32 projections validate before any device work:
    INVALID_ARGUMENT for bad sizes, a missing scratch or a workspace that is
    misaligned or smaller than skv_prompt_gemm_workspace_bytes; UNSUPPORTED
    (nothing launched, hipBLASLt not asked) for fp32 weights, in_dim not a
    multiple of 8, an output count not a multiple of 8, a rotated head_dim not
    a multiple of 8."""
    lib = skv.gemm_lib()
    eps = ctypes.c_float(1e-5)
    wsb = lib.skv_prompt_gemm_workspace_bytes
    # [2 rows][K] bf16 parts, [2 rows][outputs] fp32 and a RoPE table of 4 rows (outputs / 3) bytes, each
    # rounded up to 256 bytes, + 32 MiB
    assert wsb(1024, 2048, 2560) == 4 * 1024 * 2048 + 8 * 1024 * 2560 + 4 * 1024 * 853 + (32 << 20)
    assert wsb(3, 8, 8) == 256 + 256 + 256 + (32 << 20)
    assert wsb(0, 2048, 2048) == 0
    B = skv.DTYPE_BF16
    strides = (ctypes.c_int64 * 3)(2048, 2048, 2048)
    big = wsb(64, 8192, 16384)
    qkv = lambda rows, gamma, dt, K, hd, position, normalized, ws=FAKE, nbytes=big: lib.skv_fused_qkv_gemm_f32(
        FAKE, rows, gamma, eps, FAKE, FAKE, FAKE, dt, 1, strides, None, None, None, K, 32, 4, hd, position,
        FAKE, FAKE, FAKE, normalized, ws, nbytes, None)
    assert qkv(0, FAKE, B, 2048, 64, 0, FAKE) == skv.SKV_ERR_INVALID_ARGUMENT       # no rows
    assert qkv(4, FAKE, B, 2048, 64, 0, None) == skv.SKV_ERR_INVALID_ARGUMENT       # gamma without scratch
    assert qkv(4, FAKE, B, 2048, 64, 0, FAKE, ws=FAKE + 16) == skv.SKV_ERR_INVALID_ARGUMENT   # misaligned
    assert qkv(4, FAKE, B, 2048, 64, 0, FAKE, nbytes=wsb(4, 2048, 2560) - 1) == skv.SKV_ERR_INVALID_ARGUMENT
    assert qkv(4, FAKE, skv.DTYPE_FP32, 2048, 64, 0, FAKE) == skv.SKV_ERR_UNSUPPORTED
    assert qkv(4, FAKE, B, 2044, 64, 0, FAKE) == skv.SKV_ERR_UNSUPPORTED            # K not a multiple of 8
    assert qkv(4, FAKE, B, 2048, 12, 0, FAKE) == skv.SKV_ERR_UNSUPPORTED            # rotated head_dim 12
    gate_up = lambda rows, K, out: lib.skv_fused_gate_up_swiglu_gemm_f32(
        FAKE, rows, FAKE, eps, FAKE, FAKE, B, 1, K, K, None, None, K, out, FAKE, FAKE, FAKE, big, None)
    assert gate_up(0, 2048, 5632) == skv.SKV_ERR_INVALID_ARGUMENT
    assert gate_up(3, 2048, 5636) == skv.SKV_ERR_UNSUPPORTED                        # out_dim not a multiple of 8
    res = lambda rows, K, out, nbytes=big: lib.skv_linear_residual_gemm_f32(
        FAKE, rows, FAKE, B, 1, K, K, out, None, FAKE, FAKE, FAKE, nbytes, None)
    assert res(-1, 2048, 2048) == skv.SKV_ERR_INVALID_ARGUMENT
    assert res(2, 2048, 2048, nbytes=0) == skv.SKV_ERR_INVALID_ARGUMENT
    assert res(2, 2048, 2052) == skv.SKV_ERR_UNSUPPORTED                            # out_dim not a multiple of 8
    ffn = lambda rows, H, I, normalized=FAKE, nbytes=big: lib.skv_ffn_swiglu_gemm_f32(
        FAKE, rows, FAKE, eps, FAKE, FAKE, FAKE, B, 1, H, H, I, None, None, None, H, I, FAKE, normalized, FAKE,
        nbytes, None)
    assert ffn(0, 2048, 5632) == skv.SKV_ERR_INVALID_ARGUMENT
    assert ffn(4, 2048, 5632, normalized=None) == skv.SKV_ERR_INVALID_ARGUMENT       # gamma without scratch
    assert ffn(4, 2048, 5632, nbytes=wsb(4, 5632, 11264) - 1) == skv.SKV_ERR_INVALID_ARGUMENT
    assert ffn(4, 2048, 5636) == skv.SKV_ERR_UNSUPPORTED                            # inter not a multiple of 8

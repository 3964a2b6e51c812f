/*
 * oracle.h -- CPU restatement of StrataKV's paged-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (stratakv_amd/, include/)
 * links, loads or calls this code; only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg use it, and only as the checker / the timed CPU
 * baseline.  Every function cites the reference lines it restates
 * (paths relative to the StrataKV source tree).
 *
 * Pinning (what checks each function independently of this restatement):
 *   oracle_bf16_*          phase7 known-answer bytes (tests/phase7_smoke.cpp:41-53),
 *                          an independent nearest-value rounding model in numpy,
 *                          and the reference's own Tensor::set_value via oracle/_ref.
 *   oracle_pool_trace      main.cpp Phase 3/4 known answers (src/main.cpp:298-408,
 *                          73-156) and random traces against the reference's own
 *                          BlockPool/PageTable via oracle/_ref.
 *   oracle_kv_append       the layout invariant (element at the F2 index equals the
 *                          input bits, every other element unchanged) and a numpy
 *                          fancy-index scatter.
 *   oracle_paged_decode_*  phase6 RoPE closed form (tests/phase6_smoke.cpp:60-96),
 *                          float64 brute force, special cases (L=1, equal keys,
 *                          dominant key, group sharing, block-permutation
 *                          invariance) and the reference's own
 *                          PagedAttention::forward via oracle/_ref.
 */
#ifndef STRATAKV_ORACLE_H
#define STRATAKV_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- bf16 rules ---------------------------------------------------------- */
/* Exact widen: bits << 16 (src/cpu/tensor.cpp:200-206). */
float oracle_bf16_to_f32(uint16_t h);
/* Round to nearest, ties to even on raw bits (src/cpu/tensor.cpp:218-225). */
uint16_t oracle_f32_to_bf16_rne(float x);
/* Truncation (src/cuda/gemm_cuda.cu:74-83, src/io/safetensors.cpp:660-666). */
uint16_t oracle_f32_to_bf16_trunc(float x);
void oracle_bf16_to_f32_n(const uint16_t* in, float* out, size_t n);
void oracle_f32_to_bf16_rne_n(const float* in, uint16_t* out, size_t n);

/* ---- BlockPool / PageTable ------------------------------------------------ */
#define ORACLE_OP_ALLOC_SEQ 1  /* PageTable::allocate_sequence */
#define ORACLE_OP_APPEND    2  /* PageTable::append_token      */
#define ORACLE_OP_FREE_SEQ  3  /* PageTable::free_sequence     */
#define ORACLE_ST_OK        0
#define ORACLE_ST_OOM       1  /* std::runtime_error("OOM")              */
#define ORACLE_ST_UNKNOWN   2  /* runtime_error ": unknown seq_id=..."   */
#define ORACLE_ST_EXISTS    3  /* runtime_error "... already exists"     */
/*
 * Replay ops[2*i] = opcode, ops[2*i+1] = seq_id (0 <= seq_id < max_seqs) on a
 * fresh pool of `total` blocks of `block_size` tokens.  Per op writes
 * results[2*i] = status, results[2*i+1] = block id taken by the op or -1.
 * Afterwards: lens[s] = sequence length or -1 when absent, blocks[s*max_blocks_out + k]
 * = its k-th block (-1 padded), and drain[0..total) = the ids allocate_block()
 * hands out until the pool is empty (the free stack from the top), returning
 * how many were drained.
 */
int oracle_pool_trace(int total, int block_size, const int32_t* ops, int n_ops,
                      int max_seqs, int32_t* results, int32_t* lens, int32_t* blocks,
                      int max_blocks_out, int32_t* drain);

/* ---- KV append ------------------------------------------------------------ */
/* Same contract as skv_kv_append (src/models/transformer_block.cpp:484-509). */
void oracle_kv_append(const void* k_new, const void* v_new, int src_fp32,
                      uint16_t* k_pool, uint16_t* v_pool, int64_t total_blocks,
                      const int32_t* tables, int max_blocks, const int32_t* positions,
                      const int32_t* offsets, int num_seqs, int tokens_per_seq,
                      int num_kv_heads, int head_dim, int block_size);

/* ---- paged decode attention ---------------------------------------------- */
/*
 * Two-pass fp32 softmax attention over bf16 pools widened exactly to fp32,
 * loop for loop as src/layers/attention.cpp:263-337: dot in d order, score =
 * dot*scale, max, exp(score-max), denominator, then out[d] = sum_p (s_p/den)*v_p[d].
 * q, out: [B][Hq][hd] fp32.  Returns 0, or -1 (non-finite / non-positive
 * denominator, attention.cpp:313-316), -2 (block outside the pool,
 * attention.cpp:139-143), -3 (no page for a position, attention.cpp:282-285).
 * Sequences with lens[b] <= 0 give zeros.
 */
int oracle_paged_decode_f32(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                            int64_t total_blocks, const int32_t* tables, int max_blocks,
                            const int32_t* lens, int B, int Hq, int Hkv, int hd, int bs,
                            float scale, float* out);
/* The same attention in double precision with libm exp (the "truth"). */
int oracle_paged_decode_f64(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                            int64_t total_blocks, const int32_t* tables, int max_blocks,
                            const int32_t* lens, int B, int Hq, int Hkv, int hd, int bs,
                            double scale, double* out);
/* The same loops over fp32 pools, the reference's own cache element type
 * (src/memory/block_pool.cpp:85-105); used to compare with the reference on
 * exactly the values it cached. */
int oracle_paged_decode_f32_fp32pool(const float* q, const float* k_pool, const float* v_pool,
                                     int64_t total_blocks, const int32_t* tables, int max_blocks,
                                     const int32_t* lens, int B, int Hq, int Hkv, int hd, int bs,
                                     float scale, float* out);
/* oracle_paged_decode_f32 with the (sequence, head) pairs spread over
 * `threads` POSIX threads (threads <= 1: the single-threaded loop). */
int oracle_paged_decode_f32_mt(const float* q, const uint16_t* k_pool, const uint16_t* v_pool,
                               int64_t total_blocks, const int32_t* tables, int max_blocks,
                               const int32_t* lens, int B, int Hq, int Hkv, int hd, int bs,
                               float scale, float* out, int threads);

#ifdef __cplusplus
}
#endif

#endif /* STRATAKV_ORACLE_H */

/*
 * stratakv_amd.h -- C ABI of the MI355X (gfx950) paged KV-cache hot path.
 *
 * Plain C types only: bf16 values are `uint16_t` bit patterns, block tables are
 * `int32_t`, outputs are `float`, a stream is an opaque `void*` (a hipStream_t;
 * NULL is the default stream).  Every entry point returns an `int` status
 * (SKV_OK == 0) and never throws; `skv_last_error()` gives the message of the
 * last failure on the calling thread.  Nothing on the append/decode path
 * allocates: the caller passes every buffer, including a workspace sized by
 * `skv_paged_decode_workspace_bytes`.
 *
 * KV layout (unchanged from the reference, src/models/transformer_block.cpp:493-499,
 * src/layers/attention.cpp:137-151): separate K and V pools, each
 *     [total_blocks][block_size][num_kv_heads][head_dim]   (bf16)
 * element offset = ((block * block_size + slot) * num_kv_heads + kv_head) * head_dim + d,
 * computed in 64-bit.  The reference stores FP32; this build stores bf16 in the
 * same index space.
 *
 * Reference interfaces replaced (paths relative to the StrataKV source tree):
 *   skv_kv_append               <- the two cudaMemcpy D2D of one token's K/V rows,
 *                                  src/models/transformer_block.cpp:484-509
 *                                  (CPU twin src/layers/attention.cpp:236-259)
 *   skv_paged_attention_decode  <- paged_attention_decode_cuda,
 *                                  include/stratakv/cuda/gemm_cuda.h:40-44,
 *                                  src/cuda/gemm_cuda.cu:915-935
 *   skv_paged_decode            <- the same, batched over sequences (the reference
 *                                  decodes exactly one sequence per call)
 *   skv_malloc / skv_free / skv_memcpy_*
 *                               <- the cudaMalloc/cudaFree/cudaMemcpy calls of
 *                                  BlockPool and PageTable,
 *                                  src/memory/block_pool.cpp:85-105,118-145,
 *                                  src/memory/page_table.cpp:180-238
 */
#ifndef STRATAKV_AMD_H
#define STRATAKV_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes -------------------------------------------------------- */
#define SKV_OK                   0
#define SKV_ERR_INVALID_ARGUMENT 1  /* reference: std::invalid_argument        */
#define SKV_ERR_HIP              2  /* reference: CUDA failure -> runtime_error */
#define SKV_ERR_WORKSPACE        3  /* workspace missing or too small           */
#define SKV_ERR_UNSUPPORTED      4  /* shape outside every compiled kernel      */

/* ---- element types ------------------------------------------------------- */
#define SKV_DTYPE_BF16 0
#define SKV_DTYPE_FP32 1
#define SKV_DTYPE_F16  2  /* checkpoint tensors only (skv_convert_*, skv_embedding_f32) */

/* ---- device status flags (bits of an int32 in device memory, set by the
 *      token-choice and embedding kernels; never cleared by them) ---------- */
#define SKV_FLAG_NONFINITE_LOGITS 1  /* a logit was NaN or infinite            */
#define SKV_FLAG_BAD_TOKEN        2  /* an embedding id outside [0, vocab)      */
#define SKV_FLAG_NONFINITE_SCALED 4  /* a logit / temperature was not finite   */
#define SKV_FLAG_BAD_DISTRIBUTION 8  /* the filtered softmax total was not > 0  */

/* Message of the last failing call on this thread ("" if none). */
const char* skv_last_error(void);
/* ABI version, bumped on any signature change. */
int skv_abi_version(void);

/* ---- device plumbing (no counterpart on the hot path; used by the C++
 *      BlockPool/PageTable, the tests and the benchmark) -------------------- */
int skv_device_count(int* count);
int skv_set_device(int device);
int skv_malloc(void** ptr, size_t bytes);
int skv_free(void* ptr);
int skv_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int skv_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int skv_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int skv_memset_d8(void* dst, int value, size_t bytes, void* stream);
int skv_stream_create(void** stream);
int skv_stream_destroy(void* stream);
int skv_stream_synchronize(void* stream);
int skv_device_synchronize(void);
/* Events for timing and ordering on a given stream. */
int skv_event_create(void** event);
int skv_event_destroy(void* event);
int skv_event_record(void* event, void* stream);
int skv_event_synchronize(void* event);
int skv_event_elapsed_ms(float* ms, void* start, void* stop);
/* *done = 1 when the work before the event has completed, else 0 (no wait). */
int skv_event_query(void* event, int* done);
/* Page-locked host memory, so host-to-device copies can run asynchronously. */
int skv_host_alloc(void** ptr, size_t bytes);
int skv_host_free(void* ptr);
/* Asynchronous copy on `stream` (src should be page-locked; the call returns
 * before the copy completes). */
int skv_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void* stream);
/* The same device-to-host (dst should be page-locked). */
int skv_memcpy_d2h_async(void* dst, const void* src, size_t bytes, void* stream);
/* dst[pairs[2i]] = pairs[2i+1] for i < n: applies a batch of (index, value)
 * updates to a device int32 array (incremental block-table upload). */
int skv_scatter_i32(int32_t* dst, const int32_t* pairs, int n, void* stream);
/* dst[i] = values[i] for i < n (n <= 16), ordered on `stream`; the values are
 * copied into the launch, so `values` (host memory) may be reused on return. */
int skv_write_i32(int32_t* dst, const int32_t* values, int n, void* stream);

/* ---- synthetic data ------------------------------------------------------ */
/* dst[i] = bf16_rne(N(0,1) sample derived from (seed, first_index + i)) via a
 * counter hash (no library RNG), so any sub-range can be regenerated alone. */
int skv_fill_normal_bf16(uint16_t* dst, size_t count, uint64_t seed,
                         uint64_t first_index, void* stream);
/* The same with each sample scaled by stddev before rounding (random-init
 * weights, e.g. N(0, 0.02)). */
int skv_fill_normal_scaled_bf16(uint16_t* dst, size_t count, uint64_t seed,
                                uint64_t first_index, float stddev, void* stream);
/* Fill count elements of a bf16 buffer with one 16-bit pattern. */
int skv_fill_u16(uint16_t* dst, size_t count, uint16_t value, void* stream);

/* ---- KV append ------------------------------------------------------------
 * Scatter new tokens' K and V rows into the paged pools through the block
 * tables.  Token j of sequence b (its row is
 *     k_new[(token_offsets ? token_offsets[b] : b * tokens_per_seq) + j]
 * a row being num_kv_heads*head_dim elements) lands at logical position
 * positions[b] + j of that sequence:
 *     block = block_tables[b * max_blocks_per_seq + pos / block_size],
 *     slot  = pos % block_size.
 * Sequence b receives tokens_per_seq tokens, or, when token_offsets is
 * non-NULL, min(token_offsets[b+1]-token_offsets[b], tokens_per_seq) tokens
 * (ragged batches pass the longest count as tokens_per_seq).
 * src_dtype SKV_DTYPE_BF16: the pool receives the input bits unchanged.
 * src_dtype SKV_DTYPE_FP32: round-to-nearest-even to bf16 with the rule of
 * Tensor::set_value (src/cpu/tensor.cpp:209-229).
 * Rows whose table entry falls outside [0, total_blocks) or whose position
 * falls outside the table are skipped, never written.
 * Replaces: src/models/transformer_block.cpp:484-509. */
int skv_kv_append(const void* k_new, const void* v_new, int src_dtype,
                  uint16_t* k_pool, uint16_t* v_pool, int64_t total_blocks,
                  const int32_t* block_tables, int max_blocks_per_seq,
                  const int32_t* positions, const int32_t* token_offsets,
                  int num_seqs, int tokens_per_seq,
                  int num_kv_heads, int head_dim, int block_size,
                  void* stream);

/* Single-token append with the position passed by value: the exact
 * replacement for the two per-token cudaMemcpy of one K row and one V row
 * (src/models/transformer_block.cpp:484-509).  block_table is the
 * sequence's device table of table_len entries. */
int skv_kv_append_token(const void* k_row, const void* v_row, int src_dtype,
                        uint16_t* k_pool, uint16_t* v_pool, int64_t total_blocks,
                        const int32_t* block_table, int table_len, int position,
                        int num_kv_heads, int head_dim, int block_size,
                        void* stream);

/* ---- paged decode attention ---------------------------------------------
 * One query token per sequence, grouped-query attention over the paged pools:
 * q head h reads kv head h / (num_q_heads / num_kv_heads) (reference
 * src/cuda/gemm_cuda.cu:324-325, src/layers/attention.cpp:270).
 *   q     [num_seqs][num_q_heads][head_dim], bf16 or fp32 (q_dtype)
 *   out   [num_seqs][num_q_heads][head_dim], fp32
 *   out[b,h] = sum_t softmax_t(scale * q[b,h].k_t) v_t over t < context_lens[b]
 * fp32 accumulation.  Sequences with context_lens[b] <= 0 produce zeros.
 * Context positions beyond max_blocks_per_seq*block_size and table entries
 * outside [0, total_blocks) are not read.
 * workspace: device memory of at least skv_paged_decode_workspace_bytes(...)
 * bytes for the same arguments; its contents need no initialisation.
 * Replaces: paged_attention_decode_cuda (include/stratakv/cuda/gemm_cuda.h:40-44). */
size_t skv_paged_decode_workspace_bytes(int num_seqs, int num_q_heads,
                                        int num_kv_heads, int head_dim);
int skv_paged_decode(const void* q, int q_dtype,
                     const uint16_t* k_pool, const uint16_t* v_pool,
                     int64_t total_blocks,
                     const int32_t* block_tables, int max_blocks_per_seq,
                     const int32_t* context_lens, int num_seqs,
                     int num_q_heads, int num_kv_heads, int head_dim,
                     int block_size, float scale, float* out,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Fused decode step: appends each sequence's new token at position
 * context_lens[b] - 1 and decodes over context_lens[b] tokens, in one launch.
 * k_new / v_new: [num_seqs][num_kv_heads][head_dim] in kv_dtype (bf16 bits are
 * stored as given, fp32 is rounded to nearest-even like skv_kv_append).  The
 * pools and `out` end up bit-identical to skv_kv_append(k_new, v_new, ...,
 * positions = context_lens - 1, tokens_per_seq = 1) followed by
 * skv_paged_decode(...) on the same stream; the same positions are skipped
 * (beyond the table, or a block outside the pool).  Workspace as for
 * skv_paged_decode.
 * Replaces: the per-token K/V copy followed by paged_attention_decode_cuda in
 * forward_into (src/models/transformer_block.cpp:484-509 then 511-518), for a
 * batch of sequences. */
int skv_paged_decode_append(const void* q, int q_dtype,
                            const void* k_new, const void* v_new, int kv_dtype,
                            uint16_t* k_pool, uint16_t* v_pool,
                            int64_t total_blocks,
                            const int32_t* block_tables, int max_blocks_per_seq,
                            const int32_t* context_lens, int num_seqs,
                            int num_q_heads, int num_kv_heads, int head_dim,
                            int block_size, float scale, float* out,
                            void* workspace, size_t workspace_bytes, void* stream);

/* skv_paged_decode_append without a workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The partial results live in a library-owned device array of 24 MiB per GPU
 * (held from the first use until the process ends); the grid uses as many
 * ranges as fit in it (every benchmark shape fits its full persistent grid),
 * and a shape with more query heads x head_dim than one range per head needs
 * is refused with SKV_ERR_UNSUPPORTED.  Calls no allocation routine.  All
 * calls on one GPU share that array: calls that overlap in time on one GPU
 * (different streams, no ordering between them) race and must not be made. */
int skv_paged_decode_append_noalloc(const void* q, int q_dtype,
                                    const void* k_new, const void* v_new, int kv_dtype,
                                    uint16_t* k_pool, uint16_t* v_pool,
                                    int64_t total_blocks,
                                    const int32_t* block_tables, int max_blocks_per_seq,
                                    const int32_t* context_lens, int num_seqs,
                                    int num_q_heads, int num_kv_heads, int head_dim,
                                    int block_size, float scale, float* out, void* stream);

/* Chunked prefill attention over the paged cache.  The query rows
 * seq_offsets[b] .. seq_offsets[b+1]-1 of q ([num_tokens][num_q_heads][head_dim],
 * q_dtype) are sequence b's chunk: the last n_b positions of its
 * context_lens[b]-token context, already appended to the pools
 * (skv_kv_append).  Row i of the chunk attends causally to positions
 * 0 .. context_lens[b] - n_b + i of its sequence.  out: [num_tokens][Hq][hd]
 * fp32.  seq_offsets [num_seqs + 1] and context_lens [num_seqs] are device
 * arrays; num_tokens (= seq_offsets[num_seqs]) sizes the grid on the host.
 * num_seqs <= 4096.  Blocks outside the pool and positions past the table are
 * skipped as in skv_paged_decode; a row with no visible key gives zeros.
 * Numerics (block_size 16, head_dim 64 or 128): scores in bf16 x bf16 (an fp32
 * query split into hi + lo parts) and P.V in fp16 x fp16 on the matrix cores,
 * fp32 accumulation; V converts to fp16 exactly in [2^-14, 65504], and a
 * workgroup whose keys hold a V element beyond 65504 recomputes its rows in
 * fp32.  Other shapes run in fp32 throughout.
 * Replaces: the CPU-only multi-token path of PagedAttention::forward
 * (src/layers/attention.cpp:197-337), which the reference has no GPU kernel
 * for. */
int skv_paged_prefill(const void* q, int q_dtype, const uint16_t* k_pool,
                      const uint16_t* v_pool, int64_t total_blocks,
                      const int32_t* block_tables, int max_blocks_per_seq,
                      const int32_t* seq_offsets, const int32_t* context_lens,
                      int num_seqs, int num_tokens, int num_q_heads,
                      int num_kv_heads, int head_dim, int block_size, float scale,
                      float* out, void* stream);

/* Single-sequence decode with the reference's argument list (gemm_cuda.h:41-44)
 * on bf16 pools, plus the pool size, workspace and stream.  Equivalent to
 * skv_paged_decode with num_seqs = 1, an fp32 query, max_blocks_per_seq =
 * ceil(context_len / block_size) and context_lens = {context_len}; the
 * context length is passed to the kernels by value (no host-device copy).
 * Invalid arguments (context_len <= 0, num_q_heads % num_kv_heads != 0,
 * non-finite or non-positive scale, NULL pointers) return
 * SKV_ERR_INVALID_ARGUMENT like the reference's std::invalid_argument
 * (src/cuda/gemm_cuda.cu:920-928). */
size_t skv_paged_attention_decode_workspace_bytes(int num_q_heads,
                                                  int num_kv_heads,
                                                  int head_dim);
int skv_paged_attention_decode(const float* query, const uint16_t* key_cache,
                               const uint16_t* value_cache,
                               int64_t total_blocks,
                               const int32_t* block_table, float* output,
                               int context_len, int block_size,
                               int num_q_heads, int num_kv_heads, int head_dim,
                               float scale, void* workspace,
                               size_t workspace_bytes, void* stream);

/* skv_paged_attention_decode that first appends one token's K/V rows
 * ([num_kv_heads][head_dim], kv_dtype) at position context_len - 1, in the same
 * launch; equal to skv_kv_append_token(key_row, value_row, kv_dtype, ...,
 * table_len = ceil(context_len / block_size), position = context_len - 1)
 * followed by skv_paged_attention_decode.
 * Replaces: transformer_block.cpp:484-509 (the K/V cudaMemcpy pair) plus the
 * paged_attention_decode_cuda call that follows it (:511-518). */
int skv_paged_attention_decode_append(const float* query, const void* key_row,
                                      const void* value_row, int kv_dtype,
                                      uint16_t* key_cache, uint16_t* value_cache,
                                      int64_t total_blocks,
                                      const int32_t* block_table, float* output,
                                      int context_len, int block_size,
                                      int num_q_heads, int num_kv_heads,
                                      int head_dim, float scale, void* workspace,
                                      size_t workspace_bytes, void* stream);

/* ---- decoder-layer sub-steps around the path -----------------------------
 * Used by TransformerBlock::forward_into (include/stratakv/models/) for the
 * steps before and after the KV append and decode; fp32 activations.
 * Reference kernels replaced: rmsnorm_cuda, matmul_cuda_tiled's M=1 GEMV,
 * rope_split_half_cuda + generate_rope_frequencies_cuda, swiglu_inplace_cuda,
 * add_inplace_cuda (include/stratakv/cuda/gemm_cuda.h:13-38). */
/* out[r] = in[r] / sqrt(mean(in[r]^2) + epsilon) * gamma, rows of `hidden`. */
int skv_rmsnorm_f32(const float* input, float* output, const float* gamma,
                    int rows, int hidden, float epsilon, void* stream);
/* y[r][n] = sum_k x[r][k] * W[k][n] (+ bias[n]); W element (k, n) lives at
 * weight[k * stride_k + n * stride_n], bf16 or fp32 (weight_dtype); either
 * stride_k == 1 (output-major rows) or stride_n == 1 (GEMM-ready). */
int skv_linear_f32(const float* x, int rows, const void* weight, int weight_dtype,
                   int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                   const float* bias, float* y, void* stream);
/* In-place split-half rotary embedding of `heads` contiguous head vectors at
 * `position` (src/layers/attention.cpp:96-135).  The angles are computed on
 * the host in double and rounded to float (cos, sin per pair), so head_dim is
 * at most 512; larger head dimensions give SKV_ERR_INVALID_ARGUMENT. */
int skv_rope_f32(float* x, int heads, int head_dim, int position, void* stream);
/* gate[i] = gate[i] * sigmoid(gate[i]) * up[i]. */
int skv_swiglu_f32(float* gate, const float* up, int n, void* stream);
/* skv_rope_f32 over `rows` rows of `heads` head vectors, row r at position
 * first_position + r; cos/sin of each angle computed on the device in double
 * from the same float inverse frequencies and rounded to float
 * (src/layers/attention.cpp:96-135 per token). */
int skv_rope_rows_f32(float* x, int rows, int heads, int head_dim, int first_position,
                      void* stream);
/* target[i] += source[i]. */
int skv_add_f32(float* target, const float* source, int n, void* stream);

/* Fused projections of one decode step (a single token), each one launch and
 * bit-identical to the separate kernels above on the same inputs.  Weights
 * must be output-major rows (stride_k == 1: the transpose view of a checkpoint
 * [out][in] matrix), 16-byte aligned, with in_dim <= 8192; otherwise the call
 * returns SKV_ERR_UNSUPPORTED and changes nothing (use the separate kernels).
 * The outputs must not alias the input x / hidden.
 *
 * q, k, v = (rmsnorm(hidden; gamma) W_q, W_k, W_v) + bias; with position >= 0
 * q and k are then rotated like skv_rope_f32 at that position (gamma NULL: no
 * normalisation).  stride_n[3]: row strides of W_q, W_k, W_v.
 * Replaces: rmsnorm_cuda + 3 x Linear::forward_into + generate_rope_frequencies
 * + 2 x rope_split_half_cuda (src/models/transformer_block.cpp:432-474). */
int skv_fused_qkv_f32(const float* hidden, const float* gamma, float epsilon,
                      const void* wq, const void* wk, const void* wv, int weight_dtype,
                      int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                      const float* bias_k, const float* bias_v, int hidden_dim,
                      int num_heads, int num_kv_heads, int head_dim, int position,
                      float* q, float* k, float* v, void* stream);
/* skv_fused_qkv_f32 at a position held in device memory, for a decode step
 * captured once in a HIP graph and replayed per token: the position is
 * *position_at (device int32, clamped to [0, rope_positions)), and q and k are
 * rotated by the cos/sin pairs rope_cos_sin[position][head_dim / 2][2]
 * (device fp32, filled from skv_rope_cos_sin).  With the same position the
 * results are bit-identical to skv_fused_qkv_f32.  No counterpart in the
 * reference: its decode step takes the position from the host. */
int skv_fused_qkv_at_f32(const float* hidden, const float* gamma, float epsilon,
                         const void* wq, const void* wk, const void* wv, int weight_dtype,
                         int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                         const float* bias_k, const float* bias_v, int hidden_dim,
                         int num_heads, int num_kv_heads, int head_dim, const int32_t* position_at,
                         const float* rope_cos_sin, int rope_positions, float* q, float* k,
                         float* v, void* stream);
/* Host function (no device work): cos_sin[p][i] = (cos, sin) of position
 * first_position + p at pair i, for p < positions and i < head_dim / 2, as
 * float pairs ([positions][head_dim] floats): the values skv_fused_qkv_f32
 * rotates by, for the device table of skv_fused_qkv_at_f32. */
int skv_rope_cos_sin(int head_dim, int first_position, int positions, float* cos_sin);
/* act[n] = swiglu(gate_n, up_n), gate/up = rmsnorm(x; gamma) W + bias.
 * Replaces: rmsnorm_cuda + gate/up Linear::forward_into + swiglu_inplace_cuda
 * (src/models/transformer_block.cpp:542-575). */
int skv_fused_gate_up_swiglu_f32(const float* x, const float* gamma, float epsilon,
                                 const void* w_gate, const void* w_up, int weight_dtype,
                                 int64_t stride_k, int64_t stride_n_gate,
                                 int64_t stride_n_up, const float* bias_gate,
                                 const float* bias_up, int in_dim, int out_dim,
                                 float* act, void* stream);
/* y = x W + bias + residual (y may alias residual).
 * Replaces: Linear::forward_into + add_inplace_cuda of o_proj and of
 * down_proj (src/models/transformer_block.cpp:528-541, 582-594). */
int skv_linear_residual_f32(const float* x, const void* weight, int weight_dtype,
                            int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                            const float* bias, const float* residual, float* y,
                            void* stream);

/* The same three projections for `rows` consecutive tokens of one sequence
 * (prompt prefill): hidden / x / residual / q / k / v / act / y are row-major
 * [rows][dim].  Every row's outputs have the bits the one-token entry point
 * gives for that row alone (token r of skv_fused_qkv_rows_f32 rotated at
 * first_position + r); each weight row is read from HBM once for all rows.
 * With gamma, `normalized` is caller scratch of rows * in_dim floats (the
 * normalised inputs are written there; distinct from every other buffer).
 * SKV_ERR_UNSUPPORTED (nothing launched) unless the weights are aligned
 * output-major rows with in_dim a multiple of 512 and <= 6,144 (bf16) or of
 * 256 and <= 2,048 (fp32).
 * Replaces: the multi-token rows of the reference's CPU
 * TransformerBlock::forward (src/models/transformer_block.cpp:300-332), whose
 * GPU forward_into takes one token (:348-351). */
int skv_fused_qkv_rows_f32(const float* hidden, int rows, const float* gamma, float epsilon,
                           const void* wq, const void* wk, const void* wv, int weight_dtype,
                           int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                           const float* bias_k, const float* bias_v, int hidden_dim,
                           int num_heads, int num_kv_heads, int head_dim, int first_position,
                           float* q, float* k, float* v, float* normalized, void* stream);
int skv_fused_gate_up_swiglu_rows_f32(const float* x, int rows, const float* gamma, float epsilon,
                                      const void* w_gate, const void* w_up, int weight_dtype,
                                      int64_t stride_k, int64_t stride_n_gate,
                                      int64_t stride_n_up, const float* bias_gate,
                                      const float* bias_up, int in_dim, int out_dim,
                                      float* act, float* normalized, void* stream);
int skv_linear_residual_rows_f32(const float* x, int rows, const void* weight, int weight_dtype,
                                 int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                                 const float* bias, const float* residual, float* y,
                                 void* stream);

/* The same three projections for `rows` tokens on the matrix cores, for long
 * prompts.  With gamma, the inputs are first normalised into `normalized`
 * (rows * in_dim floats, as in the rows variants).  Each input value v is
 * split into bf16 parts hi = bf16(v) and lo = bf16(v - hi), and each output
 * is W hi + W lo with fp32 accumulation: every product is exact and v keeps
 * ~16 significant bits (the lo part is itself rounded to bf16: a relative
 * error up to ~2^-16 per input, against fp32's 2^-24), so the results agree
 * with the one-token entry points within that bound, not bit for bit.  RoPE, bias, SwiGLU
 * and the residual are applied as in the rows variants (y may alias
 * residual).  SKV_ERR_UNSUPPORTED (nothing launched) unless the weights are
 * bf16 aligned output-major rows, in_dim is a multiple of 128 from 512 to
 * 8,192, every output count is a multiple of 32 (gate/up: 16), head_dim is a
 * multiple of 32 when rotating, and the input (the normalised rows with
 * gamma), outputs and residual are 16-byte aligned.
 * Replaces: the same reference code as the rows variants
 * (src/models/transformer_block.cpp:300-332); no counterpart of its own. */
int skv_fused_qkv_mm_f32(const float* hidden, int rows, const float* gamma, float epsilon,
                         const void* wq, const void* wk, const void* wv, int weight_dtype,
                         int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                         const float* bias_k, const float* bias_v, int hidden_dim,
                         int num_heads, int num_kv_heads, int head_dim, int first_position,
                         float* q, float* k, float* v, float* normalized, void* stream);
int skv_fused_gate_up_swiglu_mm_f32(const float* x, int rows, const float* gamma, float epsilon,
                                    const void* w_gate, const void* w_up, int weight_dtype,
                                    int64_t stride_k, int64_t stride_n_gate,
                                    int64_t stride_n_up, const float* bias_gate,
                                    const float* bias_up, int in_dim, int out_dim,
                                    float* act, float* normalized, void* stream);
int skv_linear_residual_mm_f32(const float* x, int rows, const void* weight, int weight_dtype,
                               int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                               const float* bias, const float* residual, float* y,
                               void* stream);

/* The same projections with their products as hipBLASLt GEMMs, for long
 * prompts (skv_*_gemm_f32), are declared in stratakv_amd_gemm.h and exported
 * by libstratakv_amd_gemm.so, the only library of this build that links
 * hipBLASLt. */

/* ---- model boundary: checkpoint tensors, embedding, token choice --------
 * Checkpoint decode on the device (the host only moves file bytes).  src holds
 * `count` little-endian elements of src_dtype (SKV_DTYPE_BF16 / F16 / FP32).
 * skv_convert_to_bf16: dst = the upper 16 bits of the exact fp32 value (BF16
 *   copied, F16 widened exactly then truncated, FP32 truncated), the rule of
 *   load_linear_bf16_transposed and convert_fp32_to_bf16_cuda
 *   (src/io/safetensors.cpp:610-681, src/cuda/gemm_cuda.cu:74-83).
 * skv_convert_to_f32: dst = the exact fp32 value (src/io/safetensors.cpp:98-104,
 *   :219-250 for F16).
 * skv_check_finite: no output.
 * When nonfinite is not NULL, *nonfinite |= 1 if any element is NaN or
 * infinite (the check behind the reference's "Non-finite weight" error,
 * src/generation/generator.cpp:265-290). */
int skv_convert_to_bf16(const void* src, int src_dtype, size_t count, uint16_t* dst,
                        int32_t* nonfinite, void* stream);
int skv_convert_to_f32(const void* src, int src_dtype, size_t count, float* dst,
                       int32_t* nonfinite, void* stream);
int skv_check_finite(const void* src, int src_dtype, size_t count, int32_t* nonfinite,
                     void* stream);

/* out[i] = table[token_ids[index] * hidden + i] as fp32 (exact widening of a
 * BF16 / F16 table).  The id is read on the device; an id outside [0, vocab)
 * writes zeros and sets SKV_FLAG_BAD_TOKEN in *flags (flags may be NULL).
 * Replaces: embedding_lookup_cuda (src/cuda/gemm_cuda.cu:286-300,900-912). */
int skv_embedding_f32(const void* table, int table_dtype, int vocab, int hidden,
                      const int32_t* token_ids, int index, float* out, int32_t* flags,
                      void* stream);
/* The same for `rows` consecutive ids (a prompt): out[r][i] =
 * table[token_ids[first_index + r] * hidden + i], r < rows <= 65,535, in one
 * launch. */
int skv_embedding_rows_f32(const void* table, int table_dtype, int vocab, int hidden,
                           const int32_t* token_ids, int first_index, int rows, float* out,
                           int32_t* flags, void* stream);
/* skv_embedding_f32 with the index held in device memory (*index_at) and the
 * flag word flags[*flag_at] (flag_at NULL: flags[0]), for a decode step
 * captured once in a HIP graph and replayed per token.  No counterpart in the
 * reference. */
int skv_embedding_at_f32(const void* table, int table_dtype, int vocab, int hidden,
                         const int32_t* token_ids, const int32_t* index_at, float* out,
                         int32_t* flags, const int32_t* flag_at, void* stream);

/* token_ids[index] = the first index of the maximum of logits[0..n) (greedy,
 * src/generation/sampler.cpp:57-62).  A non-finite logit sets
 * SKV_FLAG_NONFINITE_LOGITS.  Replaces the logits download + host argmax of
 * the reference's generate loop (src/generation/generator.cpp:700-735). */
int skv_argmax_f32(const float* logits, int n, int32_t* token_ids, int index,
                   int32_t* flags, void* stream);
/* skv_argmax_f32 writing token_ids[*index_at] and flagging flags[*flag_at]
 * (flag_at NULL: flags[0]), both indices in device memory, for a decode step
 * captured once in a HIP graph and replayed per token.  No counterpart in the
 * reference. */
int skv_argmax_at_f32(const float* logits, int n, int32_t* token_ids, const int32_t* index_at,
                      int32_t* flags, const int32_t* flag_at, void* stream);

/* token_ids[index] = Sampler::sample(logits) (src/generation/sampler.cpp:43-147):
 * temperature 0 -> greedy as skv_argmax_f32; otherwise logits / temperature,
 * top-k (0 = off), top-p (1 = off), softmax of what is kept, and the
 * categorical draw of std::discrete_distribution for the uniform `uniform`
 * in [0, 1), which the caller draws as generate_canonical<double, 53> from the
 * sampler's mt19937 (one draw per call with temperature > 0 and n >= 2).
 * Configuration errors return SKV_ERR_INVALID_ARGUMENT with the reference's
 * messages; data errors set SKV_FLAG_NONFINITE_LOGITS / _NONFINITE_SCALED /
 * _BAD_DISTRIBUTION in *flags and write token 0.  Masses are summed in double
 * in a different order than the reference's float loops, so the chosen token
 * can differ only where `uniform` or top_p falls within rounding of a
 * cumulative boundary. */
int skv_sample_f32(const float* logits, int n, float temperature, int top_k, float top_p,
                   double uniform, int32_t* token_ids, int index, int32_t* flags,
                   void* stream);

/* ---- test support --------------------------------------------------------
 * Copy the blocks listed in table[0..num_blocks) of a pool into a contiguous
 * device buffer dst[num_blocks][block_elems] (so one sequence can be read back
 * without copying a whole pool).  Entries outside [0, total_blocks) give
 * zero-filled blocks. */
int skv_gather_blocks(const uint16_t* pool, int64_t total_blocks,
                      const int32_t* table, int num_blocks,
                      int64_t block_elems, uint16_t* dst, void* stream);

/* Copy `count` chunks of `chunk_bytes` bytes (a multiple of 16; every pointer
 * 16-byte aligned, no chunk overlapping another's destination): chunk i from
 * src[i] to dst[i].  src and dst are device arrays of `count` device pointers;
 * count up to 65,535.  One launch.  The Generator saves the K/V blocks a
 * generation will write with it and puts them back afterwards.
 * Replaces: the deep copies of every pool that the reference's SequenceGuard
 * makes and restores (src/generation/generator.cpp:347-371, the BlockPool
 * copy constructor src/memory/block_pool.cpp:118-145). */
int skv_copy_chunks(const void* const* src, void* const* dst, int count, size_t chunk_bytes, void* stream);

/* ---- HIP graphs of recorded launches ----------------------------------------
 * For a sequence of launches replayed many times with the same arguments (the
 * greedy decode step of Generator, whose per-token values live in device
 * memory).  skv_graph_begin_capture starts recording the launches queued on
 * `stream` (a created stream, not the null stream; launches from this thread
 * only); skv_graph_end_capture stops and instantiates them into *graph_exec;
 * skv_graph_abort_capture stops and discards a recording (after a failed
 * launch); skv_graph_launch queues one replay on any stream; skv_graph_destroy
 * frees an instantiated graph (NULL: nothing).  Nothing recorded may be a
 * memset.  No counterpart in the reference. */
int skv_graph_begin_capture(void* stream);
int skv_graph_end_capture(void* stream, void** graph_exec);
int skv_graph_abort_capture(void* stream);
int skv_graph_launch(void* graph_exec, void* stream);
int skv_graph_destroy(void* graph_exec);

/* ---- measurement ----------------------------------------------------------
 * Load-pattern calibration of skv_paged_decode: the MFMA decode kernel's K/V
 * reads (the same grid for this geometry, the same block order per
 * wavefront, the same buffer loads and cache hints) with the attention math
 * replaced by a checksum.  checksums[b * num_kv_heads + h] (device,
 * [num_seqs][num_kv_heads] uint32) receives the wrapping 32-bit sum of the
 * 32-bit words of the head-h slice of all block_size rows of K and of V in the
 * first min(ceil(context_lens[b] / block_size), max_blocks_per_seq) blocks of
 * sequence b's table (an entry outside [0, total_blocks) adds 0).  Its
 * duration is the rate the decode's loads alone reach: the ceiling the decode
 * kernel is measured against.  The geometry of the MFMA decode path only
 * (block_size 16, head_dim 64 or 128, num_q_heads / num_kv_heads in
 * {1, 2, 4, 8, 16}, 16-byte aligned pools), at most 4096 sequences; other
 * shapes give SKV_ERR_UNSUPPORTED.  No counterpart in the reference. */
int skv_paged_block_checksum(const uint16_t* k_pool, const uint16_t* v_pool,
                             int64_t total_blocks, const int32_t* block_tables,
                             int max_blocks_per_seq, const int32_t* context_lens,
                             int num_seqs, int num_q_heads, int num_kv_heads,
                             int head_dim, int block_size, uint32_t* checksums,
                             void* stream);

/* Streaming-read calibration: reads `bytes` bytes at `data` (device, 16-byte
 * aligned, a positive multiple of 16) once, with the non-temporal 16-byte
 * loads the decode uses, from a persistent grid of wavefronts taking 4 MiB
 * chunks in turn, and writes the wrapping 32-bit sum of its 32-bit words to
 * *checksum (device).  Its duration gives the rate plain reads reach on this
 * GPU, beside the decode's own load pattern (skv_paged_block_checksum).
 * Clears *checksum with an asynchronous memset first (not for graph
 * capture).  No counterpart in the reference. */
int skv_stream_read_checksum(const void* data, int64_t bytes, uint32_t* checksum, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STRATAKV_AMD_H */

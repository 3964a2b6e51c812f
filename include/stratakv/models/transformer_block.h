// transformer_block.h -- one Llama decoder layer; forward_into is the GPU
// decode step of one token of one sequence, the drop-in boundary of the paged
// KV-cache path.
//
// Interface of the reference's stratakv::models::TransformerBlock
// (include/stratakv/models/transformer_block.h:13-103).  to(Device::GPU)
// moves the parameters and allocates the persistent scratchpads once (the
// reference's 11 FP32 workspaces plus the decode workspace); forward_into
// never allocates.  Sub-steps (src/models/transformer_block.cpp:334-613):
// rmsnorm, q/k/v projections, split-half RoPE at the token's position,
// PageTable::append_token, the KV append of the rotated K and V rows into the
// bf16 pools (skv_kv_append_token), the device block table, paged decode
// attention (skv_paged_attention_decode), o_proj + residual, rmsnorm,
// gate/up, SwiGLU, down + residual, and the final copy that keeps
// hidden_states/output aliasing safe.  All device work is queued on one
// stream (the null stream by default, as the reference's legacy stream).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>

#include "stratakv/layers/attention.h"
#include "stratakv/layers/linear.h"
#include "stratakv/layers/rmsnorm.h"

namespace stratakv {
namespace models {

class TransformerBlock {
public:
    TransformerBlock(std::size_t hidden_dim, std::size_t intermediate_dim, std::size_t num_heads,
                     int total_blocks, int block_size, Device device = Device::CPU);
    TransformerBlock(std::size_t hidden_dim, std::size_t intermediate_dim, std::size_t num_heads,
                     std::size_t num_kv_heads, int total_blocks, int block_size,
                     Device device = Device::CPU);

    TransformerBlock(const TransformerBlock&) = delete;
    TransformerBlock& operator=(const TransformerBlock&) = delete;
    TransformerBlock(TransformerBlock&&) noexcept = default;
    TransformerBlock& operator=(TransformerBlock&&) noexcept = default;
    ~TransformerBlock() = default;

    void to(Device device);
    // For the STRATAKV_PARITY diagnostic (the reference's per-op report of
    // layer 0, src/models/transformer_block.cpp:405-595): row `row` of the
    // values the last forward_into (row 0) or prefill_into chunk left in this
    // block's scratch, copied to the host after the stream drains -- q and k
    // after RoPE, v, the attention context, the residual stream after
    // o_proj, and the SwiGLU activations.  The fused kernels write no other
    // intermediate (the normalised rows, q and k before RoPE, gate and up
    // stay in registers).  A prefill scratch shared by several blocks holds
    // the last block's rows.  No counterpart in the reference.
    struct ParityRow {
        std::vector<float> q, k, v, context, residual, act;
    };
    ParityRow parity_row(int row) const;
    // Stream for the device work of forward_into (a hipStream_t; nullptr =
    // the default stream).
    void set_stream(void* stream) noexcept { stream_ = stream; }

    // GPU tensors: allocates the result and runs forward_into.  CPU tensors:
    // the reference's CPU path, not provided by this build (throws).
    Tensor forward(const Tensor& hidden_states, int seq_id, memory::PageTable& page_table,
                   memory::BlockPool& block_pool, bool append_tokens = true);
    // Runs the layer over hidden_states.shape()[0] new tokens of seq_id (a
    // prompt, or a chunk of one), GPU only: appends their K/V at the next
    // positions and attends causally over the whole context
    // (skv_paged_prefill); output may alias hidden_states.  The reference's
    // GPU forward_into takes one token (src/models/transformer_block.cpp:
    // 348-351); its CPU forward computes these rows (:300-332).  Chunks of
    // fewer than kPrefillMmRows tokens give every projection row the bits
    // forward_into gives for that token; longer ones (bf16 weights) run the
    // projections on the matrix cores (from kPrefillGemmRows tokens as
    // hipBLASLt GEMMs): their inputs keep ~16 significant bits (hi + lo bf16
    // parts, a relative error up to ~2^-16 each), so those rows agree with
    // forward_into within that bound, not bit for bit.  The attention
    // of the chunk runs the prefill kernel instead of the decode kernel.
    void prefill_into(const Tensor& hidden_states, Tensor& output, int seq_id,
                      memory::PageTable& page_table, memory::BlockPool& block_pool);
    // Tokens per prefill_into pass: longer inputs run in chunks of
    // prefill_chunk_rows() tokens, as many as kPrefillChunk and the scratch
    // budget allow (never fewer than kPrefillMinChunk).  Long chunks give the
    // projections and the attention large grids.
    static constexpr int kPrefillChunk = 2048;
    static constexpr int kPrefillMinChunk = 256;
    // Bytes of prefill scratch: the fp32 rows of a chunk plus the library
    // GEMMs' workspace for the projections they take.
    static constexpr std::size_t kPrefillScratchBudget = std::size_t{1} << 30;
    int prefill_chunk_rows() const noexcept;
    // Chunk length from which the projections run on the matrix cores.
    static constexpr int kPrefillMmRows = 32;
    // Chunk length from which the projections run as hipBLASLt GEMMs
    // (skv_*_gemm_f32, libstratakv_amd_gemm.so, when it can be opened): the
    // same hi + lo split as the matrix-core kernels, different summation order.
    static constexpr int kPrefillGemmRows = 256;
    // prefill_into's scratch: the chunk's q, k, v, context, residual,
    // activation and normalised rows, its metadata and the library GEMMs'
    // workspace (skv_prompt_gemm_workspace_bytes).  Blocks of one shape that
    // run one after another on one stream (a Generator's layers) may share
    // one; a block with none allocates its own on first use.  Buffers are
    // grown on demand and re-made when a block of another shape uses them.
    struct PrefillScratch {
        int rows = 0;
        std::size_t dims[4] = {0, 0, 0, 0};   // hidden, q, kv, intermediate
        std::optional<Tensor> queries, keys, values, context, residual, act, normalized, up, down, meta, gemm;
    };
    void share_prefill_scratch(std::shared_ptr<PrefillScratch> scratch) noexcept { pf_ = std::move(scratch); }
    void forward_into(const Tensor& hidden_states, Tensor& output, int seq_id,
                      memory::PageTable& page_table, memory::BlockPool& block_pool,
                      bool append_tokens = true);

    // One decode token at a position held in device memory, for a decode step
    // captured once in a HIP graph and replayed per token (Generator's greedy
    // loop).  step[0] is the token's position and step[1] the context length
    // (position + 1), both device int32; rope_cos_sin is the
    // [rope_positions][head_dim] table of skv_rope_cos_sin.  The caller has
    // already done the host bookkeeping forward_into does: appended the token
    // to the sequence's PageTable and uploaded its device block table, whose
    // stable device pointer and capacity (row length) are passed here.  The
    // same kernels as forward_into on bf16 or fp32 output-major weights, so with
    // equal inputs the outputs are equal to forward_into's bits whenever the
    // attention takes the same path (a table capacity of at most 16 blocks).
    // Returns false, having launched nothing, when a projection's weights are
    // not in the fused kernels' layout (forward_into then runs separate kernels).
    // No counterpart in the reference.
    bool forward_into_at(const Tensor& hidden_states, Tensor& output, const std::int32_t* step,
                         const float* rope_cos_sin, int rope_positions, const int* device_table,
                         int table_capacity, memory::BlockPool& block_pool);

    std::size_t last_attention_blocks_visited() const noexcept {
        return attention_.last_blocks_visited();
    }

    layers::RMSNorm& input_norm() noexcept { return norm1_; }
    const layers::RMSNorm& input_norm() const noexcept { return norm1_; }
    layers::PagedAttention& attention() noexcept { return attention_; }
    const layers::PagedAttention& attention() const noexcept { return attention_; }
    layers::RMSNorm& post_attention_norm() noexcept { return norm2_; }
    const layers::RMSNorm& post_attention_norm() const noexcept { return norm2_; }
    layers::Linear& gate_projection() noexcept { return gate_proj_; }
    const layers::Linear& gate_projection() const noexcept { return gate_proj_; }
    layers::Linear& up_projection() noexcept { return up_proj_; }
    const layers::Linear& up_projection() const noexcept { return up_proj_; }
    layers::Linear& down_projection() noexcept { return down_proj_; }
    const layers::Linear& down_projection() const noexcept { return down_proj_; }
    layers::Linear& gate_proj() noexcept { return gate_proj_; }
    const layers::Linear& gate_proj() const noexcept { return gate_proj_; }
    layers::Linear& up_proj() noexcept { return up_proj_; }
    const layers::Linear& up_proj() const noexcept { return up_proj_; }
    layers::Linear& down_proj() noexcept { return down_proj_; }
    const layers::Linear& down_proj() const noexcept { return down_proj_; }

private:
    std::size_t hidden_dim_;
    layers::RMSNorm norm1_;
    layers::PagedAttention attention_;
    layers::RMSNorm norm2_;
    layers::Linear gate_proj_;
    layers::Linear up_proj_;
    layers::Linear down_proj_;
    bool last_pass_prefill_ = false;   // which scratch parity_row reads
    void* stream_ = nullptr;
    // Persistent GPU scratchpads, allocated by to(Device::GPU) and reused by
    // every forward_into; a block serves one request at a time.
    std::optional<Tensor> normalized_input_workspace_;
    std::optional<Tensor> query_workspace_;
    std::optional<Tensor> key_workspace_;
    std::optional<Tensor> value_workspace_;
    std::optional<Tensor> context_workspace_;
    std::optional<Tensor> normalized_residual_workspace_;
    std::optional<Tensor> gate_workspace_;
    std::optional<Tensor> up_workspace_;
    std::optional<Tensor> down_workspace_;
    std::optional<Tensor> decode_workspace_;  // skv_paged_attention_decode scratch
    // prefill_into scratch, [rows][dim] for up to pf_->rows tokens (allocated
    // on first use, grown to prefill_chunk_rows() at most; up and down only
    // when the separate-kernel fallback runs).
    void ensure_prefill_workspace(int rows);
    std::shared_ptr<PrefillScratch> pf_;
    // The shared workspace grown to at least `bytes`; its 256-byte aligned start.
    void* prefill_gemm_workspace(std::size_t bytes);
    // Which projections of a chunk of `rows` tokens go to the library GEMMs
    // (libstratakv_amd_gemm.so opened, rows >= kPrefillGemmRows, and the
    // layout rules the entry points check on the weights: bf16, in_dim a
    // multiple of 8 up to 8,192), and the workspace those take.
    struct PrefillGemmUse {
        bool qkv = false, o = false, ffn = false, gate_up = false, down = false;
        std::size_t bytes = 0;
    };
    PrefillGemmUse prefill_gemm_use(int rows) const noexcept;
};

}  // namespace models
}  // namespace stratakv

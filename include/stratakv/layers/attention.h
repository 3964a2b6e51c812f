// attention.h -- the attention layer's parameters and geometry.
//
// Mirrors the reference's stratakv::layers::PagedAttention
// (include/stratakv/layers/attention.h:14-93) as the holder of the q/k/v/o
// projections and the (num_heads, num_kv_heads, head_dim) geometry that
// TransformerBlock uses.  In this build the KV cache lives in BlockPool's
// device pools and the decode runs through TransformerBlock::forward_into;
// the reference's CPU multi-token forward (its private FP32 cache) is not
// part of this build and throws.
#pragma once

#include <cstddef>

#include "stratakv/layers/linear.h"
#include "stratakv/memory/block_pool.h"
#include "stratakv/memory/page_table.h"

namespace stratakv {
namespace models {
class TransformerBlock;
}
namespace layers {

class PagedAttention {
public:
    PagedAttention(std::size_t hidden_dim, std::size_t num_heads, int total_blocks, int block_size,
                   Device device = Device::CPU);
    PagedAttention(std::size_t hidden_dim, std::size_t num_heads, std::size_t num_kv_heads,
                   int total_blocks, int block_size, Device device = Device::CPU);

    PagedAttention(const PagedAttention&) = delete;
    PagedAttention& operator=(const PagedAttention&) = delete;
    PagedAttention(PagedAttention&&) noexcept = default;
    PagedAttention& operator=(PagedAttention&&) noexcept = default;
    ~PagedAttention() = default;

    // The reference's CPU path; not provided by this build (throws).
    Tensor forward(const Tensor& hidden_states, int seq_id, memory::PageTable& page_table,
                   memory::BlockPool& block_pool, bool append_tokens = true);
    // Distinct pool blocks the last attention read (src/layers/attention.cpp:
    // 230-232, 291-296, where only the CPU forward counts them).  Here
    // TransformerBlock::forward_into and prefill_into set it: the blocks of
    // the sequence's context.  Replayed graph steps (forward_into_at) leave it.
    std::size_t last_blocks_visited() const noexcept { return last_blocks_visited_; }

    Linear& query_projection() noexcept { return q_proj_; }
    const Linear& query_projection() const noexcept { return q_proj_; }
    Linear& key_projection() noexcept { return k_proj_; }
    const Linear& key_projection() const noexcept { return k_proj_; }
    Linear& value_projection() noexcept { return v_proj_; }
    const Linear& value_projection() const noexcept { return v_proj_; }
    Linear& output_projection() noexcept { return out_proj_; }
    const Linear& output_projection() const noexcept { return out_proj_; }
    Device device() const noexcept { return device_; }
    std::size_t num_heads() const noexcept { return num_heads_; }
    std::size_t num_kv_heads() const noexcept { return num_kv_heads_; }
    std::size_t head_dim() const noexcept { return head_dim_; }
    int total_blocks() const noexcept { return total_blocks_; }
    int block_size() const noexcept { return block_size_; }

private:
    std::size_t hidden_dim_;
    std::size_t num_heads_;
    std::size_t num_kv_heads_;
    std::size_t head_dim_;
    int total_blocks_;
    int block_size_;
    Device device_;
    Linear q_proj_;
    Linear k_proj_;
    Linear v_proj_;
    Linear out_proj_;
    std::size_t last_blocks_visited_ = 0;
    friend class models::TransformerBlock;   // sets last_blocks_visited_
};

}  // namespace layers
}  // namespace stratakv

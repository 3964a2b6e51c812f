// block_pool.h -- physical KV block allocator with bf16 device storage.
//
// Interface of the reference's stratakv::memory::BlockPool
// (include/stratakv/memory/block_pool.h:28-87): a LIFO free list of block
// ids (the constructor pushes total-1 ... 0, so block 0 is handed out
// first), allocate_block() throwing std::runtime_error("OOM") when empty, and
// in GPU mode the K and V pools [total][block_size][num_kv_heads][head_dim].
// The one intended change: the pools hold bf16 (std::uint16_t bit patterns)
// instead of float, so key_cache()/value_cache() return std::uint16_t*.
// Storage is allocated through the C ABI (skv_malloc) and left uninitialised,
// like cudaMalloc in the reference.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <vector>

#include "stratakv/tensor.h"

namespace stratakv {
namespace memory {

class BlockPool {
public:
    BlockPool(int total, int blk_sz);
    BlockPool(int total, int blk_sz, int num_kv_heads, int head_dim, Device device = Device::CPU);
    BlockPool(int total, int blk_sz, Device device, int num_kv_heads, int head_dim);

    // Copies deep-copy the device pools (device to device), as the reference does.
    BlockPool(const BlockPool& other);
    BlockPool& operator=(const BlockPool& other);
    BlockPool(BlockPool&& other) noexcept;
    BlockPool& operator=(BlockPool&& other) noexcept;
    ~BlockPool() noexcept;

    // Pop the most recently freed (or lowest initial) block id; throws
    // std::runtime_error("OOM") when the pool is exhausted.
    int allocate_block();
    // Push a block id back.  Out-of-range ids and double frees (undefined in
    // the reference) throw std::invalid_argument here.
    void free_block(int block_id);

    std::size_t free_count() const noexcept { return free_list_.size(); }
    // Extension: the free stack (back() is handed out next), and putting a
    // saved one back.  Generator uses them as the reference's SequenceGuard
    // uses a pool copy (src/generation/generator.cpp:347-371), without
    // copying the KV storage: after a generation the free list, and so the
    // block ids of the next one, are what they were before it.  restore
    // throws std::invalid_argument for an id out of range or listed twice.
    const std::vector<int>& free_list() const noexcept { return free_list_; }
    void restore_free_list(const std::vector<int>& ids);
    int block_size() const noexcept { return block_size_; }
    int total_blocks() const noexcept { return total_blocks_; }
    int num_kv_heads() const noexcept { return num_kv_heads_; }
    int head_dim() const noexcept { return head_dim_; }
    Device device() const noexcept { return device_; }
    std::uint16_t* key_cache() noexcept { return key_cache_; }
    std::uint16_t* value_cache() noexcept { return value_cache_; }
    const std::uint16_t* key_cache() const noexcept { return key_cache_; }
    const std::uint16_t* value_cache() const noexcept { return value_cache_; }
    // Elements of one block of one pool: block_size * num_kv_heads * head_dim.
    std::size_t block_elements() const noexcept {
        return static_cast<std::size_t>(block_size_) * static_cast<std::size_t>(num_kv_heads_) *
               static_cast<std::size_t>(head_dim_);
    }

private:
    void initialize_storage();
    void release_storage() noexcept;

    int total_blocks_;
    int block_size_;
    int num_kv_heads_ = 0;
    int head_dim_ = 0;
    Device device_ = Device::CPU;
    std::uint16_t* key_cache_ = nullptr;
    std::uint16_t* value_cache_ = nullptr;
    std::vector<int> free_list_;          // stack: back() is handed out next
    std::vector<unsigned char> is_free_;  // double-free detection
};

}  // namespace memory
}  // namespace stratakv

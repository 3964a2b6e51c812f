// block_pool.cpp -- LIFO block-id allocator and bf16 device K/V pools.
// Behaviour follows src/memory/block_pool.cpp of the reference: the
// constructor pushes total-1 ... 0 (block 0 is handed out first, lines
// 72-76), allocate_block pops or throws "OOM" (193-200), free_block pushes
// (205-207), copies deep-copy the device pools (118-145).
#include "stratakv/memory/block_pool.h"

#include <limits>
#include <string>
#include <utility>

#include "abi_check.h"

namespace stratakv {
namespace memory {
namespace {

std::size_t pool_bytes(int total, int block_size, int num_kv_heads, int head_dim) {
    if (total <= 0 || block_size <= 0 || num_kv_heads <= 0 || head_dim <= 0)
        throw std::invalid_argument("BlockPool: GPU storage dimensions must be positive");
    const std::size_t elems = static_cast<std::size_t>(total) * static_cast<std::size_t>(block_size) *
                              static_cast<std::size_t>(num_kv_heads) *
                              static_cast<std::size_t>(head_dim);
    if (elems > std::numeric_limits<std::size_t>::max() / sizeof(std::uint16_t))
        throw std::overflow_error("BlockPool: KV storage size overflow");
    return elems * sizeof(std::uint16_t);
}

}  // namespace

BlockPool::BlockPool(int total, int blk_sz) : BlockPool(total, blk_sz, 0, 0, Device::CPU) {}

BlockPool::BlockPool(int total, int blk_sz, int num_kv_heads, int head_dim, Device device)
    : total_blocks_(total),
      block_size_(blk_sz),
      num_kv_heads_(num_kv_heads),
      head_dim_(head_dim),
      device_(device) {
    if (total <= 0) throw std::invalid_argument("BlockPool: total must be > 0");
    if (blk_sz <= 0) throw std::invalid_argument("BlockPool: block_size must be > 0");
    if (device_ == Device::GPU && (num_kv_heads_ <= 0 || head_dim_ <= 0))
        throw std::invalid_argument("BlockPool: GPU mode requires positive KV dimensions");
    free_list_.reserve(static_cast<std::size_t>(total));
    for (int id = total - 1; id >= 0; --id) free_list_.push_back(id);
    is_free_.assign(static_cast<std::size_t>(total), 1);
    initialize_storage();
}

BlockPool::BlockPool(int total, int blk_sz, Device device, int num_kv_heads, int head_dim)
    : BlockPool(total, blk_sz, num_kv_heads, head_dim, device) {}

void BlockPool::initialize_storage() {
    if (device_ != Device::GPU) return;
    const std::size_t bytes = pool_bytes(total_blocks_, block_size_, num_kv_heads_, head_dim_);
    void* k = nullptr;
    void* v = nullptr;
    detail::check(skv_malloc(&k, bytes), "BlockPool: key pool allocation");
    const int rc = skv_malloc(&v, bytes);
    if (rc != SKV_OK) {
        (void)skv_free(k);
        detail::check(rc, "BlockPool: value pool allocation");
    }
    key_cache_ = static_cast<std::uint16_t*>(k);
    value_cache_ = static_cast<std::uint16_t*>(v);
}

void BlockPool::release_storage() noexcept {
    if (key_cache_ != nullptr) (void)skv_free(key_cache_);
    if (value_cache_ != nullptr) (void)skv_free(value_cache_);
    key_cache_ = nullptr;
    value_cache_ = nullptr;
}

BlockPool::BlockPool(const BlockPool& other)
    : total_blocks_(other.total_blocks_),
      block_size_(other.block_size_),
      num_kv_heads_(other.num_kv_heads_),
      head_dim_(other.head_dim_),
      device_(other.device_),
      free_list_(other.free_list_),
      is_free_(other.is_free_) {
    initialize_storage();
    if (device_ == Device::GPU) {
        const std::size_t bytes = pool_bytes(total_blocks_, block_size_, num_kv_heads_, head_dim_);
        try {
            detail::check(skv_memcpy_d2d(key_cache_, other.key_cache_, bytes, nullptr), "BlockPool copy");
            detail::check(skv_memcpy_d2d(value_cache_, other.value_cache_, bytes, nullptr), "BlockPool copy");
            detail::check(skv_stream_synchronize(nullptr), "BlockPool copy");
        } catch (...) {
            release_storage();
            throw;
        }
    }
}

BlockPool& BlockPool::operator=(const BlockPool& other) {
    if (this == &other) return *this;
    BlockPool copy(other);
    *this = std::move(copy);
    return *this;
}

BlockPool::BlockPool(BlockPool&& other) noexcept
    : total_blocks_(other.total_blocks_),
      block_size_(other.block_size_),
      num_kv_heads_(other.num_kv_heads_),
      head_dim_(other.head_dim_),
      device_(other.device_),
      key_cache_(std::exchange(other.key_cache_, nullptr)),
      value_cache_(std::exchange(other.value_cache_, nullptr)),
      free_list_(std::move(other.free_list_)),
      is_free_(std::move(other.is_free_)) {}

BlockPool& BlockPool::operator=(BlockPool&& other) noexcept {
    if (this == &other) return *this;
    release_storage();
    total_blocks_ = other.total_blocks_;
    block_size_ = other.block_size_;
    num_kv_heads_ = other.num_kv_heads_;
    head_dim_ = other.head_dim_;
    device_ = other.device_;
    key_cache_ = std::exchange(other.key_cache_, nullptr);
    value_cache_ = std::exchange(other.value_cache_, nullptr);
    free_list_ = std::move(other.free_list_);
    is_free_ = std::move(other.is_free_);
    return *this;
}

BlockPool::~BlockPool() noexcept { release_storage(); }

int BlockPool::allocate_block() {
    if (free_list_.empty()) throw std::runtime_error("OOM");
    const int id = free_list_.back();
    free_list_.pop_back();
    is_free_[static_cast<std::size_t>(id)] = 0;
    return id;
}

void BlockPool::free_block(int block_id) {
    if (block_id < 0 || block_id >= total_blocks_)
        throw std::invalid_argument("BlockPool::free_block: block " + std::to_string(block_id) +
                                    " is outside the pool");
    if (is_free_[static_cast<std::size_t>(block_id)])
        throw std::invalid_argument("BlockPool::free_block: block " + std::to_string(block_id) +
                                    " is already free");
    is_free_[static_cast<std::size_t>(block_id)] = 1;
    free_list_.push_back(block_id);
}

}  // namespace memory
}  // namespace stratakv

namespace stratakv {
namespace memory {

void BlockPool::restore_free_list(const std::vector<int>& ids) {
    std::vector<unsigned char> seen(static_cast<std::size_t>(total_blocks_), 0);
    for (int id : ids) {
        if (id < 0 || id >= total_blocks_ || seen[static_cast<std::size_t>(id)])
            throw std::invalid_argument("BlockPool::restore_free_list: invalid or repeated block id " +
                                        std::to_string(id));
        seen[static_cast<std::size_t>(id)] = 1;
    }
    free_list_ = ids;
    is_free_ = std::move(seen);
}

}  // namespace memory
}  // namespace stratakv

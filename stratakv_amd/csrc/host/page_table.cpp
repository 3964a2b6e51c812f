// page_table.cpp -- sequence -> block mapping (reference semantics of
// src/memory/page_table.cpp:107-178) and device-resident block tables.
#include "stratakv/memory/page_table.h"

#include <algorithm>
#include <atomic>
#include <limits>
#include <string>
#include <utility>

#include "abi_check.h"

namespace stratakv {
namespace memory {
namespace {

std::uint64_t next_generation() noexcept {
    static std::atomic<std::uint64_t> counter{0};
    return ++counter;
}

SequenceState& checked_lookup(std::unordered_map<int, SequenceState>& table, int seq_id,
                              const char* caller) {
    auto it = table.find(seq_id);
    if (it == table.end())
        throw std::runtime_error(std::string(caller) + ": unknown seq_id=" + std::to_string(seq_id));
    return it->second;
}

}  // namespace

PageTable::PageTable(const PageTable& other) : table_(other.table_) {}

PageTable& PageTable::operator=(const PageTable& other) {
    if (this != &other) {
        release_device_block_table();
        table_ = other.table_;
    }
    return *this;
}

PageTable::PageTable(PageTable&& other) noexcept
    : table_(std::move(other.table_)),
      d_block_table_(std::exchange(other.d_block_table_, nullptr)),
      h_block_table_(std::exchange(other.h_block_table_, nullptr)),
      d_block_table_capacity_(std::exchange(other.d_block_table_capacity_, 0)),
      staged_seq_id_(other.staged_seq_id_),
      staged_block_count_(std::exchange(other.staged_block_count_, 0)),
      device_table_dirty_(std::exchange(other.device_table_dirty_, true)),
      upload_event_(std::exchange(other.upload_event_, nullptr)),
      upload_stream_(std::exchange(other.upload_stream_, nullptr)) {}

PageTable& PageTable::operator=(PageTable&& other) noexcept {
    if (this != &other) {
        release_device_block_table();
        table_ = std::move(other.table_);
        d_block_table_ = std::exchange(other.d_block_table_, nullptr);
        h_block_table_ = std::exchange(other.h_block_table_, nullptr);
        d_block_table_capacity_ = std::exchange(other.d_block_table_capacity_, 0);
        staged_seq_id_ = other.staged_seq_id_;
        staged_block_count_ = std::exchange(other.staged_block_count_, 0);
        device_table_dirty_ = std::exchange(other.device_table_dirty_, true);
        upload_event_ = std::exchange(other.upload_event_, nullptr);
        upload_stream_ = std::exchange(other.upload_stream_, nullptr);
    }
    return *this;
}

PageTable::~PageTable() noexcept { release_device_block_table(); }

void PageTable::release_device_block_table() noexcept {
    // Queued kernels and copies may still use the table and its mirror.
    if (d_block_table_ != nullptr || h_block_table_ != nullptr) (void)skv_device_synchronize();
    if (d_block_table_ != nullptr) (void)skv_free(d_block_table_);
    if (h_block_table_ != nullptr) (void)skv_host_free(h_block_table_);
    if (upload_event_ != nullptr) (void)skv_event_destroy(upload_event_);
    d_block_table_ = nullptr;
    h_block_table_ = nullptr;
    upload_event_ = nullptr;
    upload_stream_ = nullptr;
    d_block_table_capacity_ = 0;
    staged_block_count_ = 0;
    device_table_dirty_ = true;
}

void PageTable::allocate_sequence(int seq_id, BlockPool& pool) {
    if (table_.count(seq_id))
        throw std::runtime_error("allocate_sequence: seq_id=" + std::to_string(seq_id) +
                                 " already exists");
    SequenceState state;
    state.physical_blocks.push_back(pool.allocate_block());  // the first block, eagerly
    state.generation = next_generation();
    table_.emplace(seq_id, std::move(state));
    device_table_dirty_ = true;
}

void PageTable::append_token(int seq_id, BlockPool& pool) {
    SequenceState& state = checked_lookup(table_, seq_id, "append_token");
    if (state.sequence_length == std::numeric_limits<int>::max())
        throw std::overflow_error("append_token: sequence length exceeds int range");
    const std::size_t capacity =
        state.physical_blocks.size() * static_cast<std::size_t>(pool.block_size());
    // A new block only when every assigned block is full.
    if (static_cast<std::size_t>(state.sequence_length) >= capacity)
        state.physical_blocks.push_back(pool.allocate_block());
    ++state.sequence_length;
}

void PageTable::free_sequence(int seq_id, BlockPool& pool) {
    SequenceState& state = checked_lookup(table_, seq_id, "free_sequence");
    for (int blk : state.physical_blocks) pool.free_block(blk);
    table_.erase(seq_id);
    device_table_dirty_ = true;
}

const SequenceState& PageTable::get_state(int seq_id) const {
    auto it = table_.find(seq_id);
    if (it == table_.end())
        throw std::runtime_error("get_state: unknown seq_id=" + std::to_string(seq_id));
    return it->second;
}

bool PageTable::has_sequence(int seq_id) const noexcept { return table_.count(seq_id) != 0; }

const int* PageTable::get_device_block_table(int seq_id, void* stream) {
    const SequenceState& state = get_state(seq_id);
    const std::size_t required = state.physical_blocks.size();
    if (required == 0) throw std::runtime_error("get_device_block_table: sequence has no physical blocks");
    if (required > d_block_table_capacity_) {
        // Grow geometrically so a growing sequence reallocates O(log n) times.
        reserve_device_block_table(std::max(required, 2 * d_block_table_capacity_));
    }
    // Blocks are only ever appended to a live sequence, so when the same
    // sequence is staged and nothing else changed, only the tail is new and
    // the mirror entries it writes were never handed to a copy before.
    std::size_t first = 0;
    if (!device_table_dirty_ && staged_seq_id_ == seq_id && staged_block_count_ <= required)
        first = staged_block_count_;
    else if (staged_block_count_ > 0) {
        // A full rewrite of the mirror: earlier copies out of it must be done.
        // They are when the last one (on the same stream) is.
        if (upload_event_ != nullptr && upload_stream_ == stream)
            detail::check(skv_event_synchronize(upload_event_), "PageTable: block table upload");
        else
            detail::check(skv_device_synchronize(), "PageTable: block table upload");
    }
    if (first < required) {
        std::copy(state.physical_blocks.begin() + static_cast<std::ptrdiff_t>(first),
                  state.physical_blocks.end(), h_block_table_ + first);
        detail::check(skv_memcpy_h2d_async(d_block_table_ + first, h_block_table_ + first,
                                           (required - first) * sizeof(int), stream),
                      "PageTable: block table upload");
        if (upload_event_ == nullptr)
            detail::check(skv_event_create(&upload_event_), "PageTable: block table upload");
        detail::check(skv_event_record(upload_event_, stream), "PageTable: block table upload");
        upload_stream_ = stream;
    }
    staged_seq_id_ = seq_id;
    staged_block_count_ = required;
    device_table_dirty_ = false;
    return d_block_table_;
}

void PageTable::reserve_device_block_table(std::size_t capacity) {
    if (capacity <= d_block_table_capacity_) return;
    if (capacity > std::numeric_limits<std::size_t>::max() / sizeof(int))
        throw std::overflow_error("reserve_device_block_table: capacity is too large");
    void* replacement = nullptr;
    void* mirror = nullptr;
    detail::check(skv_malloc(&replacement, capacity * sizeof(int)), "PageTable: block table allocation");
    const int rc = skv_host_alloc(&mirror, capacity * sizeof(int));
    if (rc != SKV_OK) {
        (void)skv_free(replacement);
        detail::check(rc, "PageTable: block table allocation");
    }
    release_device_block_table();
    d_block_table_ = static_cast<int*>(replacement);
    h_block_table_ = static_cast<int*>(mirror);
    d_block_table_capacity_ = capacity;
    device_table_dirty_ = true;
}

// ---------------------------------------------------------------------------
// DeviceBatch
// ---------------------------------------------------------------------------
DeviceBatch::DeviceBatch(int max_seqs, int max_blocks_per_seq)
    : max_seqs_(max_seqs), max_blocks_(max_blocks_per_seq) {
    if (max_seqs <= 0 || max_blocks_per_seq <= 0)
        throw std::invalid_argument("DeviceBatch: sizes must be positive");
    const std::size_t table = static_cast<std::size_t>(max_seqs) * static_cast<std::size_t>(max_blocks_per_seq);
    lens_off_ = table;
    pos_off_ = table + static_cast<std::size_t>(max_seqs);
    const std::size_t words = pos_off_ + static_cast<std::size_t>(max_seqs);
    patch_capacity_ = words;  // every entry at most once per flush
    void* p = nullptr;
    detail::check(skv_malloc(&p, words * sizeof(std::int32_t)), "DeviceBatch: state allocation");
    state_ = static_cast<std::int32_t*>(p);
    try {
        detail::check(skv_memset_d8(state_, 0xff, words * sizeof(std::int32_t), nullptr), "DeviceBatch");
        detail::check(skv_malloc(&p, 2 * patch_capacity_ * sizeof(std::int32_t)), "DeviceBatch: staging");
        patch_dev_ = static_cast<std::int32_t*>(p);
        detail::check(skv_host_alloc(&p, 2 * patch_capacity_ * sizeof(std::int32_t)), "DeviceBatch: host staging");
        patch_host_ = static_cast<std::int32_t*>(p);
        detail::check(skv_event_create(&copy_done_), "DeviceBatch: event");
        detail::check(skv_stream_synchronize(nullptr), "DeviceBatch");
    } catch (...) {
        (void)skv_free(state_);
        (void)skv_free(patch_dev_);
        (void)skv_host_free(patch_host_);
        throw;
    }
}

DeviceBatch::~DeviceBatch() noexcept {
    if (copy_done_ != nullptr) {
        (void)skv_event_synchronize(copy_done_);
        (void)skv_event_destroy(copy_done_);
    }
    (void)skv_free(state_);
    (void)skv_free(patch_dev_);
    (void)skv_host_free(patch_host_);
}

void DeviceBatch::bind(const PageTable& pages, const std::vector<int>& seq_ids, void* stream) {
    if (static_cast<int>(seq_ids.size()) > max_seqs_)
        throw std::invalid_argument("DeviceBatch::bind: more sequences than max_seqs");
    seq_ids_ = seq_ids;
    uploaded_blocks_.assign(seq_ids.size(), 0);
    uploaded_len_.assign(seq_ids.size(), -1);
    uploaded_gen_.assign(seq_ids.size(), 0);
    sync(pages, stream);
}

void DeviceBatch::sync(const PageTable& pages, void* stream) {
    // The previous flush's host staging must have been consumed.
    detail::check(skv_event_synchronize(copy_done_), "DeviceBatch::sync");
    // Every bound sequence is checked before anything is staged, so a throw
    // leaves the uploaded_* bookkeeping matching what the device holds.
    std::vector<const SequenceState*> states(seq_ids_.size());
    for (std::size_t i = 0; i < seq_ids_.size(); ++i) {
        const SequenceState& st = pages.get_state(seq_ids_[i]);
        const int nb = static_cast<int>(st.physical_blocks.size());
        if (nb > max_blocks_)
            throw std::length_error("DeviceBatch::sync: sequence " + std::to_string(seq_ids_[i]) +
                                    " has more blocks than max_blocks_per_seq");
        if (st.generation == uploaded_gen_[i] && nb < uploaded_blocks_[i])
            throw std::logic_error("DeviceBatch::sync: sequence " + std::to_string(seq_ids_[i]) +
                                   " lost blocks without being re-allocated; rebind the batch");
        states[i] = &st;
    }
    n_patches_ = 0;
    auto add = [&](std::size_t index, int value) {
        patch_host_[2 * n_patches_] = static_cast<std::int32_t>(index);
        patch_host_[2 * n_patches_ + 1] = value;
        ++n_patches_;
    };
    for (std::size_t i = 0; i < seq_ids_.size(); ++i) {
        const SequenceState& st = *states[i];
        if (st.generation != uploaded_gen_[i]) {  // bound anew, or freed and allocated again
            uploaded_blocks_[i] = 0;
            uploaded_len_[i] = -1;
            uploaded_gen_[i] = st.generation;
        }
        const int nb = static_cast<int>(st.physical_blocks.size());
        for (int k = uploaded_blocks_[i]; k < nb; ++k)
            add(i * static_cast<std::size_t>(max_blocks_) + static_cast<std::size_t>(k), st.physical_blocks[k]);
        uploaded_blocks_[i] = nb;
        if (st.sequence_length != uploaded_len_[i]) {
            add(lens_off_ + i, st.sequence_length);
            add(pos_off_ + i, st.sequence_length - 1);
            uploaded_len_[i] = st.sequence_length;
        }
    }
    flush(stream);
}

void DeviceBatch::flush(void* stream) {
    if (n_patches_ == 0) return;
    detail::check(skv_memcpy_h2d_async(patch_dev_, patch_host_, 2 * n_patches_ * sizeof(std::int32_t), stream),
                  "DeviceBatch: staging copy");
    detail::check(skv_event_record(copy_done_, stream), "DeviceBatch: staging event");
    detail::check(skv_scatter_i32(state_, patch_dev_, static_cast<int>(n_patches_), stream),
                  "DeviceBatch: table update");
}

}  // namespace memory
}  // namespace stratakv

// page_table.h -- sequence -> physical block mapping, with device-resident
// block tables.
//
// PageTable keeps the reference's interface (include/stratakv/memory/
// page_table.h:40-106): allocate_sequence takes the first block eagerly,
// append_token takes a new block only when every assigned block is full (so
// N tokens use max(1, ceil(N / block_size)) blocks), free_sequence returns the
// blocks in table order.  get_device_block_table keeps a device copy of one
// sequence's table; unlike the reference, which re-uploads the whole table
// whenever it is dirty (every token), it uploads only the block ids appended
// since the last call, as an asynchronous copy from a page-locked mirror
// queued on the caller's stream (the host never waits for the GPU there).
//
// DeviceBatch is new API for the batched entry points (the reference decodes
// one sequence per call): device arrays [max_seqs][max_blocks] block tables,
// [num_seqs] context lengths and [num_seqs] append positions for a set of
// sequences, updated incrementally (new block ids and changed lengths only)
// with one asynchronous copy from page-locked memory and one scatter kernel.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <unordered_map>
#include <vector>

#include "stratakv/memory/block_pool.h"

namespace stratakv {
namespace memory {

struct SequenceState {
    int sequence_length = 0;         // tokens appended so far
    std::vector<int> physical_blocks;  // ordered block ids
    // Extension: unique per allocate_sequence in the process, so a holder of
    // uploaded block ids (DeviceBatch) notices a seq_id that was freed and
    // allocated again.
    std::uint64_t generation = 0;
};

class PageTable {
public:
    PageTable() = default;
    PageTable(const PageTable& other);
    PageTable& operator=(const PageTable& other);
    PageTable(PageTable&& other) noexcept;
    PageTable& operator=(PageTable&& other) noexcept;
    ~PageTable() noexcept;

    // Throws std::runtime_error when seq_id already exists (or "OOM").
    void allocate_sequence(int seq_id, BlockPool& pool);
    // Throws std::runtime_error for an unknown seq_id (or "OOM"; the length
    // is then unchanged).
    void append_token(int seq_id, BlockPool& pool);
    // Throws std::runtime_error for an unknown seq_id.
    void free_sequence(int seq_id, BlockPool& pool);
    const SequenceState& get_state(int seq_id) const;
    bool has_sequence(int seq_id) const noexcept;

    // Device copy of the sequence's block ids (valid until the next call),
    // brought up to date by work queued on `stream` (a hipStream_t; nullptr =
    // the default stream): kernels that read it must run on that stream or
    // after it.
    const int* get_device_block_table(int seq_id, void* stream = nullptr);
    // Pre-size the device table so growth never allocates in the token loop.
    void reserve_device_block_table(std::size_t capacity);

private:
    void release_device_block_table() noexcept;

    std::unordered_map<int, SequenceState> table_;
    int* d_block_table_ = nullptr;
    int* h_block_table_ = nullptr;  // page-locked mirror the uploads copy from
    std::size_t d_block_table_capacity_ = 0;
    int staged_seq_id_ = 0;
    std::size_t staged_block_count_ = 0;
    bool device_table_dirty_ = true;
    void* upload_event_ = nullptr;   // recorded after the last upload out of the mirror
    void* upload_stream_ = nullptr;  // the stream of that upload
};

class DeviceBatch {
public:
    DeviceBatch(int max_seqs, int max_blocks_per_seq);
    ~DeviceBatch() noexcept;
    DeviceBatch(const DeviceBatch&) = delete;
    DeviceBatch& operator=(const DeviceBatch&) = delete;

    // Bind the batch to `seq_ids` (in this order) and upload their tables.
    void bind(const PageTable& pages, const std::vector<int>& seq_ids, void* stream = nullptr);
    // Upload what changed since the last bind/sync: block ids appended to the
    // bound sequences, their context lengths and append positions.  A bound
    // seq_id that was freed and allocated again since (a new generation) has
    // its whole row and length uploaded again.  Throws if a bound sequence is
    // unknown or lost blocks without being re-allocated (rebind instead).
    void sync(const PageTable& pages, void* stream = nullptr);

    int num_seqs() const noexcept { return static_cast<int>(seq_ids_.size()); }
    int max_seqs() const noexcept { return max_seqs_; }
    int max_blocks_per_seq() const noexcept { return max_blocks_; }
    const std::vector<int>& seq_ids() const noexcept { return seq_ids_; }
    // Device arrays: tables [max_seqs][max_blocks_per_seq], context_lens and
    // positions [num_seqs] (position = context length - 1: the slot the
    // newest token's K/V is written to).
    const std::int32_t* tables() const noexcept { return state_; }
    const std::int32_t* context_lens() const noexcept { return state_ + lens_off_; }
    const std::int32_t* positions() const noexcept { return state_ + pos_off_; }

private:
    void flush(void* stream);

    int max_seqs_;
    int max_blocks_;
    std::size_t lens_off_;
    std::size_t pos_off_;
    std::int32_t* state_ = nullptr;        // device
    std::int32_t* patch_dev_ = nullptr;    // device staging of (index, value) pairs
    std::int32_t* patch_host_ = nullptr;   // page-locked host staging
    std::size_t patch_capacity_ = 0;       // pairs
    std::size_t n_patches_ = 0;
    void* copy_done_ = nullptr;            // event: the last staging copy finished
    std::vector<int> seq_ids_;
    std::vector<int> uploaded_blocks_;
    std::vector<int> uploaded_len_;
    std::vector<std::uint64_t> uploaded_gen_;  // SequenceState::generation of the uploaded row
};

}  // namespace memory
}  // namespace stratakv

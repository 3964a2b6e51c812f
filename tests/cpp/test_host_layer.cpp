// test_host_layer.cpp -- host logic around device memory: DeviceBatch's
// incremental table uploads, PageTable::get_device_block_table, BlockPool
// copies of device pools, and Sampler's configuration, RNG stream and error
// paths.
//
// The checks read device memory back through the C ABI and compare it with
// the PageTable state, so they hold for any implementation of the ABI.  When
// no device memory can be allocated (the release library on a machine with
// no GPU) the device sections report themselves skipped; the sanitizer build
// links the host-memory stand-in of the ABI and runs them all.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "stratakv/generation/sampler.h"
#include "stratakv/memory/block_pool.h"
#include "stratakv/memory/page_table.h"
#include "stratakv/tensor.h"
#include "stratakv_amd.h"

namespace {

int failures = 0;

void check(bool ok, const std::string& what) {
    if (!ok) {
        ++failures;
        std::fprintf(stderr, "FAIL: %s\n", what.c_str());
    }
}

template <class E, class F>
bool throws(F&& f) {
    try {
        f();
    } catch (const E&) {
        return true;
    } catch (...) {
        return false;
    }
    return false;
}

bool device_memory_available() {
    void* p = nullptr;
    if (skv_malloc(&p, 64) != SKV_OK || p == nullptr) return false;
    (void)skv_free(p);
    return true;
}

std::vector<std::int32_t> download(const std::int32_t* dev, std::size_t n) {
    std::vector<std::int32_t> host(n);
    if (skv_device_synchronize() != SKV_OK ||
        skv_memcpy_d2h(host.data(), dev, n * sizeof(std::int32_t), nullptr) != SKV_OK)
        throw std::runtime_error(std::string("download: ") + skv_last_error());
    return host;
}

using stratakv::memory::BlockPool;
using stratakv::memory::DeviceBatch;
using stratakv::memory::PageTable;

// Device rows, context lengths and positions of every bound sequence equal
// the PageTable's view.
bool batch_matches(DeviceBatch& db, const PageTable& pt) {
    const int n = db.num_seqs(), mb = db.max_blocks_per_seq();
    const auto tables = download(db.tables(), static_cast<std::size_t>(db.max_seqs()) * mb);
    const auto lens = download(db.context_lens(), n);
    const auto pos = download(db.positions(), n);
    for (int i = 0; i < n; ++i) {
        const auto& st = pt.get_state(db.seq_ids()[i]);
        if (lens[i] != st.sequence_length || pos[i] != st.sequence_length - 1) return false;
        for (std::size_t k = 0; k < st.physical_blocks.size(); ++k)
            if (tables[static_cast<std::size_t>(i) * mb + k] != st.physical_blocks[k]) return false;
    }
    return true;
}

// Random appends, frees and re-allocations of bound sequences, a sync after
// each step, rebinds in new orders.
void device_batch_trace() {
    std::mt19937 rng(1234);
    BlockPool pool(512, 4);
    PageTable pt;
    const int kSeqs = 6, kMaxBlocks = 24;
    for (int s = 0; s < kSeqs; ++s) pt.allocate_sequence(10 + s, pool);
    DeviceBatch db(8, kMaxBlocks);
    std::vector<int> ids = {10, 11, 12, 13, 14, 15};
    db.bind(pt, ids);
    check(batch_matches(db, pt), "bind uploads every row");
    bool ok = true;
    for (int step = 0; step < 600 && ok; ++step) {
        const int sid = ids[rng() % ids.size()];
        const unsigned op = rng() % 100;
        if (op < 4) {  // free and allocate the same seq_id: a new generation
            pt.free_sequence(sid, pool);
            pt.allocate_sequence(sid, pool);
        } else if (op < 6) {  // rebind a shuffled subset
            std::shuffle(ids.begin(), ids.end(), rng);
            std::vector<int> sub(ids.begin(), ids.begin() + 1 + rng() % ids.size());
            db.bind(pt, sub);
            ok = batch_matches(db, pt);
            db.bind(pt, ids);
        } else {
            const int burst = 1 + static_cast<int>(rng() % 9);
            for (int t = 0; t < burst; ++t) {
                if (pt.get_state(sid).physical_blocks.size() == kMaxBlocks &&
                    pt.get_state(sid).sequence_length % 4 == 0) {
                    pt.free_sequence(sid, pool);
                    pt.allocate_sequence(sid, pool);
                }
                pt.append_token(sid, pool);
            }
        }
        db.sync(pt);
        ok = ok && batch_matches(db, pt);
        if (!ok) std::fprintf(stderr, "  mismatch after step %d (seq %d, op %u)\n", step, sid, op);
    }
    check(ok, "DeviceBatch rows follow a random append/free/rebind trace");
}

// A sync that throws uploads nothing and leaves the bookkeeping as it was:
// the next good sync still sends what the failed one would have.
void device_batch_errors() {
    BlockPool pool(64, 2);
    PageTable pt;
    pt.allocate_sequence(1, pool);
    pt.allocate_sequence(2, pool);
    DeviceBatch db(2, 3);
    db.bind(pt, {1, 2});
    for (int t = 0; t < 5; ++t) pt.append_token(1, pool);  // seq 1: 3 blocks
    for (int t = 0; t < 7; ++t) pt.append_token(2, pool);  // seq 2: 4 blocks > 3
    check(throws<std::length_error>([&] { db.sync(pt); }), "sync rejects a row longer than max_blocks_per_seq");
    pt.free_sequence(2, pool);
    pt.allocate_sequence(2, pool);
    pt.append_token(2, pool);
    db.sync(pt);
    check(batch_matches(db, pt), "a failed sync does not lose the other rows' new blocks");

    pt.free_sequence(1, pool);
    check(throws<std::runtime_error>([&] { db.sync(pt); }), "sync rejects an unknown bound seq_id");
    pt.allocate_sequence(1, pool);
    db.sync(pt);
    check(batch_matches(db, pt), "a re-allocated seq_id is uploaded whole");
    check(throws<std::invalid_argument>([] { DeviceBatch(0, 4); }), "DeviceBatch rejects zero sizes");
    check(throws<std::invalid_argument>([&] { db.bind(pt, {1, 2, 1}); }), "bind rejects more than max_seqs");
}

// get_device_block_table: incremental uploads while one sequence grows, a
// whole upload when the staged sequence changes, growth past the reserve.
void page_table_device_copy() {
    BlockPool pool(300, 2);
    PageTable pt;
    pt.allocate_sequence(5, pool);
    pt.allocate_sequence(6, pool);
    pt.reserve_device_block_table(4);
    bool ok = true;
    for (int t = 0; t < 240 && ok; ++t) {
        const int sid = (t % 7 == 0) ? 6 : 5;
        pt.append_token(sid, pool);
        const auto& blocks = pt.get_state(sid).physical_blocks;
        const int* dev = pt.get_device_block_table(sid);
        const auto got = download(dev, blocks.size());
        ok = std::equal(blocks.begin(), blocks.end(), got.begin());
    }
    check(ok, "get_device_block_table follows appends and sequence switches");
    PageTable copy(pt);
    const auto& blocks = copy.get_state(5).physical_blocks;
    const auto got = download(copy.get_device_block_table(5), blocks.size());
    check(std::equal(blocks.begin(), blocks.end(), got.begin()), "a copied PageTable uploads its own table");
}

// Copies of a device pool are deep (device to device); a moved-from pool
// owns nothing.
void block_pool_device_copies() {
    BlockPool a(8, 4, 2, 16, stratakv::Device::GPU);
    const std::size_t n = a.block_elements() * static_cast<std::size_t>(a.total_blocks());
    std::vector<std::uint16_t> pattern(n);
    for (std::size_t i = 0; i < n; ++i) pattern[i] = static_cast<std::uint16_t>(i * 2654435761u >> 16);
    check(skv_memcpy_h2d(a.key_cache(), pattern.data(), n * 2, nullptr) == SKV_OK, "upload a key pool");
    (void)a.allocate_block();
    BlockPool b(a);
    check(b.key_cache() != a.key_cache() && b.free_count() == a.free_count(), "copy owns new storage");
    std::vector<std::uint16_t> back(n);
    check(skv_device_synchronize() == SKV_OK &&
              skv_memcpy_d2h(back.data(), b.key_cache(), n * 2, nullptr) == SKV_OK && back == pattern,
          "copy holds the same keys");
    BlockPool c(std::move(b));
    check(b.key_cache() == nullptr && c.free_count() == a.free_count(), "move leaves the source empty");
    b = a;
    check(b.key_cache() != nullptr && b.key_cache() != a.key_cache(), "assignment to a moved-from pool copies");
}

// Host-side Sampler rules: configuration validation, one uniform draw per
// non-greedy choice, move semantics, shape errors before any device work.
void sampler_host_rules(bool device) {
    using stratakv::generation::Sampler;
    using stratakv::generation::SamplerConfig;
    check(throws<std::invalid_argument>([] { (void)Sampler({-1.0f, 0, 1.0f}, 1); }), "negative temperature");
    check(throws<std::invalid_argument>([] { (void)Sampler({NAN, 0, 1.0f}, 1); }), "NaN temperature");
    check(throws<std::invalid_argument>([] { (void)Sampler({1.0f, -1, 1.0f}, 1); }), "negative top_k");
    check(throws<std::invalid_argument>([] { (void)Sampler({1.0f, 0, 0.0f}, 1); }), "top_p 0");
    check(throws<std::invalid_argument>([] { (void)Sampler({1.0f, 0, 1.5f}, 1); }), "top_p above 1");

    Sampler s({0.8f, 5, 0.9f}, 42);
    const std::mt19937 start = s.rng_state();
    std::mt19937 twin(42);
    check(start == twin, "the stream starts at the seed");
    Sampler moved(std::move(s));
    check(moved.rng_state() == start && moved.config().top_k == 5, "move keeps the stream and config");
    Sampler assigned({0.0f, 0, 1.0f}, 7);
    assigned = std::move(moved);
    check(assigned.rng_state() == start, "move assignment keeps the stream");

    stratakv::Tensor bad({2, 3});
    check(throws<std::invalid_argument>([&] { (void)assigned.sample(bad); }), "[2,3] logits are rejected");
    stratakv::Tensor empty({0});
    check(throws<std::invalid_argument>([&] { (void)assigned.sample(empty); }), "empty logits are rejected");
    if (!device) return;
    stratakv::Tensor logits({5});
    for (int i = 0; i < 5; ++i) logits[i] = static_cast<float>(i == 3 ? 4.0 : 0.5 * i);
    // Either the choice kernel runs (a real device) or the error surfaces as
    // an exception; both leave the stream one draw further on.
    bool ran = false;
    try {
        const int tok = assigned.sample(logits);
        ran = tok >= 0 && tok < 5;
    } catch (const std::runtime_error&) {
        ran = true;
    }
    std::generate_canonical<double, 53>(twin);
    check(ran && assigned.rng_state() == twin, "one draw per sampled choice");
    Sampler greedy({0.0f, 0, 1.0f}, 9);
    const std::mt19937 g0 = greedy.rng_state();
    try {
        const int tok = greedy.sample(logits);
        check(tok == 3, "greedy picks the maximum");
    } catch (const std::runtime_error&) {
    }
    check(greedy.rng_state() == g0, "greedy choices draw nothing");
}

}  // namespace

// Tensor::rows_view: rows [first, first + count) of a contiguous matrix share
// its storage (values, writes through the view, the transpose view of a
// block) and outlive the matrix's own handle; out-of-range blocks throw.
void tensor_rows_view() {
    using stratakv::DataType;
    using stratakv::Device;
    using stratakv::Tensor;
    stratakv::Tensor view({1}, DataType::FP32, Device::CPU);
    {
        Tensor m({6, 4}, DataType::BF16, Device::CPU);
        for (std::size_t i = 0; i < 24; ++i) m[i] = static_cast<float>(i);
        view = m.rows_view(2, 3);
        check(view.shape() == std::vector<std::size_t>({3, 4}) && view.num_elements() == 12, "rows_view shape");
        check(view.raw_data() == static_cast<const char*>(m.raw_data()) + 2 * 4 * 2, "rows_view shares storage");
        view[5] = 100.0f;
        check(static_cast<float>(m[13]) == 100.0f, "a write through rows_view lands in the matrix");
        const Tensor t = m.rows_view(4, 2).transpose_2d();
        check(t.shape() == std::vector<std::size_t>({4, 2}) && t.value_at(1) == 20.0f, "transpose of a row block");
        check(throws<std::invalid_argument>([&] { (void)m.rows_view(4, 3); }), "rows_view past the last row throws");
        check(throws<std::invalid_argument>([&] { (void)m.rows_view(0, 0); }), "an empty rows_view throws");
        check(throws<std::invalid_argument>([&] { (void)t.rows_view(0, 1); }), "rows_view of a transpose view throws");
    }
    bool same = true;
    for (std::size_t i = 0; i < 12; ++i) same = same && view.value_at(i) == (i == 5 ? 100.0f : static_cast<float>(8 + i));
    check(same, "rows_view keeps the storage alive after the matrix handle is gone");
}

int main() {
    const bool device = device_memory_available();
    try {
        tensor_rows_view();
        sampler_host_rules(device);
        if (device) {
            device_batch_trace();
            device_batch_errors();
            page_table_device_copy();
            block_pool_device_copies();
        } else {
            std::printf("test_host_layer: no device memory; device sections skipped\n");
        }
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: unexpected exception %s\n", e.what());
        return 1;
    }
    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("test_host_layer: all checks passed%s\n", device ? "" : " (host sections)");
    return 0;
}

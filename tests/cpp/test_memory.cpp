// test_memory.cpp -- CPU tests of the C++ host layer: Tensor bf16 rules,
// BlockPool / PageTable against the reference's known answers
// (src/main.cpp:298-408 Phase 3, :73-156 Phase 4, tests/phase7_smoke.cpp:41-53)
// and, op for op, against the oracle's restatement on random traces.
// Standalone main() with check(), like the reference's own tests.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "oracle.h"
#include "stratakv/memory/block_pool.h"
#include "stratakv/memory/page_table.h"
#include "stratakv/tensor.h"

namespace {

int failures = 0;

void check(bool ok, const std::string& what) {
    if (!ok) {
        std::fprintf(stderr, "FAIL: %s\n", what.c_str());
        ++failures;
    }
}

template <typename E, typename F>
void rejects(F&& f, const std::string& what, const char* message = nullptr) {
    try {
        f();
    } catch (const E& e) {
        if (message && std::string(e.what()) != message)
            check(false, what + ": message '" + e.what() + "'");
        return;
    } catch (const std::exception& e) {
        check(false, what + ": wrong exception type (" + e.what() + ")");
        return;
    }
    check(false, what + ": no exception");
}

using stratakv::memory::BlockPool;
using stratakv::memory::PageTable;

void phase3_known_answer() {
    BlockPool pool(100, 16);
    PageTable pt;
    pt.allocate_sequence(1, pool);
    pt.allocate_sequence(2, pool);
    for (int i = 0; i < 20; ++i) pt.append_token(1, pool);
    for (int i = 0; i < 5; ++i) pt.append_token(2, pool);
    pt.allocate_sequence(3, pool);
    for (int i = 0; i < 35; ++i) pt.append_token(3, pool);
    check(pt.get_state(1).physical_blocks == std::vector<int>({0, 2}), "phase3 seq1 blocks [0,2]");
    check(pt.get_state(2).physical_blocks == std::vector<int>({1}), "phase3 seq2 blocks [1]");
    check(pt.get_state(3).physical_blocks == std::vector<int>({3, 4, 5}), "phase3 seq3 blocks [3,4,5]");
    check(pt.get_state(1).sequence_length == 20 && pt.get_state(2).sequence_length == 5 &&
              pt.get_state(3).sequence_length == 35,
          "phase3 lengths");
    check(pool.free_count() == 94, "phase3 six blocks used");
    pt.free_sequence(1, pool);
    pt.free_sequence(2, pool);
    pt.free_sequence(3, pool);
    check(pool.free_count() == 100, "phase3 pool reclaimed");
}

void phase4_pages() {
    BlockPool pool(8, 4);
    PageTable pt;
    pt.allocate_sequence(1, pool);
    pt.allocate_sequence(2, pool);
    for (int i = 0; i < 5; ++i) pt.append_token(1, pool);
    check(pt.get_state(1).physical_blocks == std::vector<int>({0, 2}), "phase4 pages [0,2]");
}

void errors_and_lifo() {
    BlockPool pool(2, 4);
    PageTable pt;
    pt.allocate_sequence(0, pool);
    rejects<std::runtime_error>([&] { pt.allocate_sequence(0, pool); }, "duplicate sequence");
    rejects<std::runtime_error>([&] { pt.append_token(7, pool); }, "unknown append");
    rejects<std::runtime_error>([&] { pt.free_sequence(7, pool); }, "unknown free");
    rejects<std::runtime_error>([&] { (void)pt.get_state(7); }, "unknown state");
    pt.allocate_sequence(1, pool);
    rejects<std::runtime_error>([&] { pt.allocate_sequence(2, pool); }, "OOM on allocate", "OOM");
    for (int i = 0; i < 4; ++i) pt.append_token(0, pool);
    rejects<std::runtime_error>([&] { pt.append_token(0, pool); }, "OOM on append", "OOM");
    check(pt.get_state(0).sequence_length == 4, "length unchanged on OOM");
    rejects<std::invalid_argument>([&] { pool.free_block(5); }, "free out of range");
    pt.free_sequence(1, pool);
    rejects<std::invalid_argument>([&] { pool.free_block(1); }, "double free");
    // LIFO: the last block freed is the first handed out.
    BlockPool p2(10, 16);
    PageTable t2;
    t2.allocate_sequence(0, p2);
    for (int i = 0; i < 33; ++i) t2.append_token(0, p2);
    t2.free_sequence(0, p2);
    check(p2.allocate_block() == 2 && p2.allocate_block() == 1 && p2.allocate_block() == 0 &&
              p2.allocate_block() == 3,
          "LIFO reuse order");
    // Copies copy the free list; moves transfer it.
    BlockPool a(5, 4);
    (void)a.allocate_block();
    BlockPool b(a);
    check(b.free_count() == 4 && b.allocate_block() == 1, "copy keeps free list");
    BlockPool c(std::move(b));
    check(c.free_count() == 3, "move keeps free list");
    rejects<std::invalid_argument>([] { BlockPool bad(0, 16); }, "zero blocks");
    rejects<std::invalid_argument>([] { BlockPool bad(4, 16, 0, 64, stratakv::Device::GPU); },
                                   "GPU pool without KV dims");
}

// Replay the oracle's trace format on this build's classes.
int trace_with_classes(int total, int bs, const std::vector<int32_t>& ops, int max_seqs,
                       std::vector<int32_t>& results, std::vector<int32_t>& lens,
                       std::vector<int32_t>& blocks, int max_blocks_out, std::vector<int32_t>& drain) {
    BlockPool pool(total, bs);
    PageTable pt;
    const int n = static_cast<int>(ops.size() / 2);
    for (int i = 0; i < n; ++i) {
        const int op = ops[2 * i], sid = ops[2 * i + 1];
        int st = ORACLE_ST_OK, blk = -1;
        try {
            if (op == ORACLE_OP_ALLOC_SEQ) {
                pt.allocate_sequence(sid, pool);
                blk = pt.get_state(sid).physical_blocks.front();
            } else if (op == ORACLE_OP_APPEND) {
                const std::size_t before = pt.has_sequence(sid) ? pt.get_state(sid).physical_blocks.size() : 0;
                pt.append_token(sid, pool);
                if (pt.get_state(sid).physical_blocks.size() > before) blk = pt.get_state(sid).physical_blocks.back();
            } else if (op == ORACLE_OP_FREE_SEQ) {
                pt.free_sequence(sid, pool);
            }
        } catch (const std::runtime_error& e) {
            const std::string m = e.what();
            st = m == "OOM" ? ORACLE_ST_OOM
                 : m.find("already exists") != std::string::npos ? ORACLE_ST_EXISTS
                 : m.find("unknown seq_id") != std::string::npos ? ORACLE_ST_UNKNOWN
                                                                : 99;
        }
        results[2 * i] = st;
        results[2 * i + 1] = blk;
    }
    for (int sid = 0; sid < max_seqs; ++sid) {
        const bool live = pt.has_sequence(sid);
        lens[sid] = live ? pt.get_state(sid).sequence_length : -1;
        for (int k = 0; k < max_blocks_out; ++k) {
            int v = -1;
            if (live && k < static_cast<int>(pt.get_state(sid).physical_blocks.size()))
                v = pt.get_state(sid).physical_blocks[k];
            blocks[static_cast<std::size_t>(sid) * max_blocks_out + k] = v;
        }
    }
    int drained = 0;
    while (pool.free_count() > 0) drain[drained++] = pool.allocate_block();
    return drained;
}

void random_traces_match_oracle() {
    std::mt19937 rng(12345);
    for (int trial = 0; trial < 200; ++trial) {
        const int total = 1 + static_cast<int>(rng() % 40), bs = 1 + static_cast<int>(rng() % 8);
        const int max_seqs = 6, mbo = 64, n = 300;
        std::vector<int32_t> ops(2 * n);
        for (int i = 0; i < n; ++i) {
            const unsigned r = rng() % 100;
            ops[2 * i] = r < 15 ? ORACLE_OP_ALLOC_SEQ : r < 25 ? ORACLE_OP_FREE_SEQ : ORACLE_OP_APPEND;
            ops[2 * i + 1] = static_cast<int32_t>(rng() % max_seqs);
        }
        std::vector<int32_t> r1(2 * n), l1(max_seqs), b1(max_seqs * mbo), d1(total + n + 1);
        std::vector<int32_t> r2(2 * n), l2(max_seqs), b2(max_seqs * mbo), d2(total + n + 1);
        const int k1 = oracle_pool_trace(total, bs, ops.data(), n, max_seqs, r1.data(), l1.data(), b1.data(), mbo,
                                         d1.data());
        const int k2 = trace_with_classes(total, bs, ops, max_seqs, r2, l2, b2, mbo, d2);
        const bool same = k1 == k2 && r1 == r2 && l1 == l2 && b1 == b2 &&
                          std::equal(d1.begin(), d1.begin() + k1, d2.begin());
        check(same, "random trace " + std::to_string(trial) + " matches the oracle");
    }
}

// SequenceState::generation: unique per allocate_sequence, unchanged by
// append_token, new after free + allocate of the same seq_id (DeviceBatch
// relies on it to re-upload a re-allocated sequence's row).
void sequence_generations() {
    BlockPool pool(8, 4);
    PageTable pt;
    pt.allocate_sequence(3, pool);
    pt.allocate_sequence(4, pool);
    const auto g3 = pt.get_state(3).generation, g4 = pt.get_state(4).generation;
    check(g3 != 0 && g4 != 0 && g3 != g4, "generations are nonzero and distinct");
    for (int i = 0; i < 9; ++i) pt.append_token(3, pool);
    check(pt.get_state(3).generation == g3, "append_token keeps the generation");
    pt.free_sequence(3, pool);
    pt.allocate_sequence(3, pool);
    check(pt.get_state(3).generation != g3 && pt.get_state(3).generation != g4,
          "a re-allocated seq_id gets a new generation");
    PageTable copy(pt);
    check(copy.get_state(3).generation == pt.get_state(3).generation, "a copy keeps the generations");
}

void tensor_rules() {
    using stratakv::DataType;
    using stratakv::Tensor;
    Tensor v({3}, DataType::BF16);
    v[0] = 1.0f;
    v[1] = -2.5f;
    v[2] = 3.25f;
    const auto* raw = static_cast<const unsigned char*>(v.raw_data());
    check(raw[0] == 0x80 && raw[1] == 0x3f && raw[2] == 0x20 && raw[3] == 0xc0, "bf16 bytes (phase7)");
    check(v[0] == 1.0f && v[1] == -2.5f && v[2] == 3.25f, "bf16 round trip");
    check(v.data() == nullptr, "bf16 exposes no float pointer");
    // RNE against the oracle on rounding-critical patterns.
    const uint32_t lowers[] = {0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF};
    Tensor w({6 * 256}, DataType::BF16);
    std::vector<float> xs;
    for (uint32_t up = 0; up < 0x10000; up += 0x101) {
        for (uint32_t lo : lowers) {
            const uint32_t bits = up << 16 | lo;
            float f;
            std::memcpy(&f, &bits, 4);
            xs.push_back(f);
        }
    }
    bool ok = true;
    for (std::size_t i = 0; i < xs.size() && i < w.num_elements(); ++i) {
        w[i] = xs[i];
        ok = ok && static_cast<const uint16_t*>(w.raw_data())[i] == oracle_f32_to_bf16_rne(xs[i]);
    }
    check(ok, "bf16 narrowing matches the oracle RNE rule");
    // Transpose view shares storage and swaps logical indices.
    Tensor m({2, 3}, DataType::BF16);
    for (int i = 0; i < 6; ++i) m[i] = static_cast<float>(i);
    Tensor t = m.transpose_2d();
    check(t.shape() == std::vector<std::size_t>({3, 2}) && !t.is_contiguous(), "transpose shape");
    check(t[1] == 3.0f && t[2] == 1.0f && t.raw_data() == m.raw_data(), "transpose indexing");
    Tensor c = m.to(stratakv::Device::CPU);
    check(c[4] == 4.0f && c.raw_data() != m.raw_data(), "to(CPU) deep copy");
}

}  // namespace

int main() {
    try {
        phase3_known_answer();
        phase4_pages();
        errors_and_lifo();
        random_traces_match_oracle();
        sequence_generations();
        tensor_rules();
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: unexpected exception %s\n", e.what());
        return 1;
    }
    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("test_memory: all checks passed\n");
    return 0;
}

// ref_driver.cpp -- C entry points over the reference's own CPU classes, used
// to pin the oracle restatement.  Compiled together with the reference's
// sources where they lie (oracle/Makefile, target `ref`) into
// oracle/_ref/libstratakv_ref.so; only tests/ load it.  This file is test
// infrastructure: it calls the reference's public API (BlockPool, PageTable,
// Tensor, PagedAttention) and contains none of its code.
#include "stratakv/layers/attention.h"
#include "stratakv/memory/block_pool.h"
#include "stratakv/memory/page_table.h"
#include "stratakv/tensor.h"

#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

namespace {

int status_of(const std::exception& e) {
    const std::string m = e.what();
    if (m == "OOM") return 1;
    if (m.find("unknown seq_id") != std::string::npos) return 2;
    if (m.find("already exists") != std::string::npos) return 3;
    return 99;
}

// Split-half RoPE angle table as PagedAttention builds it (inverse
// frequencies 10000^(-2i/hd) in double, stored as float, angle in double).
void rope_rows(float* row, int heads, int hd, int position) {
    const int half = hd / 2;
    for (int h = 0; h < heads; ++h) {
        float* x = row + static_cast<std::size_t>(h) * hd;
        for (int i = 0; i < half; ++i) {
            const float inv = static_cast<float>(std::pow(10000.0, -2.0 * i / static_cast<double>(hd)));
            const double angle = static_cast<double>(position) * static_cast<double>(inv);
            const float c = static_cast<float>(std::cos(angle));
            const float s = static_cast<float>(std::sin(angle));
            const float a = x[i], b = x[i + half];
            x[i] = a * c - b * s;
            x[i + half] = a * s + b * c;
        }
    }
}

}  // namespace

extern "C" {

// Same contract as oracle_pool_trace, executed by the reference's BlockPool
// and PageTable.
int ref_pool_trace(int total, int block_size, const int32_t* ops, int n_ops, int max_seqs,
                   int32_t* results, int32_t* lens, int32_t* blocks, int max_blocks_out,
                   int32_t* drain) {
    using stratakv::memory::BlockPool;
    using stratakv::memory::PageTable;
    BlockPool pool(total, block_size);
    PageTable pt;
    for (int i = 0; i < n_ops; ++i) {
        const int op = ops[2 * i], sid = ops[2 * i + 1];
        int st = 0, blk = -1;
        try {
            if (op == 1) {
                pt.allocate_sequence(sid, pool);
                blk = pt.get_state(sid).physical_blocks.front();
            } else if (op == 2) {
                const std::size_t before =
                    pt.has_sequence(sid) ? pt.get_state(sid).physical_blocks.size() : 0;
                pt.append_token(sid, pool);
                const auto& st_blocks = pt.get_state(sid).physical_blocks;
                if (st_blocks.size() > before) blk = st_blocks.back();
            } else if (op == 3) {
                pt.free_sequence(sid, pool);
            }
        } catch (const std::exception& e) {
            st = status_of(e);
        }
        results[2 * i] = st;
        results[2 * i + 1] = blk;
    }
    for (int sid = 0; sid < max_seqs; ++sid) {
        const bool live = pt.has_sequence(sid);
        lens[sid] = live ? pt.get_state(sid).sequence_length : -1;
        for (int k = 0; k < max_blocks_out; ++k) {
            int v = -1;
            if (live) {
                const auto& pbs = pt.get_state(sid).physical_blocks;
                if (k < static_cast<int>(pbs.size())) v = pbs[k];
            }
            blocks[static_cast<std::size_t>(sid) * max_blocks_out + k] = v;
        }
    }
    int drained = 0;
    for (;;) {
        try {
            drain[drained] = pool.allocate_block();
            ++drained;
        } catch (const std::exception&) {
            break;
        }
    }
    return drained;
}

// bf16 bytes written by Tensor::set_value for each input (little-endian pair).
int ref_bf16_rne_n(const float* in, uint16_t* out, std::size_t n) {
    try {
        stratakv::Tensor t({n}, stratakv::DataType::BF16);
        for (std::size_t i = 0; i < n; ++i) t[i] = in[i];
        const auto* raw = static_cast<const unsigned char*>(t.raw_data());
        for (std::size_t i = 0; i < n; ++i)
            out[i] = static_cast<uint16_t>(raw[2 * i] | (raw[2 * i + 1] << 8));
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// Run x[0..n_tokens) one token at a time through the reference's
// PagedAttention::forward with identity-like projections: q = x, k = x[:kv_dim],
// v = x[hidden-kv_dim:], out_proj = I.  A second sequence takes one token after
// each step so the first sequence's pages interleave with it (non-contiguous).
// Outputs: out[t] = the reference's context row for token t (attention over
// positions 0..t), q_eff/k_eff/v_eff = the query, cached key and cached value
// rows after RoPE, table[0..*n_blocks) = the first sequence's physical blocks.
int ref_attention_trace(int hidden, int heads, int kv_heads, int total_blocks, int block_size,
                        int n_tokens, const float* x, float* out, float* q_eff, float* k_eff,
                        float* v_eff, int32_t* table, int* n_blocks) {
    using stratakv::Tensor;
    try {
        stratakv::layers::PagedAttention attn(hidden, heads, kv_heads, total_blocks, block_size);
        const int hd = hidden / heads;
        const int kv_dim = kv_heads * hd;
        const int voff = hidden - kv_dim;
        auto& wq = attn.query_projection().weight();
        auto& wk = attn.key_projection().weight();
        auto& wv = attn.value_projection().weight();
        auto& wo = attn.output_projection().weight();
        for (int i = 0; i < hidden; ++i) {
            for (int j = 0; j < hidden; ++j) {
                wq[static_cast<std::size_t>(i) * hidden + j] = i == j ? 1.0f : 0.0f;
                wo[static_cast<std::size_t>(i) * hidden + j] = i == j ? 1.0f : 0.0f;
            }
            for (int j = 0; j < kv_dim; ++j) {
                wk[static_cast<std::size_t>(i) * kv_dim + j] = i == j ? 1.0f : 0.0f;
                wv[static_cast<std::size_t>(i) * kv_dim + j] = i == j + voff ? 1.0f : 0.0f;
            }
        }
        stratakv::memory::BlockPool pool(total_blocks, block_size);
        stratakv::memory::PageTable pages;
        pages.allocate_sequence(0, pool);
        pages.allocate_sequence(1, pool);
        for (int t = 0; t < n_tokens; ++t) {
            Tensor xt({1, static_cast<std::size_t>(hidden)});
            for (int i = 0; i < hidden; ++i) xt[i] = x[static_cast<std::size_t>(t) * hidden + i];
            Tensor o = attn.forward(xt, 0, pages, pool);
            for (int i = 0; i < hidden; ++i) out[static_cast<std::size_t>(t) * hidden + i] = o[i];
            pages.append_token(1, pool);

            float* qr = q_eff + static_cast<std::size_t>(t) * hidden;
            float* kr = k_eff + static_cast<std::size_t>(t) * kv_dim;
            float* vr = v_eff + static_cast<std::size_t>(t) * kv_dim;
            std::memcpy(qr, x + static_cast<std::size_t>(t) * hidden, sizeof(float) * hidden);
            std::memcpy(kr, x + static_cast<std::size_t>(t) * hidden, sizeof(float) * kv_dim);
            std::memcpy(vr, x + static_cast<std::size_t>(t) * hidden + voff, sizeof(float) * kv_dim);
            rope_rows(qr, heads, hd, t);
            rope_rows(kr, kv_heads, hd, t);
        }
        const auto& pbs = pages.get_state(0).physical_blocks;
        *n_blocks = static_cast<int>(pbs.size());
        for (std::size_t k = 0; k < pbs.size(); ++k) table[k] = pbs[k];
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// The same setup as ref_attention_trace, but the tokens go through
// PagedAttention::forward in chunks of chunk_lens[c] tokens (a prefill chunk
// per call: every token of a chunk attends causally to all earlier tokens,
// those of the same chunk included).  The second sequence takes one token
// after each chunk, so the first sequence's pages are non-contiguous.
int ref_prefill_trace(int hidden, int heads, int kv_heads, int total_blocks, int block_size,
                      int n_chunks, const int32_t* chunk_lens, const float* x, float* out,
                      float* q_eff, float* k_eff, float* v_eff, int32_t* table, int* n_blocks) {
    using stratakv::Tensor;
    try {
        stratakv::layers::PagedAttention attn(hidden, heads, kv_heads, total_blocks, block_size);
        const int hd = hidden / heads;
        const int kv_dim = kv_heads * hd;
        const int voff = hidden - kv_dim;
        auto& wq = attn.query_projection().weight();
        auto& wk = attn.key_projection().weight();
        auto& wv = attn.value_projection().weight();
        auto& wo = attn.output_projection().weight();
        for (int i = 0; i < hidden; ++i) {
            for (int j = 0; j < hidden; ++j) {
                wq[static_cast<std::size_t>(i) * hidden + j] = i == j ? 1.0f : 0.0f;
                wo[static_cast<std::size_t>(i) * hidden + j] = i == j ? 1.0f : 0.0f;
            }
            for (int j = 0; j < kv_dim; ++j) {
                wk[static_cast<std::size_t>(i) * kv_dim + j] = i == j ? 1.0f : 0.0f;
                wv[static_cast<std::size_t>(i) * kv_dim + j] = i == j + voff ? 1.0f : 0.0f;
            }
        }
        stratakv::memory::BlockPool pool(total_blocks, block_size);
        stratakv::memory::PageTable pages;
        pages.allocate_sequence(0, pool);
        pages.allocate_sequence(1, pool);
        int t0 = 0;
        for (int c = 0; c < n_chunks; ++c) {
            const int n = chunk_lens[c];
            Tensor xt({static_cast<std::size_t>(n), static_cast<std::size_t>(hidden)});
            for (int t = 0; t < n; ++t)
                for (int i = 0; i < hidden; ++i)
                    xt[static_cast<std::size_t>(t) * hidden + i] = x[static_cast<std::size_t>(t0 + t) * hidden + i];
            Tensor o = attn.forward(xt, 0, pages, pool);
            for (int t = 0; t < n; ++t)
                for (int i = 0; i < hidden; ++i)
                    out[static_cast<std::size_t>(t0 + t) * hidden + i] = o[static_cast<std::size_t>(t) * hidden + i];
            pages.append_token(1, pool);
            for (int t = t0; t < t0 + n; ++t) {
                float* qr = q_eff + static_cast<std::size_t>(t) * hidden;
                float* kr = k_eff + static_cast<std::size_t>(t) * kv_dim;
                float* vr = v_eff + static_cast<std::size_t>(t) * kv_dim;
                std::memcpy(qr, x + static_cast<std::size_t>(t) * hidden, sizeof(float) * hidden);
                std::memcpy(kr, x + static_cast<std::size_t>(t) * hidden, sizeof(float) * kv_dim);
                std::memcpy(vr, x + static_cast<std::size_t>(t) * hidden + voff, sizeof(float) * kv_dim);
                rope_rows(qr, heads, hd, t);
                rope_rows(kr, kv_heads, hd, t);
            }
            t0 += n;
        }
        const auto& pbs = pages.get_state(0).physical_blocks;
        *n_blocks = static_cast<int>(pbs.size());
        for (std::size_t k = 0; k < pbs.size(); ++k) table[k] = pbs[k];
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

}  // extern "C"

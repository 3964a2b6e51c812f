// ref_driver.cpp -- C entry points over the reference's own CPU classes, used
// to pin the oracle restatement and to write golden vectors.  Compiled
// together with the reference's sources where they lie (oracle/Makefile,
// target `ref`) into oracle/_ref/libstratakv_ref.so; only tests/ load it.
// This file is test infrastructure: it calls the reference's public API
// (BlockPool, PageTable, Tensor, PagedAttention, TransformerBlock, RMSNorm,
// Linear, load_safetensors, Sampler) and contains none of its code.
#include "stratakv/generation/sampler.h"
#include "stratakv/io/safetensors.h"
#include "stratakv/layers/attention.h"
#include "stratakv/layers/rmsnorm.h"
#include "stratakv/memory/block_pool.h"
#include "stratakv/memory/page_table.h"
#include "stratakv/models/transformer_block.h"
#include "stratakv/tensor.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <limits>
#include <numeric>
#include <random>
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

// Time the reference's single-token PagedAttention::forward (identity
// projections as in ref_attention_trace) at a context of `context` tokens --
// the first context - 1 written by one multi-token forward -- and, on a fresh
// sequence, at a context of 1.  Each is the median of `reps` calls in ms (the
// timed calls append their token, so the long context grows by one per call).
// The difference is the attention over the context; the rest of forward (the
// four projections, RoPE, the cache write) is the same in both.
int ref_decode_timing(int hidden, int heads, int kv_heads, int block_size, int context, int reps,
                      double* ms_context, double* ms_one) {
    using stratakv::Tensor;
    using clock = std::chrono::steady_clock;
    try {
        const int total_blocks = (context + reps) / block_size + reps + 4;
        stratakv::layers::PagedAttention attn(hidden, heads, kv_heads, total_blocks, block_size);
        const int hd = hidden / heads;
        const int kv_dim = kv_heads * hd;
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
                wv[static_cast<std::size_t>(i) * kv_dim + j] = i == j + hidden - kv_dim ? 1.0f : 0.0f;
            }
        }
        std::mt19937 rng(1234);
        std::normal_distribution<float> nd(0.0f, 1.0f);
        stratakv::memory::BlockPool pool(total_blocks, block_size);
        stratakv::memory::PageTable pages;
        pages.allocate_sequence(0, pool);
        Tensor prefix({static_cast<std::size_t>(context - 1), static_cast<std::size_t>(hidden)});
        for (std::size_t i = 0; i < prefix.num_elements(); ++i) prefix[i] = nd(rng);
        (void)attn.forward(prefix, 0, pages, pool);
        auto time_one = [&](int seq_id) {
            Tensor xt({1, static_cast<std::size_t>(hidden)});
            for (int i = 0; i < hidden; ++i) xt[i] = nd(rng);
            const auto t0 = clock::now();
            Tensor o = attn.forward(xt, seq_id, pages, pool);
            const double ms = std::chrono::duration<double, std::milli>(clock::now() - t0).count();
            if (!std::isfinite(o[0])) throw std::runtime_error("non-finite output");
            return ms;
        };
        std::vector<double> t_ctx, t_one;
        for (int r = 0; r < reps; ++r) t_ctx.push_back(time_one(0));
        for (int r = 0; r < reps; ++r) {
            pages.allocate_sequence(1 + r, pool);
            t_one.push_back(time_one(1 + r));
        }
        std::sort(t_ctx.begin(), t_ctx.end());
        std::sort(t_one.begin(), t_one.end());
        *ms_context = t_ctx[t_ctx.size() / 2];
        *ms_one = t_one[t_one.size() / 2];
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

// ---- checkpoint loader ----------------------------------------------------
// Loads `path` with the reference's load_safetensors.  On success returns 0,
// the number of tensors in *count, and, when `name` is given, copies that
// tensor's FP32 values into out[0..cap) and its element count into *n.
// On failure returns 1 and the exception text in err[0..err_cap).
int ref_load_tensor(const char* path, int require_mapped_f32, const char* name, float* out,
                    std::size_t cap, std::size_t* n, int* count, char* err, int err_cap) {
    try {
        auto weights = stratakv::io::load_safetensors(path, require_mapped_f32 != 0);
        *count = static_cast<int>(weights.size());
        if (name != nullptr) {
            const auto it = weights.find(name);
            if (it == weights.end()) {
                std::snprintf(err, err_cap, "no tensor %s", name);
                return 2;
            }
            const auto& t = it->second;
            *n = t.num_elements();
            for (std::size_t i = 0; i < t.num_elements() && i < cap; ++i) out[i] = t[i];
        }
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(err, err_cap, "%s", e.what());
        return 1;
    }
}

// load_linear_bf16_transposed of an [out_f, in_f] FP32 source; dst receives
// the [in_f, out_f] bf16 bit patterns.
int ref_linear_bf16_transposed(const float* src, std::size_t out_f, std::size_t in_f, uint16_t* dst) {
    try {
        stratakv::Tensor t({out_f, in_f});
        std::memcpy(t.data(), src, sizeof(float) * out_f * in_f);
        const auto r = stratakv::io::load_linear_bf16_transposed(t, out_f, in_f);
        std::memcpy(dst, r.raw_data(), sizeof(uint16_t) * out_f * in_f);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// ---- sampler ----------------------------------------------------------------
// tokens[r] = Sampler(config, seed).sample(logits row r) for rows in order,
// one sampler (one mt19937 stream) across all rows.  Returns 0, or 1 with the
// exception text (and the failing row in *failed_row).
int ref_sample_rows(const float* logits, int rows, int vocab, float temperature, int top_k,
                    float top_p, uint32_t seed, int32_t* tokens, int* failed_row, char* err,
                    int err_cap) {
    int r = 0;
    try {
        stratakv::generation::Sampler sampler({temperature, top_k, top_p}, seed);
        stratakv::Tensor t({static_cast<std::size_t>(vocab)});
        for (r = 0; r < rows; ++r) {
            std::memcpy(t.data(), logits + static_cast<std::size_t>(r) * vocab, sizeof(float) * vocab);
            tokens[r] = sampler.sample(t);
        }
        return 0;
    } catch (const std::exception& e) {
        *failed_row = r;
        std::snprintf(err, err_cap, "%s", e.what());
        return 1;
    }
}

// The uniform draws a std::discrete_distribution makes from std::mt19937(seed):
// generate_canonical<double, 53>, one per draw.
void ref_canonical_draws(uint32_t seed, int n, double* out) {
    std::mt19937 g(seed);
    for (int i = 0; i < n; ++i)
        out[i] = std::generate_canonical<double, std::numeric_limits<double>::digits>(g);
}

// ---- greedy generation trace ---------------------------------------------
// The reference's CPU generation path (Generator::generate with Device::CPU,
// src/generation/generator.cpp:617-803) driven through the public classes so
// the logits of every step can be recorded: the checkpoint is loaded with
// load_safetensors, the Llama weights are placed as the Generator places them
// (linears through load_linear_bf16_transposed), the prompt tokens[0..n_prompt)
// run as one multi-token forward, then every later step feeds tokens[p]
// (teacher forcing with the caller's stream) one token at a time.
// Step s (0..n_tokens-n_prompt) records the greedy argmax and the top_k
// logits (ids and values, descending, ties by index) of the logits that
// predict position n_prompt + s.  A negative tokens[p] (p >= n_prompt) is
// replaced by the argmax that predicts it (plain greedy generation).
int ref_generate_trace(const char* path, int layers, int heads, int kv_heads, int32_t* tokens,
                       int n_tokens, int n_prompt, int top_k, int32_t* argmax, int32_t* top_ids,
                       float* top_vals, char* err, int err_cap) {
    using stratakv::Tensor;
    try {
        auto w = stratakv::io::load_safetensors(path);
        auto take = [&](const std::string& k) {
            auto it = w.find(k);
            if (it == w.end()) throw std::invalid_argument("missing " + k);
            Tensor t = std::move(it->second);
            w.erase(it);
            return t;
        };
        Tensor emb = take("model.embed_tokens.weight");
        const std::size_t vocab = emb.shape()[0], h = emb.shape()[1];
        const std::size_t hd = h / heads;
        const std::size_t kvd = hd * kv_heads;
        auto set_linear = [&](stratakv::layers::Linear& lin, const std::string& k, std::size_t out_f,
                              std::size_t in_f) {
            Tensor src = take(k);
            lin.set_weight(stratakv::io::load_linear_bf16_transposed(src, out_f, in_f));
        };
        std::vector<stratakv::models::TransformerBlock> blocks;
        std::vector<stratakv::memory::BlockPool> pools;
        std::vector<stratakv::memory::PageTable> pages(layers);
        Tensor gate0 = std::move(w.at("model.layers.0.mlp.gate_proj.weight"));
        const std::size_t inter = gate0.shape()[0];
        w.at("model.layers.0.mlp.gate_proj.weight") = std::move(gate0);
        blocks.reserve(layers);
        for (int l = 0; l < layers; ++l) {
            blocks.emplace_back(h, inter, heads, kv_heads, 1024, 16, stratakv::Device::CPU);
            pools.emplace_back(1024, 16);
            auto& b = blocks.back();
            const std::string p = "model.layers." + std::to_string(l) + ".";
            b.input_norm() = stratakv::layers::RMSNorm(take(p + "input_layernorm.weight"));
            b.post_attention_norm() = stratakv::layers::RMSNorm(take(p + "post_attention_layernorm.weight"));
            set_linear(b.attention().query_projection(), p + "self_attn.q_proj.weight", h, h);
            set_linear(b.attention().key_projection(), p + "self_attn.k_proj.weight", kvd, h);
            set_linear(b.attention().value_projection(), p + "self_attn.v_proj.weight", kvd, h);
            set_linear(b.attention().output_projection(), p + "self_attn.o_proj.weight", h, h);
            set_linear(b.gate_projection(), p + "mlp.gate_proj.weight", inter, h);
            set_linear(b.up_projection(), p + "mlp.up_proj.weight", inter, h);
            set_linear(b.down_projection(), p + "mlp.down_proj.weight", h, inter);
            pages[l].allocate_sequence(0, pools[l]);
        }
        stratakv::layers::RMSNorm final_norm(take("model.norm.weight"));
        stratakv::layers::Linear lm_head(h, vocab);
        set_linear(lm_head, "lm_head.weight", vocab, h);

        auto embed = [&](const int32_t* ids, std::size_t n) {
            Tensor x({n, h});
            for (std::size_t r = 0; r < n; ++r)
                for (std::size_t c = 0; c < h; ++c) x[r * h + c] = emb[static_cast<std::size_t>(ids[r]) * h + c];
            return x;
        };
        auto forward = [&](Tensor x) {
            for (int l = 0; l < layers; ++l) x = blocks[l].forward(x, 0, pages[l], pools[l], true);
            return x;
        };
        Tensor hidden = forward(embed(tokens, n_prompt));
        Tensor last({1, h});
        for (std::size_t c = 0; c < h; ++c) last[c] = hidden[(n_prompt - 1) * h + c];
        std::vector<std::size_t> order(vocab);
        for (int s = 0; n_prompt + s <= n_tokens; ++s) {
            Tensor logits = lm_head.forward(final_norm.forward(last));
            std::size_t best = 0;
            for (std::size_t i = 1; i < vocab; ++i)
                if (logits[i] > logits[best]) best = i;
            argmax[s] = static_cast<int32_t>(best);
            std::iota(order.begin(), order.end(), std::size_t{0});
            std::partial_sort(order.begin(), order.begin() + top_k, order.end(),
                              [&](std::size_t a, std::size_t b) {
                                  if (logits[a] != logits[b]) return logits[a] > logits[b];
                                  return a < b;
                              });
            for (int k = 0; k < top_k; ++k) {
                top_ids[static_cast<std::size_t>(s) * top_k + k] = static_cast<int32_t>(order[k]);
                top_vals[static_cast<std::size_t>(s) * top_k + k] = logits[order[k]];
            }
            if (n_prompt + s == n_tokens) break;
            if (tokens[n_prompt + s] < 0) tokens[n_prompt + s] = static_cast<int32_t>(best);
            last = forward(embed(tokens + n_prompt + s, 1));
        }
        return 0;
    } catch (const std::exception& e) {
        std::snprintf(err, err_cap, "%s", e.what());
        return 1;
    }
}

}  // extern "C"

// generator.cpp -- Generator: weight placement, and a generation loop whose
// every step (embedding, layers, final norm, lm_head, token choice) is queued
// on the device with the token ids kept in device memory.
//
// Configuration, weight-schema and generate() rules with their messages
// follow src/generation/generator.cpp:169-200 (validate_config), :265-345
// (take / load_linear / take_embedding / take_final_norm), :374-518 (the
// constructor) and :617-803 (generate).
#include "stratakv/generation/generator.h"

#include <algorithm>
#include <chrono>
#include <climits>
#include <cstdint>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <limits>
#include <memory>
#include <stdexcept>
#include <string>
#include <random>
#include <utility>

#include "abi_check.h"
#include "parity_model.h"

namespace stratakv {
namespace generation {
namespace {

using Clock = std::chrono::steady_clock;

std::size_t checked_elements(std::initializer_list<std::size_t> dims) {
    const auto byte_limit = std::min<std::size_t>(std::numeric_limits<std::size_t>::max() - 63u,
                                                  static_cast<std::size_t>(std::numeric_limits<std::ptrdiff_t>::max()));
    const std::size_t limit = byte_limit / sizeof(float);
    std::size_t n = 1;
    for (std::size_t d : dims) {
        if (d == 0 || n > limit / d) throw std::overflow_error("Generator: invalid/overflowing tensor size");
        n *= d;
    }
    return n;
}

GeneratorConfig validate_config(GeneratorConfig c) {
    if (c.device != Device::GPU) throw std::invalid_argument("Generator: GPU builds require Device::GPU");
    const std::size_t kv = c.num_kv_heads == 0 ? c.num_heads : c.num_kv_heads;
    if (c.hidden_dim == 0 || c.intermediate_dim == 0 || c.num_heads == 0 || c.num_layers == 0 || kv == 0 ||
        c.num_heads % kv != 0 || c.vocab_size == 0 || c.vocab_size > static_cast<std::size_t>(INT_MAX) ||
        c.total_blocks <= 0 || c.block_size <= 0 || c.hidden_dim % c.num_heads != 0 || c.eos_token_id < -1 ||
        (c.eos_token_id >= 0 && static_cast<std::size_t>(c.eos_token_id) >= c.vocab_size))
        throw std::invalid_argument("Generator: invalid configuration");
    checked_elements({c.hidden_dim, c.hidden_dim});
    checked_elements({c.hidden_dim, c.intermediate_dim});
    checked_elements({c.vocab_size, c.hidden_dim});
    checked_elements({c.num_layers, c.hidden_dim, c.hidden_dim});
    checked_elements({c.num_layers, c.hidden_dim, c.intermediate_dim});
    const std::size_t kv_dim = kv * (c.hidden_dim / c.num_heads);
    checked_elements({c.num_layers, c.hidden_dim, kv_dim});
    checked_elements({c.num_layers, static_cast<std::size_t>(c.total_blocks), static_cast<std::size_t>(c.block_size),
                      kv_dim});
    return c;
}

// Takes weights out of the map, checks shape and finiteness (on the device)
// and converts them to the role's device form.
class WeightTaker {
public:
    WeightTaker(io::WeightMap& weights, void* stream) : weights_(weights), stream_(stream) {
        void* p = nullptr;
        detail::check(skv_malloc(&p, sizeof(std::int32_t)), "Generator: weight check");
        flag_ = static_cast<std::int32_t*>(p);
    }
    ~WeightTaker() { (void)skv_free(flag_); }
    WeightTaker(const WeightTaker&) = delete;
    WeightTaker& operator=(const WeightTaker&) = delete;

    bool has(const std::string& key) const { return weights_.find(key) != weights_.end(); }

    // Device tensor with the expected shape and only finite values, in its
    // stored dtype (BF16 or FP32).
    Tensor take(const std::string& key, std::initializer_list<std::size_t> expected) {
        auto it = weights_.find(key);
        if (it == weights_.end()) throw std::invalid_argument("Missing weight: " + key);
        const Tensor& src = it->second;
        if (src.shape() != std::vector<std::size_t>(expected) || src.num_elements() != checked_elements(expected) ||
            !src.raw_data() || !src.is_contiguous())
            throw std::invalid_argument("Wrong shape/storage: " + key);
        Tensor t = src.device() == Device::GPU ? std::move(it->second) : src.to(Device::GPU);
        weights_.erase(it);
        const int dt = t.dtype() == DataType::BF16 ? SKV_DTYPE_BF16 : SKV_DTYPE_FP32;
        detail::check(skv_memset_d8(flag_, 0, sizeof(std::int32_t), stream_), "Generator: weight check");
        detail::check(skv_check_finite(t.raw_data(), dt, t.num_elements(), flag_, stream_), "Generator: weight check");
        std::int32_t bad = 0;
        detail::check(skv_memcpy_d2h(&bad, flag_, sizeof(bad), stream_), "Generator: weight check");
        if (bad != 0) throw std::invalid_argument("Non-finite weight: " + key);
        return t;
    }

    // FP32 norm gamma [n].
    Tensor take_f32(const std::string& key, std::size_t n) {
        Tensor t = take(key, {n});
        if (t.dtype() == DataType::FP32) return t;
        Tensor f({n}, DataType::FP32, Device::GPU);
        detail::check(skv_convert_to_f32(t.raw_data(), SKV_DTYPE_BF16, n, static_cast<float*>(f.raw_data()), nullptr,
                                         stream_),
                      "Generator: norm weight");
        detail::check(skv_stream_synchronize(stream_), "Generator: norm weight");
        return f;
    }

    // A checkpoint [out, in] linear as BF16 rows behind a [in, out] view;
    // FP32 values keep their upper 16 bits (src/generation/generator.cpp:292-328).
    void take_linear(const std::string& key, layers::Linear& layer) {
        const std::size_t in = layer.input_dim(), out = layer.output_dim();
        Tensor t = take(key, {out, in});
        if (t.dtype() != DataType::BF16) {
            Tensor b({out, in}, DataType::BF16, Device::GPU);
            detail::check(skv_convert_to_bf16(t.raw_data(), SKV_DTYPE_FP32, out * in,
                                              static_cast<std::uint16_t*>(b.raw_data()), nullptr, stream_),
                          "Generator: linear weight");
            detail::check(skv_stream_synchronize(stream_), "Generator: linear weight");
            t = std::move(b);
        }
        layer.set_weight(t.transpose_2d());
    }

    // Several checkpoint linears with one input width as consecutive row
    // blocks of ONE bf16 allocation ([sum of out, in]), each layer holding a
    // view of its block: the same values and strides as take_linear gives, so
    // every kernel reads the same bits, and the prompt path's library GEMMs
    // then run q/k/v (or gate/up) as one GEMM (skv_*_gemm_f32 detect rows
    // that follow one another).
    void take_linears_packed(std::initializer_list<std::pair<std::string, layers::Linear*>> items) {
        std::size_t in = 0, rows = 0;
        for (const auto& [key, layer] : items) {
            if (in != 0 && layer->input_dim() != in) throw std::invalid_argument("Wrong shape/storage: " + key);
            in = layer->input_dim();
            rows += layer->output_dim();
        }
        Tensor packed({rows, in}, DataType::BF16, Device::GPU);
        std::size_t first = 0;
        for (const auto& [key, layer] : items) {
            const std::size_t out = layer->output_dim();
            Tensor t = take(key, {out, in});
            auto* dst = static_cast<std::uint16_t*>(packed.raw_data()) + first * in;
            if (t.dtype() == DataType::BF16)
                detail::check(skv_memcpy_d2d(dst, t.raw_data(), out * in * sizeof(std::uint16_t), stream_),
                              "Generator: linear weight");
            else
                detail::check(skv_convert_to_bf16(t.raw_data(), SKV_DTYPE_FP32, out * in, dst, nullptr, stream_),
                              "Generator: linear weight");
            detail::check(skv_stream_synchronize(stream_), "Generator: linear weight");
            layer->set_weight(packed.rows_view(first, out).transpose_2d());
            first += out;
        }
    }

private:
    io::WeightMap& weights_;
    void* stream_;
    std::int32_t* flag_ = nullptr;
};

}  // namespace

Generator::Generator(GeneratorConfig config, io::WeightMap weights)
    : config_(validate_config(config)), sampler_(config_.sampler) {
    const auto t0 = Clock::now();
    const std::size_t h = config_.hidden_dim, inter = config_.intermediate_dim;
    const std::size_t kv_heads = config_.num_kv_heads == 0 ? config_.num_heads : config_.num_kv_heads;
    const std::size_t kv_dim = kv_heads * (h / config_.num_heads);
    blocks_.reserve(config_.num_layers);
    pools_.reserve(config_.num_layers);
    for (std::size_t l = 0; l < config_.num_layers; ++l) {
        blocks_.emplace_back(h, inter, config_.num_heads, kv_heads, config_.total_blocks, config_.block_size,
                             Device::CPU);
        pools_.emplace_back(config_.total_blocks, config_.block_size, static_cast<int>(kv_heads),
                            static_cast<int>(h / config_.num_heads), Device::GPU);
    }
    pages_.resize(config_.num_layers);

    WeightTaker w(weights, stream_);
    const char* emb_key = w.has("model.embed_tokens.weight") ? "model.embed_tokens.weight" : "tok_embeddings.weight";
    embeddings_.emplace(w.take(emb_key, {config_.vocab_size, h}));
    const char* norm_key = w.has("model.norm.weight") ? "model.norm.weight" : "norm.weight";
    final_norm_.emplace(w.take_f32(norm_key, h));
    if (w.has("model.layers.0.input_layernorm.weight")) {
        for (std::size_t l = 0; l < config_.num_layers; ++l) {
            const std::string p = "model.layers." + std::to_string(l) + ".";
            auto& b = blocks_[l];
            b.input_norm() = layers::RMSNorm(w.take_f32(p + "input_layernorm.weight", h));
            b.post_attention_norm() = layers::RMSNorm(w.take_f32(p + "post_attention_layernorm.weight", h));
            w.take_linears_packed({{p + "self_attn.q_proj.weight", &b.attention().query_projection()},
                                   {p + "self_attn.k_proj.weight", &b.attention().key_projection()},
                                   {p + "self_attn.v_proj.weight", &b.attention().value_projection()}});
            w.take_linear(p + "self_attn.o_proj.weight", b.attention().output_projection());
            w.take_linears_packed({{p + "mlp.gate_proj.weight", &b.gate_projection()},
                                   {p + "mlp.up_proj.weight", &b.up_projection()}});
            w.take_linear(p + "mlp.down_proj.weight", b.down_projection());
        }
    } else {
        // The one-layer "block.*" schema (src/generation/generator.cpp:430-461):
        // its single FFN input matrix serves as both gate and up projection.
        if (config_.num_layers != 1) throw std::invalid_argument("Generator: Llama layer weights are missing");
        auto& b = blocks_.front();
        b.input_norm() = layers::RMSNorm(w.take_f32("block.input_norm.weight", h));
        b.post_attention_norm() = layers::RMSNorm(w.take_f32("block.post_attention_norm.weight", h));
        w.take_linear("block.attn.q_proj.weight", b.attention().query_projection());
        w.take_linear("block.attn.k_proj.weight", b.attention().key_projection());
        w.take_linear("block.attn.v_proj.weight", b.attention().value_projection());
        w.take_linear("block.attn.o_proj.weight", b.attention().output_projection());
        w.take_linear("block.ffn.up_proj.weight", b.gate_projection());
        b.up_projection().set_weight(b.gate_projection().weight().to(Device::GPU));
        w.take_linear("block.ffn.down_proj.weight", b.down_projection());
    }
    lm_head_.emplace(h, config_.vocab_size);
    w.take_linear("lm_head.weight", *lm_head_);
    (void)kv_dim;

    for (auto& b : blocks_) b.to(Device::GPU);
    // The layers run one after another on one stream: one prefill scratch serves them all.
    const auto scratch = std::make_shared<models::TransformerBlock::PrefillScratch>();
    for (auto& b : blocks_) b.share_prefill_scratch(scratch);
    // STRATAKV_PARITY=1 (src/generation/generator.cpp:33-36, 485-490): every
    // layer of every position is compared with a host model of the layer
    // (parity_model.h); steps run one kernel at a time so each layer's output
    // can be read.
    if (const char* v = std::getenv("STRATAKV_PARITY"); v != nullptr && std::strcmp(v, "1") == 0) {
        parity_ = std::make_unique<detail::ParityModel>(blocks_, *final_norm_, *lm_head_, *embeddings_);
        graph_replay_ = false;
        std::fprintf(stderr, "[PARITY] host model of %zu layers (double precision, bf16 K/V cache as the pools "
                             "hold it); decode steps launched one kernel at a time\n",
                     parity_->num_layers());
    }
    // STRATAKV_GRAPH_REPLAY=0: every decode step launched one kernel at a time
    // (as set_graph_replay(false)).  For profiling: under rocprofv3's kernel
    // tracing (ROCm 7.2) a replayed step ended the process with a host-side
    // read of a runtime-owned device address inside hipGraphLaunch, in frames
    // outside this library, so kernel traces are taken with replay off.
    if (const char* v = std::getenv("STRATAKV_GRAPH_REPLAY"); v != nullptr && std::strcmp(v, "0") == 0)
        graph_replay_ = false;
    if (parity_) graph_replay_ = false;
    hidden_.emplace(std::vector<std::size_t>{1, h}, DataType::FP32, Device::GPU);
    normed_.emplace(std::vector<std::size_t>{1, h}, DataType::FP32, Device::GPU);
    logits_.emplace(std::vector<std::size_t>{1, config_.vocab_size}, DataType::FP32, Device::GPU);
    step_events_.assign(kLookahead + 2, nullptr);
    for (auto& e : step_events_) detail::check(skv_event_create(&e), "Generator: workspace");
    if (!weights.empty()) throw std::invalid_argument("Unexpected weight: " + weights.begin()->first);
    initialization_ms_ = std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

Generator::~Generator() {
    (void)skv_device_synchronize();
    release_step_graph();
    for (void* e : step_events_)
        if (e) (void)skv_event_destroy(e);
    if (ids_) (void)skv_free(ids_);
    if (flags_) (void)skv_free(flags_);
    if (host_ids_) (void)skv_host_free(host_ids_);
    if (step_state_) (void)skv_free(step_state_);
    if (rope_table_) (void)skv_free(rope_table_);
    if (capture_stream_) (void)skv_stream_destroy(capture_stream_);
    if (kv_saved_) (void)skv_free(kv_saved_);
    if (kv_chunk_ptrs_) (void)skv_free(kv_chunk_ptrs_);
    if (kv_chunk_host_) (void)skv_host_free(kv_chunk_host_);
}

void Generator::set_graph_replay(bool enabled) {
    graph_replay_ = enabled && !parity_;
    if (!enabled) {
        (void)skv_stream_synchronize(stream_);
        release_step_graph();
    }
}

void Generator::release_step_graph() noexcept {
    if (step_graph_) (void)skv_graph_destroy(step_graph_);
    step_graph_ = nullptr;
    graph_key_.clear();
}

std::vector<float> Generator::last_logits() const {
    if (!logits_) return {};
    std::vector<float> out(config_.vocab_size);
    detail::check(skv_memcpy_d2h(out.data(), logits_->raw_data(), out.size() * sizeof(float), stream_),
                  "Generator: logits");
    return out;
}

// The decode step replays the launches of step() only where they take the same
// kernels: the short-table attention (at most 16 blocks of 16 tokens, head_dim
// 64 or 128, a query-head group of 1-16), whose choice depends on the table
// length and so is fixed for the whole generation.
bool Generator::graph_eligible(std::size_t tokens) const {
    if (!graph_replay_ || config_.block_size != 16) return false;
    const std::size_t heads = config_.num_heads;
    const std::size_t kv = config_.num_kv_heads == 0 ? heads : config_.num_kv_heads;
    if (heads == 0 || kv == 0 || heads % kv != 0 || config_.hidden_dim % heads != 0) return false;
    const std::size_t hd = config_.hidden_dim / heads, group = heads / kv;
    const std::size_t blocks = tokens / 16 + (tokens % 16 != 0);
    return blocks <= 16 && (hd == 64 || hd == 128) &&
           (group == 1 || group == 2 || group == 4 || group == 8 || group == 16);
}

bool Generator::prepare_step_graph(std::size_t tokens) {
    const int hd = static_cast<int>(config_.hidden_dim / config_.num_heads);
    const int blocks = static_cast<int>(tokens / 16 + (tokens % 16 != 0));
    if (step_state_ == nullptr) {
        void* d = nullptr;
        detail::check(skv_malloc(&d, 3 * sizeof(std::int32_t)), "Generator: step state");
        step_state_ = static_cast<std::int32_t*>(d);
    }
    if (rope_positions_ < static_cast<int>(tokens)) {
        // The cos/sin pairs forward_into computes on the host, for every position.
        std::vector<float> host(tokens * static_cast<std::size_t>(hd));
        detail::check(skv_rope_cos_sin(hd, 0, static_cast<int>(tokens), host.data()), "Generator: RoPE table");
        void* d = nullptr;
        detail::check(skv_malloc(&d, host.size() * sizeof(float)), "Generator: RoPE table");
        detail::check(skv_memcpy_h2d(d, host.data(), host.size() * sizeof(float), nullptr), "Generator: RoPE table");
        if (rope_table_) {
            (void)skv_device_synchronize();   // the old table may be read by queued replays
            release_step_graph();
            (void)skv_free(rope_table_);
        }
        rope_table_ = static_cast<float*>(d);
        rope_positions_ = static_cast<int>(tokens);
    }
    std::vector<const int*> tables(blocks_.size());
    for (std::size_t l = 0; l < blocks_.size(); ++l) tables[l] = pages_[l].get_device_block_table(0, stream_);
    std::vector<const void*> key = {ids_, flags_, hidden_->raw_data(), logits_->raw_data(), step_state_,
                                    rope_table_, reinterpret_cast<const void*>(static_cast<std::intptr_t>(blocks))};
    for (const int* t : tables) key.push_back(t);
    if (step_graph_ && key == graph_key_) return true;
    (void)skv_stream_synchronize(stream_);
    release_step_graph();

    // Record one step() on a created stream (the null stream cannot be
    // recorded), then put every stream back.
    void* cs = stream_;
    if (cs == nullptr) {
        if (!capture_stream_) detail::check(skv_stream_create(&capture_stream_), "Generator: capture stream");
        cs = capture_stream_;
    }
    void* const saved = stream_;
    auto use_stream = [&](void* st) {
        stream_ = st;
        for (auto& b : blocks_) b.set_stream(st);
    };
    const int dtype = embeddings_->dtype() == DataType::BF16 ? SKV_DTYPE_BF16 : SKV_DTYPE_FP32;
    const int h = static_cast<int>(config_.hidden_dim);
    const int vocab = static_cast<int>(config_.vocab_size);
    auto* x = static_cast<float*>(hidden_->raw_data());
    use_stream(cs);
    bool recorded = true;
    try {
        detail::check(skv_graph_begin_capture(cs), "Generator: step graph");
        try {
            detail::check(skv_embedding_at_f32(embeddings_->raw_data(), dtype, vocab, h, ids_, step_state_, x, flags_,
                                               step_state_ + 2, cs),
                          "Generator: embedding");
            for (std::size_t l = 0; l < blocks_.size() && recorded; ++l)
                recorded = blocks_[l].forward_into_at(*hidden_, *hidden_, step_state_, rope_table_, rope_positions_,
                                                      tables[l], blocks, pools_[l]);
            if (recorded) logits_of(x, static_cast<float*>(logits_->raw_data()));
        } catch (...) {
            (void)skv_graph_abort_capture(cs);
            throw;
        }
        if (!recorded) {
            detail::check(skv_graph_abort_capture(cs), "Generator: step graph");
        } else {
            void* exec = nullptr;
            detail::check(skv_graph_end_capture(cs, &exec), "Generator: step graph");
            step_graph_ = exec;
            graph_key_ = std::move(key);
        }
    } catch (...) {
        use_stream(saved);
        throw;
    }
    use_stream(saved);
    return recorded;
}

void Generator::set_stream(void* stream) {
    stream_ = stream;
    for (auto& b : blocks_) b.set_stream(stream);
}

std::size_t Generator::free_block_count() const noexcept {
    std::size_t total = 0;
    for (const auto& pool : pools_) total += pool.free_count();
    return total;
}

void Generator::validate_prompt(const std::vector<int>& prompt, std::size_t extra) const {
    for (int id : prompt)
        if (id < 0 || static_cast<std::size_t>(id) >= config_.vocab_size)
            throw std::invalid_argument("Generator: prompt token outside vocabulary");
    if (prompt.size() > static_cast<std::size_t>(INT_MAX) - extra)
        throw std::overflow_error("Generator: prompt plus max exceeds INT_MAX");
}

void Generator::begin_sequence(std::size_t tokens) {
    const auto bs = static_cast<std::size_t>(config_.block_size);
    const std::size_t blocks = tokens / bs + (tokens % bs != 0);
    if (blocks > static_cast<std::size_t>(config_.total_blocks))
        throw std::length_error("Generator: prompt plus max exceeds KV capacity");
    if (tokens > ids_capacity_) {
        (void)skv_device_synchronize();
        if (ids_) (void)skv_free(ids_);
        if (host_ids_) (void)skv_host_free(host_ids_);
        if (flags_) (void)skv_free(flags_);
        ids_ = nullptr;
        host_ids_ = nullptr;
        flags_ = nullptr;
        ids_capacity_ = 0;
        flags_capacity_ = 0;
        void* d = nullptr;
        void* hp = nullptr;
        detail::check(skv_malloc(&d, tokens * sizeof(std::int32_t)), "Generator: token buffer");
        ids_ = static_cast<std::int32_t*>(d);
        detail::check(skv_host_alloc(&hp, tokens * sizeof(std::int32_t)), "Generator: token buffer");
        host_ids_ = static_cast<std::int32_t*>(hp);
        ids_capacity_ = tokens;
        // One flag word for the prompt pass, then one per sample and per step.
        detail::check(skv_malloc(&d, (2 * tokens + 2) * sizeof(std::int32_t)), "Generator: flags");
        flags_ = static_cast<std::int32_t*>(d);
        flags_capacity_ = 2 * tokens + 2;
    }
    if (parity_) parity_->reset();
    saved_free_lists_.resize(pools_.size());
    for (std::size_t l = 0; l < pools_.size(); ++l) saved_free_lists_[l] = pools_[l].free_list();
    save_kv_blocks(blocks);
    std::size_t done = 0;
    try {
        for (; done < pages_.size(); ++done) {
            pages_[done].allocate_sequence(0, pools_[done]);
            pages_[done].reserve_device_block_table(blocks);
        }
    } catch (...) {
        for (std::size_t l = 0; l < done; ++l)
            if (pages_[l].has_sequence(0)) pages_[l].free_sequence(0, pools_[l]);
        throw;
    }
}

// The blocks each layer's pool will hand out for `blocks` blocks of one
// sequence (the top of its free stack, in pop order), K and V, copied aside.
void Generator::save_kv_blocks(std::size_t blocks) {
    kv_chunks_ = 0;
    if (pools_.empty() || blocks == 0) return;
    const std::size_t elems = pools_.front().block_elements();
    const std::size_t n = 2 * pools_.size() * blocks;
    kv_chunk_bytes_ = elems * sizeof(std::uint16_t);
    if (n > kv_chunks_capacity_) {
        if (kv_saved_) (void)skv_free(kv_saved_);
        if (kv_chunk_ptrs_) (void)skv_free(kv_chunk_ptrs_);
        if (kv_chunk_host_) (void)skv_host_free(kv_chunk_host_);
        kv_saved_ = nullptr;
        kv_chunk_ptrs_ = nullptr;
        kv_chunk_host_ = nullptr;
        kv_chunks_capacity_ = 0;
        void* d = nullptr;
        detail::check(skv_malloc(&d, n * kv_chunk_bytes_), "Generator: K/V save");
        kv_saved_ = d;
        detail::check(skv_malloc(&d, 2 * n * sizeof(void*)), "Generator: K/V save");
        kv_chunk_ptrs_ = static_cast<void**>(d);
        detail::check(skv_host_alloc(&d, 2 * n * sizeof(void*)), "Generator: K/V save");
        kv_chunk_host_ = static_cast<void**>(d);
        kv_chunks_capacity_ = n;
    }
    std::size_t c = 0;
    for (std::size_t l = 0; l < pools_.size(); ++l) {
        const std::vector<int>& free = saved_free_lists_[l];
        for (std::size_t j = 0; j < blocks && j < free.size(); ++j) {
            const std::size_t id = static_cast<std::size_t>(free[free.size() - 1 - j]);
            for (std::uint16_t* pool : {pools_[l].key_cache(), pools_[l].value_cache()}) {
                kv_chunk_host_[c] = pool + id * elems;
                kv_chunk_host_[n + c] = static_cast<char*>(kv_saved_) + c * kv_chunk_bytes_;
                ++c;
            }
        }
    }
    // c <= n: the halves keep their n-entry offsets.
    for (std::size_t i = c; i < n; ++i) kv_chunk_host_[i] = kv_chunk_host_[n + i] = nullptr;
    detail::check(skv_memcpy_h2d_async(kv_chunk_ptrs_, kv_chunk_host_, 2 * n * sizeof(void*), stream_),
                  "Generator: K/V save");
    kv_half_ = n;
    kv_chunks_ = c;
    const int rc = copy_kv_chunks(0, n);
    if (rc == SKV_ERR_UNSUPPORTED) {
        for (std::size_t i = 0; i < c; ++i)
            detail::check(skv_memcpy_d2d(kv_chunk_host_[n + i], kv_chunk_host_[i], kv_chunk_bytes_, stream_),
                          "Generator: K/V save");
    } else if (rc != SKV_OK) {
        kv_chunks_ = 0;
        detail::check(rc, "Generator: K/V save");
    }
}

// The kv_chunks_ chunks from the addresses at offset `from` of kv_chunk_ptrs_
// to those at offset `to`, in launches of at most 65,535 chunks;
// SKV_ERR_UNSUPPORTED when the chunk size is not a multiple of 16 bytes.
int Generator::copy_kv_chunks(std::size_t from, std::size_t to) noexcept {
    if (kv_chunk_bytes_ % 16 != 0) return SKV_ERR_UNSUPPORTED;
    constexpr std::size_t kMaxChunks = 65535;
    for (std::size_t i = 0; i < kv_chunks_; i += kMaxChunks) {
        const int count = static_cast<int>(std::min(kMaxChunks, kv_chunks_ - i));
        if (int rc = skv_copy_chunks(const_cast<const void* const*>(kv_chunk_ptrs_ + from + i),
                                     kv_chunk_ptrs_ + to + i, count, kv_chunk_bytes_, stream_))
            return rc;
    }
    return SKV_OK;
}

// Frees sequence 0 in every layer and puts each pool's free list back as it
// was before begin_sequence, so consecutive generations use the same block
// ids in the same order, as after the reference's SequenceGuard restore
// (src/generation/generator.cpp:347-371, 639).
void Generator::end_sequence() noexcept {
    (void)skv_stream_synchronize(stream_);
    // The saved K/V blocks back into the pools, complete before generate returns.
    if (kv_chunks_ > 0) {
        if (copy_kv_chunks(kv_half_, 0) != SKV_OK)
            for (std::size_t i = 0; i < kv_chunks_; ++i)
                (void)skv_memcpy_d2d(kv_chunk_host_[i], kv_chunk_host_[kv_half_ + i], kv_chunk_bytes_, stream_);
        (void)skv_stream_synchronize(stream_);
        kv_chunks_ = 0;
    }
    last_tables_.assign(pages_.size(), {});
    for (std::size_t l = 0; l < pages_.size(); ++l) {
        try {
            if (pages_[l].has_sequence(0)) {
                last_tables_[l] = pages_[l].get_state(0).physical_blocks;
                pages_[l].free_sequence(0, pools_[l]);
            }
            if (l < saved_free_lists_.size()) pools_[l].restore_free_list(saved_free_lists_[l]);
        } catch (...) {
        }
    }
}

void Generator::step(int in_index, float* logits, std::int32_t* flags) {
    const int dtype = embeddings_->dtype() == DataType::BF16 ? SKV_DTYPE_BF16 : SKV_DTYPE_FP32;
    const int h = static_cast<int>(config_.hidden_dim);
    const int vocab = static_cast<int>(config_.vocab_size);
    auto* x = static_cast<float*>(hidden_->raw_data());
    detail::check(skv_embedding_f32(embeddings_->raw_data(), dtype, vocab, h, ids_, in_index, x, flags, stream_),
                  "Generator: embedding");
    std::vector<float> gpu_embedding;
    std::vector<std::vector<float>> gpu_layers;
    std::optional<models::TransformerBlock::ParityRow> l0;
    if (parity_ && in_index == 0) gpu_embedding = parity_download(x, config_.hidden_dim);
    for (std::size_t l = 0; l < blocks_.size(); ++l) {
        blocks_[l].forward_into(*hidden_, *hidden_, 0, pages_[l], pools_[l], true);
        if (parity_) {
            if (l == 0 && in_index == 0) l0 = blocks_[0].parity_row(0);
            gpu_layers.push_back(parity_download(x, config_.hidden_dim));
        }
    }
    if (logits != nullptr) logits_of(x, logits);
    if (parity_) parity_pass(in_index, 1, gpu_embedding, gpu_layers, l0 ? &*l0 : nullptr);
}

void Generator::prompt_pass(std::size_t P, float* logits, std::int32_t* flags) {
    const int dtype = embeddings_->dtype() == DataType::BF16 ? SKV_DTYPE_BF16 : SKV_DTYPE_FP32;
    const int h = static_cast<int>(config_.hidden_dim);
    const int vocab = static_cast<int>(config_.vocab_size);
    if (!prompt_rows_ || prompt_rows_->shape()[0] != P)
        prompt_rows_.emplace(std::vector<std::size_t>{P, config_.hidden_dim}, DataType::FP32, Device::GPU);
    auto* rows = static_cast<float*>(prompt_rows_->raw_data());
    constexpr std::size_t kEmbedRows = 65535;  // rows per embedding launch
    for (std::size_t i = 0; i < P; i += kEmbedRows)
        detail::check(skv_embedding_rows_f32(embeddings_->raw_data(), dtype, vocab, h, ids_, static_cast<int>(i),
                                             static_cast<int>(std::min(kEmbedRows, P - i)),
                                             rows + i * config_.hidden_dim, flags, stream_),
                      "Generator: embedding");
    std::vector<float> gpu_embedding;
    std::vector<std::vector<float>> gpu_layers;
    std::optional<models::TransformerBlock::ParityRow> l0;
    if (parity_) gpu_embedding = parity_download(rows, config_.hidden_dim);
    for (std::size_t l = 0; l < blocks_.size(); ++l) {
        blocks_[l].prefill_into(*prompt_rows_, *prompt_rows_, 0, pages_[l], pools_[l]);
        if (parity_) {
            // Layer 0's scratch holds row 0's ops when the prompt was one chunk.
            if (l == 0 && P <= static_cast<std::size_t>(blocks_[0].prefill_chunk_rows()))
                l0 = blocks_[0].parity_row(0);
            gpu_layers.push_back(parity_download(rows, P * config_.hidden_dim));
        }
    }
    logits_of(rows + (P - 1) * config_.hidden_dim, logits);
    if (parity_) parity_pass(0, P, gpu_embedding, gpu_layers, l0 ? &*l0 : nullptr);
}

std::vector<float> Generator::parity_download(const float* device, std::size_t count) {
    std::vector<float> v(count);
    detail::check(skv_stream_synchronize(stream_), "Generator: parity");
    detail::check(skv_memcpy_d2h(v.data(), device, count * sizeof(float), nullptr), "Generator: parity");
    return v;
}

namespace {

// One op of layer 0 in the reference's report format
// (src/models/transformer_block.cpp:63-80).
void parity_op(const char* name, const std::vector<float>& gpu, const std::vector<double>& cpu) {
    if (gpu.empty() || cpu.empty()) return;
    auto at = [](const auto& v, std::size_t i) { return i < v.size() ? static_cast<double>(v[i]) : 0.0; };
    std::fprintf(stderr,
                 "[PARITY L0] %s: max_diff = %.9g, gpu_sample[0..2] = [%.9g, %.9g, %.9g], "
                 "cpu_sample[0..2] = [%.9g, %.9g, %.9g]\n",
                 name, detail::max_abs_diff(gpu, cpu), at(gpu, 0), at(gpu, 1), at(gpu, 2), at(cpu, 0), at(cpu, 1),
                 at(cpu, 2));
}

}  // namespace

void Generator::parity_pass(int first, std::size_t rows, const std::vector<float>& gpu_embedding,
                            const std::vector<std::vector<float>>& gpu,
                            const models::TransformerBlock::ParityRow* l0) {
    const std::size_t H = config_.hidden_dim;
    for (std::size_t r = 0; r < rows; ++r) {
        const int position = first + static_cast<int>(r);
        std::vector<double> x = parity_->embedding(host_ids_[position]);
        if (position == 0) parity_op("embedding", gpu_embedding, x);
        for (std::size_t l = 0; l < parity_->num_layers(); ++l) {
            detail::HostLayerOps ops;
            const bool report_ops = position == 0 && l == 0 && l0 != nullptr;
            x = parity_->layer(l, x, report_ops ? &ops : nullptr);
            if (report_ops) {
                // The values the fused kernels leave in memory (parity_row).
                parity_op("rope_q", l0->q, ops.q_rot);
                parity_op("rope_k", l0->k, ops.k_rot);
                parity_op("v_proj", l0->v, ops.v);
                parity_op("paged_attention", l0->context, ops.context);
                parity_op("out_proj + residual", l0->residual, ops.residual);
                parity_op("swiglu", l0->act, ops.act);
            }
            const std::vector<float> g(gpu[l].begin() + static_cast<std::ptrdiff_t>(r * H),
                                       gpu[l].begin() + static_cast<std::ptrdiff_t>((r + 1) * H));
            std::fprintf(stderr, "[PARITY pos=%d layer=%zu] max_diff = %.9g\n", position, l,
                         detail::max_abs_diff(g, x));
        }
        parity_last_ = std::move(x);
    }
}

void Generator::parity_final(int position) {
    const std::vector<double> norm = parity_->final_norm(parity_last_);
    const std::vector<double> cpu = parity_->logits(norm);
    const std::vector<float> gpu_norm = parity_download(static_cast<const float*>(normed_->raw_data()),
                                                        config_.hidden_dim);
    const std::vector<float> gpu = parity_download(static_cast<const float*>(logits_->raw_data()),
                                                   config_.vocab_size);
    std::fprintf(stderr, "[PARITY pos=%d] final_norm max_diff = %.9g\n", position,
                 detail::max_abs_diff(gpu_norm, norm));
    std::size_t ga = 0, ca = 0;
    for (std::size_t i = 0; i < gpu.size() && i < cpu.size(); ++i) {
        if (gpu[i] > gpu[ga]) ga = i;
        if (cpu[i] > cpu[ca]) ca = i;
    }
    std::fprintf(stderr, "[PARITY FINAL] lm_head logits: max_diff = %.9g, gpu_argmax = %zu, cpu_argmax = %zu\n",
                 detail::max_abs_diff(gpu, cpu), ga, ca);
}

void Generator::logits_of(const float* x, float* logits) {
    const int h = static_cast<int>(config_.hidden_dim);
    const int vocab = static_cast<int>(config_.vocab_size);
    detail::check(skv_rmsnorm_f32(x, static_cast<float*>(normed_->raw_data()),
                                  static_cast<const float*>(final_norm_->gamma().raw_data()), 1, h,
                                  final_norm_->epsilon(), stream_),
                  "Generator: final rmsnorm");
    const Tensor& wt = lm_head_->weight();
    detail::check(skv_linear_f32(static_cast<const float*>(normed_->raw_data()), 1, wt.raw_data(), SKV_DTYPE_BF16,
                                 static_cast<int64_t>(wt.strides()[0]), static_cast<int64_t>(wt.strides()[1]), h,
                                 vocab, nullptr, logits, stream_),
                  "Generator: lm_head");
}

void Generator::raise_flags(std::int32_t flags) const {
    if (flags & SKV_FLAG_NONFINITE_LOGITS)
        throw std::runtime_error(
            "CRITICAL NUMERICAL COLLAPSE: NaN/Inf detected in logits! Safetensors dtype mismatch (FP16 weights "
            "fed to BF16 kernel).");
    if (flags & SKV_FLAG_NONFINITE_SCALED) throw std::invalid_argument("Sampler: scaled logits are not finite");
    if (flags & SKV_FLAG_BAD_DISTRIBUTION) throw std::runtime_error("Sampler: invalid softmax distribution");
    if (flags & SKV_FLAG_BAD_TOKEN) throw std::runtime_error("Generator: token id outside vocabulary");
}

std::vector<int> Generator::generate(const std::vector<int>& prompt, int max_new_tokens) {
    if (prompt.empty() || max_new_tokens < 0)
        throw std::invalid_argument("Generator: nonempty prompt and nonnegative max required");
    validate_prompt(prompt, static_cast<std::size_t>(max_new_tokens));
    if (max_new_tokens == 0 || prompt.back() == config_.eos_token_id) {
        last_tables_.clear();
        return prompt;
    }
    const std::size_t P = prompt.size();
    const std::size_t required = P + static_cast<std::size_t>(max_new_tokens);
    const auto bs = static_cast<std::size_t>(config_.block_size);
    if (required / bs + (required % bs != 0) > static_cast<std::size_t>(config_.total_blocks))
        throw std::length_error("Generator: prompt plus max exceeds KV capacity");
    checked_elements({P, config_.hidden_dim});
    checked_elements({P, config_.intermediate_dim});
    const auto t0 = Clock::now();
    begin_sequence(required);
    std::vector<int> result(prompt);
    try {
        for (std::size_t i = 0; i < P; ++i) host_ids_[i] = prompt[i];
        detail::check(skv_memcpy_h2d_async(ids_, host_ids_, P * sizeof(std::int32_t), stream_), "Generator: prompt");
        // Flag words: [0] the prompt pass; for generated step s, [1 + 2s] its
        // token choice and [2 + 2s] the step that embeds that token and makes
        // the next logits.  Only the words of steps up to an EOS count: steps
        // queued past it never ran in the reference.
        const std::size_t words = 2 * static_cast<std::size_t>(max_new_tokens) + 1;
        detail::check(skv_memset_d8(flags_, 0, words * sizeof(std::int32_t), stream_), "Generator: flags");
        auto* logits = static_cast<float*>(logits_->raw_data());
        const int vocab = static_cast<int>(config_.vocab_size);
        if (P >= 2) prompt_pass(P, logits, flags_);
        else step(0, logits, flags_);
        // The logits the first generated token is chosen from (the
        // reference reports them at its first step, src/generation/generator.cpp:741-769).
        if (parity_) parity_final(static_cast<int>(P) - 1);
        // Decode steps replayed from a graph where that gives the same launches.
        const bool replay = max_new_tokens >= 2 && graph_eligible(required) && prepare_step_graph(required);
        last_replayed_ = replay;

        const int R = static_cast<int>(step_events_.size());
        // The sampler's stream before each queued draw (a ring as deep as the
        // lookahead), to put it back to the state after the EOS step's draw.
        const bool draws = sampler_.config().temperature != 0.0f && vocab >= 2;
        std::vector<std::mt19937> rng_before(draws ? static_cast<std::size_t>(R) : 0);
        int checked = 0;      // generated tokens the host has read
        bool stop = false;    // EOS seen at generated index `checked - 1`
        int queued = 0;       // generated tokens queued
        auto read_one = [&](bool wait) {
            void* ev = step_events_[checked % R];
            if (wait) {
                detail::check(skv_event_synchronize(ev), "Generator: token copy");
            } else {
                int done = 0;
                detail::check(skv_event_query(ev, &done), "Generator: token copy");
                if (!done) return false;
            }
            const int tok = host_ids_[P + checked];
            ++checked;
            if (tok == config_.eos_token_id) stop = true;
            return true;
        };
        for (int s = 0; s < max_new_tokens && !stop; ++s) {
            const int pos = static_cast<int>(P) + s;
            if (draws) rng_before[s % R] = sampler_.rng_state();
            sampler_.sample_into(logits, vocab, ids_, pos, flags_ + 1 + 2 * s, stream_);
            detail::check(skv_memcpy_d2h_async(host_ids_ + pos, ids_ + pos, sizeof(std::int32_t), stream_),
                          "Generator: token copy");
            detail::check(skv_event_record(step_events_[s % R], stream_), "Generator: token copy");
            queued = s + 1;
            while (!stop && checked < queued && read_one(queued - checked > kLookahead)) {
            }
            if (stop || s + 1 == max_new_tokens) break;
            if (replay) {
                // forward_into's host bookkeeping for every layer, then the
                // step's position, context length and flag word for the replay.
                for (std::size_t l = 0; l < pages_.size(); ++l) {
                    pages_[l].append_token(0, pools_[l]);
                    (void)pages_[l].get_device_block_table(0, stream_);
                }
                const std::int32_t state[3] = {pos, pos + 1, 2 + 2 * s};
                detail::check(skv_write_i32(step_state_, state, 3, stream_), "Generator: step state");
                detail::check(skv_graph_launch(step_graph_, stream_), "Generator: step replay");
            } else {
                step(pos, logits, flags_ + 2 + 2 * s);  // embeds the token just chosen
            }
        }
        while (!stop && checked < queued) read_one(true);
        // Draws made for steps queued past the EOS step are taken back.
        if (draws && queued > checked) sampler_.set_rng_state(rng_before[checked % R]);
        detail::check(skv_stream_synchronize(stream_), "Generator: generate");
        std::vector<std::int32_t> flag_words(2 * static_cast<std::size_t>(checked));
        detail::check(skv_memcpy_d2h(flag_words.data(), flags_, flag_words.size() * sizeof(std::int32_t), stream_),
                      "Generator: flags");
        std::int32_t flags = 0;
        for (std::int32_t f : flag_words) flags |= f;
        raise_flags(flags);
        for (int s = 0; s < checked; ++s) result.push_back(host_ids_[P + s]);
    } catch (...) {
        end_sequence();
        throw;
    }
    end_sequence();
    last_generation_ms_ = std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
    return result;
}

std::vector<float> Generator::forced_logits(const std::vector<int>& tokens, std::size_t n_prompt) {
    if (n_prompt == 0 || n_prompt > tokens.size())
        throw std::invalid_argument("Generator: forced_logits needs 1 <= n_prompt <= tokens.size()");
    validate_prompt(tokens, 0);
    const std::size_t N = tokens.size();
    const std::size_t rows = N - n_prompt + 1;
    const std::size_t vocab = config_.vocab_size;
    checked_elements({rows, vocab});
    begin_sequence(N);
    std::vector<float> out(rows * vocab);
    try {
        Tensor all({rows, vocab}, DataType::FP32, Device::GPU);
        auto* base = static_cast<float*>(all.raw_data());
        for (std::size_t i = 0; i < N; ++i) host_ids_[i] = tokens[i];
        detail::check(skv_memcpy_h2d_async(ids_, host_ids_, N * sizeof(std::int32_t), stream_), "Generator: tokens");
        detail::check(skv_memset_d8(flags_, 0, sizeof(std::int32_t), stream_), "Generator: flags");
        if (n_prompt >= 2) prompt_pass(n_prompt, base, flags_);
        else step(0, base, flags_);
        for (std::size_t r = 1; r < rows; ++r) step(static_cast<int>(n_prompt - 1 + r), base + r * vocab, flags_);
        detail::check(skv_stream_synchronize(stream_), "Generator: forced_logits");
        detail::check(skv_memcpy_d2h(out.data(), base, out.size() * sizeof(float), stream_), "Generator: logits");
        std::int32_t flags = 0;
        detail::check(skv_memcpy_d2h(&flags, flags_, sizeof(flags), stream_), "Generator: flags");
        raise_flags(flags & ~SKV_FLAG_NONFINITE_LOGITS);
    } catch (...) {
        end_sequence();
        throw;
    }
    end_sequence();
    return out;
}

}  // namespace generation
}  // namespace stratakv

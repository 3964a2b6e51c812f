// generator.h -- token generation over the layer stack, on the device.
//
// Interface of the reference's stratakv::generation::Generator
// (include/stratakv/generation/generator.h:9-124, src/generation/generator.cpp):
// the configuration, the weight schema (Hugging Face Llama names, or the
// one-layer "block.*" schema), the per-layer BlockPool / PageTable, and
// generate(prompt, max_new_tokens) with its validation and EOS rule.
//
// What runs where: every token's embedding lookup, the layers'
// TransformerBlock::forward_into, the final RMSNorm, the lm_head GEMV and the
// token choice (skv_argmax_f32 / skv_sample_f32) are queued on one stream, and
// the chosen id stays in device memory where the next step's embedding lookup
// reads it.  The host queues steps ahead of the GPU and learns each token from
// a small asynchronous copy, so it waits only to stop at EOS (at most
// kLookahead steps are queued past the step it has checked).  The reference
// instead copies the full logits to the host and samples there every token
// (src/generation/generator.cpp:700-735).
//
// Weights may be the host FP32 tensors of io::load_safetensors (uploaded, and
// linears truncated to BF16, as the reference's GPU path does) or the device
// tensors of io::load_safetensors_device (used in place).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <vector>

#include "stratakv/generation/sampler.h"
#include "stratakv/io/safetensors.h"
#include "stratakv/memory/block_pool.h"
#include "stratakv/memory/page_table.h"
#include "stratakv/models/transformer_block.h"

namespace stratakv {
namespace detail {
class ParityModel;
}
namespace generation {

struct GeneratorConfig {
    Device device = Device::GPU;
    std::size_t hidden_dim = 0;
    std::size_t intermediate_dim = 0;
    std::size_t num_heads = 0;
    std::size_t num_kv_heads = 0;  // zero selects num_heads (MHA)
    std::size_t num_layers = 0;
    int total_blocks = 0;
    int block_size = 0;
    std::size_t vocab_size = 0;
    int eos_token_id = -1;  // disabled when -1
    SamplerConfig sampler{0.0f, 0, 1.0f};

    GeneratorConfig() = default;
    GeneratorConfig(std::size_t hidden, std::size_t intermediate, std::size_t heads, int total, int block,
                    std::size_t vocab, int eos)
        : hidden_dim(hidden), intermediate_dim(intermediate), num_heads(heads), num_kv_heads(0),
          num_layers(1), total_blocks(total), block_size(block), vocab_size(vocab), eos_token_id(eos) {}
    GeneratorConfig(std::size_t hidden, std::size_t intermediate, std::size_t heads, std::size_t layers,
                    int total, int block, std::size_t vocab, int eos)
        : hidden_dim(hidden), intermediate_dim(intermediate), num_heads(heads), num_kv_heads(0),
          num_layers(layers), total_blocks(total), block_size(block), vocab_size(vocab), eos_token_id(eos) {}
    GeneratorConfig(std::size_t hidden, std::size_t intermediate, std::size_t heads, std::size_t kv_heads,
                    std::size_t layers, int total, int block, std::size_t vocab, int eos)
        : hidden_dim(hidden), intermediate_dim(intermediate), num_heads(heads), num_kv_heads(kv_heads),
          num_layers(layers), total_blocks(total), block_size(block), vocab_size(vocab), eos_token_id(eos) {}
};

class Generator {
public:
    // Steps queued beyond the last one whose token the host has seen.
    static constexpr int kLookahead = 8;

    Generator(GeneratorConfig config, io::WeightMap weights);
    ~Generator();
    Generator(const Generator&) = delete;
    Generator& operator=(const Generator&) = delete;

    std::vector<int> generate(const std::vector<int>& prompt, int max_new_tokens);
    std::size_t free_block_count() const noexcept;
    double last_generation_ms() const noexcept { return last_generation_ms_; }
    double initialization_ms() const noexcept { return initialization_ms_; }

    // Extensions (no counterpart in the reference).
    // Stream for all device work (a hipStream_t; nullptr = default stream).
    void set_stream(void* stream);
    // The block table of sequence 0 in `layer` during the last generate /
    // forced_logits call (the ids it used, in table order; empty when that
    // call returned without running the model).
    std::vector<int> last_block_table(std::size_t layer) const {
        return layer < last_tables_.size() ? last_tables_[layer] : std::vector<int>{};
    }
    // Layer `layer`'s block and KV pool (read-only; no counterpart in the
    // reference, whose pools are private).  generate puts every block it
    // wrote back as it was, so a pool holds the same bytes before and after.
    const models::TransformerBlock& block(std::size_t layer) const { return blocks_.at(layer); }
    const memory::BlockPool& block_pool(std::size_t layer) const { return pools_.at(layer); }
    // Reseed the sampler's uniform stream (the reference seeds it from
    // std::random_device, as the constructor here does).
    void seed_sampler(std::uint32_t seed) { sampler_ = Sampler(config_.sampler, seed); }
    // Generations whose context fits the short-table decode (prompt + max new
    // tokens within 16 blocks, block size 16, head_dim 64 or 128, 1-16 query
    // heads per kv head, weights in the fused kernels' layout) replay each
    // decode step -- embedding, every layer, final norm and lm_head -- from one
    // HIP graph, with the position, context length and flag word in device
    // memory (TransformerBlock::forward_into_at).  The token choice before each
    // step stays a launch of its own.  The outputs are the bits of the
    // step-by-step launches.  On by default; false runs every step eagerly.
    void set_graph_replay(bool enabled);
    bool graph_replay() const noexcept { return graph_replay_; }
    // Whether the last generate call replayed its steps from a graph.
    bool last_generation_replayed() const noexcept { return last_replayed_; }
    // The logits left by the last generate call (those of the last token's
    // choice), copied to the host; empty before any call.
    std::vector<float> last_logits() const;
    // Teacher forcing: tokens[0..n_prompt) are the prompt, then every later
    // token is fed in turn.  Returns the logits after each of the positions
    // n_prompt-1 .. tokens.size()-1, row-major [(tokens.size() - n_prompt + 1) x vocab].
    std::vector<float> forced_logits(const std::vector<int>& tokens, std::size_t n_prompt);

private:
    void validate_prompt(const std::vector<int>& prompt, std::size_t extra) const;
    void begin_sequence(std::size_t tokens);
    void save_kv_blocks(std::size_t blocks);
    int copy_kv_chunks(std::size_t from, std::size_t to) noexcept;
    void end_sequence() noexcept;
    // One decode step: embedding of ids_[in_index], all layers, final norm,
    // lm_head into `logits` (device [vocab]); data errors go to *flags.
    void step(int in_index, float* logits, std::int32_t* flags);
    // The prompt ids_[0 .. P): all P embeddings, every layer over the P rows
    // at once (TransformerBlock::prefill_into), then the logits of the last row.
    void prompt_pass(std::size_t P, float* logits, std::int32_t* flags);
    // Final norm + lm_head of one hidden row into `logits`.
    void logits_of(const float* x, float* logits);
    void raise_flags(std::int32_t flags) const;
    // Whether generate may replay steps of a `tokens`-token context from a graph.
    bool graph_eligible(std::size_t tokens) const;
    // The step graph for this generation (captured, or the cached one when the
    // buffers and tables it was recorded with are unchanged); false when a
    // layer's weights do not allow the fused kernels.
    bool prepare_step_graph(std::size_t tokens);
    void release_step_graph() noexcept;
    // STRATAKV_PARITY=1: the host model's pass over `rows` tokens at positions
    // first, first + 1, ... (ids host_ids_[first ..]), each layer's output
    // against the GPU's (gpu[layer] holds the rows), printed per position and
    // layer; with first == 0 also the embedding and layer 0's ops against
    // `l0` (row 0 of layer 0's scratch).
    void parity_pass(int first, std::size_t rows, const std::vector<float>& gpu_embedding,
                     const std::vector<std::vector<float>>& gpu, const models::TransformerBlock::ParityRow* l0);
    // The final norm and logits of the host model's last hidden row against
    // the GPU's (normed_ and logits_), at `position`.
    void parity_final(int position);
    std::vector<float> parity_download(const float* device, std::size_t count);

    GeneratorConfig config_;
    void* stream_ = nullptr;
    std::vector<models::TransformerBlock> blocks_;
    std::vector<memory::BlockPool> pools_;
    std::vector<memory::PageTable> pages_;
    Sampler sampler_;
    std::optional<Tensor> embeddings_;  // [vocab, hidden], BF16 or FP32, device
    std::optional<layers::RMSNorm> final_norm_;
    std::optional<layers::Linear> lm_head_;  // [hidden, vocab] view of BF16 [vocab, hidden] rows
    std::optional<Tensor> hidden_;           // [1, hidden] FP32: embedding, then the layer stream
    std::optional<Tensor> normed_;           // [1, hidden] FP32
    std::optional<Tensor> prompt_rows_;      // [P, hidden] FP32 of the last prompt length
    std::optional<Tensor> logits_;           // [1, vocab] FP32
    std::int32_t* ids_ = nullptr;            // device token ids, capacity ids_capacity_
    std::size_t ids_capacity_ = 0;
    std::int32_t* flags_ = nullptr;          // device SKV_FLAG_* words: prompt, then sample / step pairs
    std::size_t flags_capacity_ = 0;
    std::int32_t* host_ids_ = nullptr;       // page-locked copies of the chosen ids
    std::vector<void*> step_events_;         // ring of kLookahead + 1 events
    // Free lists saved by begin_sequence and put back by end_sequence, and
    // the tables of the last sequence.
    std::vector<std::vector<int>> saved_free_lists_;
    std::vector<std::vector<int>> last_tables_;
    // The K/V blocks a generation may write (the next blocks each pool hands
    // out), saved by begin_sequence and put back by end_sequence, so the pools
    // hold the same bytes before and after generate, as after the reference's
    // SequenceGuard restores its pool copies (src/generation/generator.cpp:
    // 347-371).
    void* kv_saved_ = nullptr;              // device [chunks][kv_chunk_bytes_]
    void** kv_chunk_ptrs_ = nullptr;        // device [2][chunks]: pool block addresses, then their saved copies
    void** kv_chunk_host_ = nullptr;        // page-locked staging of kv_chunk_ptrs_
    std::size_t kv_chunks_capacity_ = 0;
    std::size_t kv_chunks_ = 0;             // chunks saved by the current sequence
    std::size_t kv_half_ = 0;               // offset of the saved copies' half of kv_chunk_ptrs_
    std::size_t kv_chunk_bytes_ = 0;
    double last_generation_ms_ = 0.0;
    double initialization_ms_ = 0.0;
    // Graph replay of the greedy decode step.
    bool graph_replay_ = true;
    bool last_replayed_ = false;
    void* capture_stream_ = nullptr;          // created for capture when stream_ is the null stream
    void* step_graph_ = nullptr;              // instantiated graph of one decode step
    std::vector<const void*> graph_key_;      // buffers and tables step_graph_ was recorded with
    std::int32_t* step_state_ = nullptr;      // device [position, context length, step flag word]
    float* rope_table_ = nullptr;             // device cos/sin pairs of positions [0, rope_positions_)
    int rope_positions_ = 0;
    // STRATAKV_PARITY=1 (graph replay then stays off).
    std::unique_ptr<detail::ParityModel> parity_;
    std::vector<double> parity_last_;   // the host model's last hidden row
};

}  // namespace generation
}  // namespace stratakv

// generate.cpp -- config 1 end to end: Generator::generate of a
// TinyLlama-shaped model (22 layers, hidden 2048, 32 Q / 4 KV heads, FFN 5632,
// vocab 32000, 1,024-block pool per layer, block size 16), 16 prompt tokens and
// 128 greedy tokens, as the reference CLI runs it (src/cli.cpp:260-311).
//
// Weights: bf16 N(0, 0.02) generated on the device from a seed (norm gammas
// 1.0), or a safetensors checkpoint loaded with io::load_safetensors_device
// (then the load is timed too).  Prints one JSON line.
//   bench_generate [--checkpoint PATH] [--repeat N] [--new N] [--prompt N] [--eager]
// --prompt N: N prompt tokens (the 16 below, then ids from a fixed 32-bit LCG)
// instead of 16, to time the prompt pass on long prompts.  --eager: every decode
// step launched one kernel at a time (Generator::set_graph_replay(false)).
// Also reported: the process's first generation (first_call_ms) and, for a
// prompt one token shorter than any run before, its first and second
// generation of one token (unseen_length_*_ms).
#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>
#include <vector>

#include "stratakv/generation/generator.h"
#include "stratakv/io/safetensors.h"
#include "stratakv_amd.h"

using namespace stratakv;

namespace {

void ok_or_die(int rc, const char* what) {
    if (rc != SKV_OK) throw std::runtime_error(std::string(what) + ": " + skv_last_error());
}

constexpr std::size_t kLayers = 22, kHidden = 2048, kInter = 5632, kHeads = 32, kKv = 4, kVocab = 32000;

io::WeightMap synthetic_weights() {
    io::WeightMap w;
    std::uint64_t seed = 0x5EED1000u;
    auto matrix = [&](const std::string& name, std::size_t rows, std::size_t cols) {
        Tensor t({rows, cols}, DataType::BF16, Device::GPU);
        ok_or_die(skv_fill_normal_scaled_bf16(static_cast<std::uint16_t*>(t.raw_data()), rows * cols, seed++, 0,
                                              0.02f, nullptr),
                  "weight fill");
        w.emplace(name, std::move(t));
    };
    auto norm = [&](const std::string& name) {
        Tensor t({kHidden}, DataType::BF16, Device::GPU);
        ok_or_die(skv_fill_u16(static_cast<std::uint16_t*>(t.raw_data()), kHidden, 0x3F80, nullptr), "norm fill");
        w.emplace(name, std::move(t));
    };
    const std::size_t kvd = kKv * (kHidden / kHeads);
    matrix("model.embed_tokens.weight", kVocab, kHidden);
    for (std::size_t l = 0; l < kLayers; ++l) {
        const std::string p = "model.layers." + std::to_string(l) + ".";
        norm(p + "input_layernorm.weight");
        matrix(p + "self_attn.q_proj.weight", kHidden, kHidden);
        matrix(p + "self_attn.k_proj.weight", kvd, kHidden);
        matrix(p + "self_attn.v_proj.weight", kvd, kHidden);
        matrix(p + "self_attn.o_proj.weight", kHidden, kHidden);
        norm(p + "post_attention_layernorm.weight");
        matrix(p + "mlp.gate_proj.weight", kInter, kHidden);
        matrix(p + "mlp.up_proj.weight", kInter, kHidden);
        matrix(p + "mlp.down_proj.weight", kHidden, kInter);
    }
    norm("model.norm.weight");
    matrix("lm_head.weight", kVocab, kHidden);
    ok_or_die(skv_device_synchronize(), "weight fill");
    return w;
}

double median(std::vector<double> v) {
    std::sort(v.begin(), v.end());
    return v[v.size() / 2];
}

}  // namespace

int main(int argc, char** argv) {
    try {
        std::string checkpoint;
        int repeat = 5, n_new = 128, n_prompt = 16;
        bool eager = false;
        for (int i = 1; i < argc; ++i) {
            const std::string a = argv[i];
            if (a == "--checkpoint" && i + 1 < argc) checkpoint = argv[++i];
            else if (a == "--repeat" && i + 1 < argc) repeat = std::max(1, std::atoi(argv[++i]));
            else if (a == "--new" && i + 1 < argc) n_new = std::max(1, std::atoi(argv[++i]));
            else if (a == "--prompt" && i + 1 < argc) n_prompt = std::max(1, std::atoi(argv[++i]));
            else if (a == "--eager") eager = true;
        }
        int devices = 0;
        if (skv_device_count(&devices) != SKV_OK || devices == 0) {
            std::fprintf(stderr, "bench_generate: no GPU\n");
            return 77;
        }
        double load_ms = 0.0;
        io::LoadBreakdown bd;
        io::WeightMap weights;
        if (!checkpoint.empty()) {
            const auto t0 = std::chrono::steady_clock::now();
            weights = io::load_safetensors_device(checkpoint);
            load_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
            bd = io::last_load_breakdown();
        } else {
            weights = synthetic_weights();
        }
        generation::GeneratorConfig cfg(kHidden, kInter, kHeads, kKv, kLayers, 1024, 16, kVocab, -1);
        generation::Generator gen(cfg, std::move(weights));
        if (eager) gen.set_graph_replay(false);
        // 16 prompt ids as numpy default_rng(42).integers(0, 32000, 16).
        std::vector<int> prompt = {2856, 24766, 20946, 14044, 13856, 27475, 2750, 22315,
                                   6447, 3013,  16847, 31219, 23544, 24356, 22959, 25154};
        prompt.resize(std::min<std::size_t>(prompt.size(), static_cast<std::size_t>(n_prompt)));
        for (std::uint32_t x = 12345u; prompt.size() < static_cast<std::size_t>(n_prompt);) {
            x = x * 1664525u + 1013904223u;
            prompt.push_back(static_cast<int>((x >> 8) % kVocab));
        }
        std::vector<int> out = gen.generate(prompt, n_new);  // warmup: the process's first generation
        const double first_call_ms = gen.last_generation_ms();
        std::vector<double> full, one;
        bool replayed = false;
        for (int r = 0; r < repeat; ++r) {
            out = gen.generate(prompt, n_new);
            replayed = gen.last_generation_replayed();
            full.push_back(gen.last_generation_ms());
            (void)gen.generate(prompt, 1);
            one.push_back(gen.last_generation_ms());
        }
        // A prompt length this process has not run (one token shorter), with
        // one new token: its first call (new shapes for the library GEMMs of
        // a long prompt) and its second.
        double unseen_first_ms = 0.0, unseen_second_ms = 0.0;
        if (prompt.size() > 1) {
            const std::vector<int> shorter(prompt.begin(), prompt.end() - 1);
            (void)gen.generate(shorter, 1);
            unseen_first_ms = gen.last_generation_ms();
            (void)gen.generate(shorter, 1);
            unseen_second_ms = gen.last_generation_ms();
        }
        const double ms = median(full), ms1 = median(one);
        const double per_token = (ms - ms1) / std::max(1, n_new - 1);
        std::printf("{\"layers\": %zu, \"prompt\": %zu, \"new_tokens\": %zu, \"gen_ms\": %.4f, "
                    "\"tokens_per_s\": %.2f, \"prefill_and_first_token_ms\": %.4f, \"decode_ms_per_token\": %.5f, "
                    "\"decode_tokens_per_s\": %.2f, \"init_ms\": %.2f, \"load_ms\": %.2f, "
                    "\"load_payload_bytes\": %zu, \"load_decode_ms\": %.2f, \"checkpoint\": %s, \"repeat\": %d, "
                    "\"graph_replay\": %s, \"first_call_ms\": %.4f, \"unseen_length_first_ms\": %.4f, "
                    "\"unseen_length_second_ms\": %.4f}\n",
                    kLayers, prompt.size(), out.size() - prompt.size(), ms,
                    (out.size() - prompt.size()) / (ms / 1e3), ms1, per_token, 1e3 / per_token,
                    gen.initialization_ms(), load_ms, bd.payload_bytes, bd.tensor_decode_ms,
                    checkpoint.empty() ? "false" : "true", repeat, replayed ? "true" : "false", first_call_ms,
                    unseen_first_ms, unseen_second_ms);
        return 0;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "bench_generate: %s\n", e.what());
        return 1;
    }
}

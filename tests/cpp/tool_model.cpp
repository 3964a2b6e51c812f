// tool_model.cpp -- command-line driver of the C++ model-boundary API for the
// Python tests (tests/test_model_*.py, tests/test_gpu_model.py).
//
//   tool_model load-host <ckpt> [--require-mapped] [--dump NAME OUT]
//       io::load_safetensors; prints {"ok": true, "count": N} or
//       {"ok": false, "error": "..."}; --dump writes NAME's FP32 values.
//   tool_model load-device <ckpt> [--dump NAME OUT]
//       io::load_safetensors_device; --dump writes NAME's raw device bytes
//       and reports its dtype.
//   tool_model transpose IN OUT_F IN_F OUT
//       io::load_linear_bf16_transposed of an FP32 [OUT_F, IN_F] file.
//   tool_model generate <ckpt> MAX_NEW EOS [--host-loader] [--temp T] [--top-k K] [--top-p P]
//       [--repeat N] [--seed S] [--first-max M] -- PROMPT...
//       [--top-k K] [--top-p P] [--repeat N] -- PROMPT...
//       Generator::generate; prints tokens and timings.
//   tool_model forced <ckpt> N_PROMPT OUT [--host-loader] -- TOKENS...
//       Generator::forced_logits; writes [rows x vocab] FP32 logits.
// Model dimensions are inferred from the checkpoint the way the reference's
// CLI does (src/cli.cpp:80-140).
#include <chrono>
#include <cstdio>
#include <cstring>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

#include "stratakv/generation/generator.h"
#include "stratakv/io/safetensors.h"
#include "stratakv_amd.h"

using namespace stratakv;

namespace {

std::string json_escape(const std::string& s) {
    std::string o;
    for (char c : s) {
        if (c == '"' || c == '\\') o += '\\';
        if (static_cast<unsigned char>(c) < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", c);
            o += buf;
            continue;
        }
        o += c;
    }
    return o;
}

void write_file(const std::string& path, const void* data, std::size_t bytes) {
    std::ofstream f(path, std::ios::binary);
    f.write(static_cast<const char*>(data), static_cast<std::streamsize>(bytes));
    if (!f) throw std::runtime_error("cannot write " + path);
}

std::vector<char> read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    return std::vector<char>(std::istreambuf_iterator<char>(f), {});
}

struct Dims {
    std::size_t hidden = 0, inter = 0, heads = 0, kv_heads = 0, layers = 0, vocab = 0;
};

Dims infer(const io::WeightMap& w) {
    auto get = [&](std::initializer_list<const char*> names) -> const Tensor& {
        for (const char* n : names) {
            auto it = w.find(n);
            if (it != w.end()) return it->second;
        }
        throw std::invalid_argument("checkpoint is missing a required architecture weight");
    };
    const Tensor& emb = get({"model.embed_tokens.weight", "tok_embeddings.weight"});
    Dims d;
    d.vocab = emb.shape()[0];
    d.hidden = emb.shape()[1];
    const bool llama = w.count("model.layers.0.input_layernorm.weight") != 0;
    if (llama) {
        while (w.count("model.layers." + std::to_string(d.layers) + ".input_layernorm.weight")) ++d.layers;
    } else {
        d.layers = 1;
    }
    const Tensor& gate = llama ? get({"model.layers.0.mlp.gate_proj.weight"}) : get({"block.ffn.up_proj.weight"});
    const Tensor& k = llama ? get({"model.layers.0.self_attn.k_proj.weight"}) : get({"block.attn.k_proj.weight"});
    const Tensor& q = llama ? get({"model.layers.0.self_attn.q_proj.weight"}) : get({"block.attn.q_proj.weight"});
    d.inter = gate.shape()[0];
    std::size_t hd = 0;
    for (std::size_t c : {64, 128, 80, 96, 32, 16, 8, 4, 2, 1})
        if (d.hidden % c == 0 && k.shape()[0] % c == 0) {
            hd = c;
            break;
        }
    d.heads = q.shape()[0] / hd;
    d.kv_heads = k.shape()[0] / hd;
    return d;
}

generation::GeneratorConfig config_for(const Dims& d, int eos) {
    generation::GeneratorConfig c;
    c.device = Device::GPU;
    c.hidden_dim = d.hidden;
    c.intermediate_dim = d.inter;
    c.num_heads = d.heads;
    c.num_kv_heads = d.kv_heads;
    c.num_layers = d.layers;
    c.total_blocks = 1024;  // the reference CLI's pool (src/cli.cpp:276-277)
    c.block_size = 16;
    c.vocab_size = d.vocab;
    c.eos_token_id = eos;
    return c;
}

int cmd_load(bool device, int argc, char** argv) {
    const std::string path = argv[2];
    bool mapped = false;
    std::string name, out;
    for (int i = 3; i < argc; ++i) {
        const std::string a = argv[i];
        if (a == "--require-mapped") mapped = true;
        if (a == "--dump" && i + 2 < argc) {
            name = argv[i + 1];
            out = argv[i + 2];
            i += 2;
        }
    }
    try {
        auto w = device ? io::load_safetensors_device(path) : io::load_safetensors(path, mapped);
        const char* dtype = "";
        if (!name.empty()) {
            auto it = w.find(name);
            if (it == w.end()) throw std::runtime_error("no tensor " + name);
            const Tensor host = it->second.to(Device::CPU);
            dtype = host.dtype() == DataType::BF16 ? "BF16" : "FP32";
            write_file(out, host.raw_data(), host.num_elements() * host.element_size());
        }
        const auto bd = io::last_load_breakdown();
        std::printf("{\"ok\": true, \"count\": %zu, \"dtype\": \"%s\", \"payload_bytes\": %zu, "
                    "\"open_ms\": %.3f, \"parse_ms\": %.3f, \"decode_ms\": %.3f}\n",
                    w.size(), dtype, bd.payload_bytes, bd.mmap_open_ms, bd.header_parse_ms, bd.tensor_decode_ms);
    } catch (const std::exception& e) {
        std::printf("{\"ok\": false, \"error\": \"%s\"}\n", json_escape(e.what()).c_str());
    }
    return 0;
}

int cmd_transpose(char** argv) {
    const auto raw = read_file(argv[2]);
    const std::size_t out_f = std::stoul(argv[3]), in_f = std::stoul(argv[4]);
    Tensor src({out_f, in_f});
    if (raw.size() != out_f * in_f * sizeof(float)) throw std::runtime_error("size mismatch");
    std::copy(raw.begin(), raw.end(), static_cast<char*>(src.raw_data()));
    const Tensor r = io::load_linear_bf16_transposed(src, out_f, in_f);
    write_file(argv[5], r.raw_data(), r.num_elements() * 2);
    return 0;
}

struct GenArgs {
    std::string path;
    bool host_loader = false;
    generation::SamplerConfig sampler{0.0f, 0, 1.0f};
    int repeat = 1;
    long long seed = -1;  // >= 0: Generator::seed_sampler
    int first_max = -1;   // >= 0: max_new of the first call (later calls use MAX_NEW)
    bool eager = false;   // Generator::set_graph_replay(false)
    bool check_pools = false;   // fill the pools with a pattern, report whether generate leaves them unchanged
    std::vector<int> tokens;
};

GenArgs parse_gen(int first, int argc, char** argv) {
    GenArgs a;
    int i = first;
    for (; i < argc; ++i) {
        const std::string s = argv[i];
        if (s == "--") {
            ++i;
            break;
        }
        if (s == "--host-loader") a.host_loader = true;
        else if (s == "--temp") a.sampler.temperature = std::stof(argv[++i]);
        else if (s == "--top-k") a.sampler.top_k = std::stoi(argv[++i]);
        else if (s == "--top-p") a.sampler.top_p = std::stof(argv[++i]);
        else if (s == "--repeat") a.repeat = std::stoi(argv[++i]);
        else if (s == "--seed") a.seed = std::stoll(argv[++i]);
        else if (s == "--first-max") a.first_max = std::stoi(argv[++i]);
        else if (s == "--eager") a.eager = true;
        else if (s == "--check-pools") a.check_pools = true;
    }
    for (; i < argc; ++i) a.tokens.push_back(std::stoi(argv[i]));
    return a;
}

struct Loaded {
    io::WeightMap weights;
    Dims dims;
    double load_ms = 0.0;
    io::LoadBreakdown breakdown;
};

Loaded load_model(const GenArgs& a) {
    Loaded l;
    const auto t0 = std::chrono::steady_clock::now();
    l.weights = a.host_loader ? io::load_safetensors(a.path) : io::load_safetensors_device(a.path);
    l.load_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    l.breakdown = io::last_load_breakdown();
    l.dims = infer(l.weights);
    return l;
}

int cmd_generate(int argc, char** argv) {
    GenArgs a = parse_gen(5, argc, argv);
    a.path = argv[2];
    const int max_new = std::stoi(argv[3]);
    const int eos = std::stoi(argv[4]);
    try {
        Loaded l = load_model(a);
        auto cfg = config_for(l.dims, eos);
        cfg.sampler = a.sampler;
        generation::Generator gen(cfg, std::move(l.weights));
        if (a.seed >= 0) gen.seed_sampler(static_cast<std::uint32_t>(a.seed));
        if (a.eager) gen.set_graph_replay(false);
        // FNV-1a over every layer's K and V pool bytes.
        auto pools_hash = [&]() {
            std::uint64_t hsh = 1469598103934665603ull;
            for (std::size_t ly = 0; ly < l.dims.layers; ++ly) {
                const memory::BlockPool& p = gen.block_pool(ly);
                const std::size_t n = static_cast<std::size_t>(p.total_blocks()) * p.block_elements();
                std::vector<std::uint16_t> host(n);
                for (const std::uint16_t* pool : {p.key_cache(), p.value_cache()}) {
                    if (skv_memcpy_d2h(host.data(), pool, n * 2, nullptr) != SKV_OK)
                        throw std::runtime_error(skv_last_error());
                    for (std::uint16_t v : host)
                        for (int b = 0; b < 2; ++b) hsh = (hsh ^ ((v >> (8 * b)) & 0xFFu)) * 1099511628211ull;
                }
            }
            return hsh;
        };
        std::uint64_t before = 0;
        if (a.check_pools) {
            for (std::size_t ly = 0; ly < l.dims.layers; ++ly) {
                const memory::BlockPool& p = gen.block_pool(ly);
                const std::size_t n = static_cast<std::size_t>(p.total_blocks()) * p.block_elements();
                if (skv_fill_normal_bf16(const_cast<std::uint16_t*>(p.key_cache()), n, 7 + 2 * ly, 0, nullptr) ||
                    skv_fill_normal_bf16(const_cast<std::uint16_t*>(p.value_cache()), n, 8 + 2 * ly, 0, nullptr))
                    throw std::runtime_error(skv_last_error());
            }
            before = pools_hash();
        }
        std::vector<int> pools_unchanged;
        std::vector<std::size_t> blocks_visited;
        std::vector<int> out;
        std::vector<std::vector<int>> runs, tables;
        std::vector<double> gen_ms;
        std::vector<int> replayed;
        std::vector<std::uint64_t> logit_hashes;
        for (int r = 0; r < a.repeat; ++r) {
            out = gen.generate(a.tokens, r == 0 && a.first_max >= 0 ? a.first_max : max_new);
            runs.push_back(out);
            tables.push_back(gen.last_block_table(0));
            gen_ms.push_back(gen.last_generation_ms());
            replayed.push_back(gen.last_generation_replayed() ? 1 : 0);
            // FNV-1a over the bits of the last logits: equal hashes for equal bits.
            std::uint64_t hsh = 1469598103934665603ull;
            for (float v : gen.last_logits()) {
                std::uint32_t bits;
                std::memcpy(&bits, &v, 4);
                for (int b = 0; b < 4; ++b) hsh = (hsh ^ ((bits >> (8 * b)) & 0xFFu)) * 1099511628211ull;
            }
            logit_hashes.push_back(hsh);
            if (a.check_pools) pools_unchanged.push_back(pools_hash() == before ? 1 : 0);
            blocks_visited.push_back(gen.block(0).last_attention_blocks_visited());
        }
        std::printf("{\"ok\": true, \"runs\": [");
        for (std::size_t r = 0; r < runs.size(); ++r) {
            std::printf("%s[", r ? ", " : "");
            for (std::size_t i = 0; i < runs[r].size(); ++i) std::printf("%s%d", i ? ", " : "", runs[r][i]);
            std::printf("]");
        }
        std::printf("], \"tables\": [");
        for (std::size_t r = 0; r < tables.size(); ++r) {
            std::printf("%s[", r ? ", " : "");
            for (std::size_t i = 0; i < tables[r].size(); ++i) std::printf("%s%d", i ? ", " : "", tables[r][i]);
            std::printf("]");
        }
        std::printf("], \"replayed\": [");
        for (std::size_t r = 0; r < replayed.size(); ++r) std::printf("%s%d", r ? ", " : "", replayed[r]);
        std::printf("], \"logits_fnv\": [");
        for (std::size_t r = 0; r < logit_hashes.size(); ++r)
            std::printf("%s\"%016llx\"", r ? ", " : "", static_cast<unsigned long long>(logit_hashes[r]));
        std::printf("], \"pools_unchanged\": [");
        for (std::size_t r = 0; r < pools_unchanged.size(); ++r) std::printf("%s%d", r ? ", " : "", pools_unchanged[r]);
        std::printf("], \"blocks_visited\": [");
        for (std::size_t r = 0; r < blocks_visited.size(); ++r) std::printf("%s%zu", r ? ", " : "", blocks_visited[r]);
        std::printf("], \"tokens\": [");
        for (std::size_t i = 0; i < out.size(); ++i) std::printf("%s%d", i ? ", " : "", out[i]);
        std::printf("], \"load_ms\": %.3f, \"payload_bytes\": %zu, \"decode_ms\": %.3f, \"init_ms\": %.3f, "
                    "\"gen_ms\": [",
                    l.load_ms, l.breakdown.payload_bytes, l.breakdown.tensor_decode_ms, gen.initialization_ms());
        for (std::size_t i = 0; i < gen_ms.size(); ++i) std::printf("%s%.4f", i ? ", " : "", gen_ms[i]);
        std::printf("], \"free_blocks\": %zu}\n", gen.free_block_count());
    } catch (const std::exception& e) {
        std::printf("{\"ok\": false, \"error\": \"%s\"}\n", json_escape(e.what()).c_str());
    }
    return 0;
}

int cmd_forced(int argc, char** argv) {
    GenArgs a = parse_gen(5, argc, argv);
    a.path = argv[2];
    const std::size_t n_prompt = std::stoul(argv[3]);
    const std::string out = argv[4];
    try {
        Loaded l = load_model(a);
        generation::Generator gen(config_for(l.dims, -1), std::move(l.weights));
        const auto logits = gen.forced_logits(a.tokens, n_prompt);
        write_file(out, logits.data(), logits.size() * sizeof(float));
        std::printf("{\"ok\": true, \"rows\": %zu, \"vocab\": %zu}\n", a.tokens.size() - n_prompt + 1, l.dims.vocab);
    } catch (const std::exception& e) {
        std::printf("{\"ok\": false, \"error\": \"%s\"}\n", json_escape(e.what()).c_str());
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) {
        std::fprintf(stderr, "usage: tool_model {load-host|load-device|transpose|generate|forced} ...\n");
        return 2;
    }
    const std::string cmd = argv[1];
    try {
        if (cmd == "load-host") return cmd_load(false, argc, argv);
        if (cmd == "load-device") return cmd_load(true, argc, argv);
        if (cmd == "transpose" && argc == 6) return cmd_transpose(argv);
        if (cmd == "generate" && argc >= 5) return cmd_generate(argc, argv);
        if (cmd == "forced" && argc >= 5) return cmd_forced(argc, argv);
    } catch (const std::exception& e) {
        std::fprintf(stderr, "tool_model: %s\n", e.what());
        return 1;
    }
    std::fprintf(stderr, "tool_model: bad arguments\n");
    return 2;
}

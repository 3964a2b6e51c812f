// layer_stack.cpp -- end-to-end decode of a TinyLlama-shaped layer stack on the
// GPU through the C++ API: per token, TransformerBlock::forward_into of every
// layer (rmsnorm, q/k/v GEMVs, RoPE, the fused KV append + paged decode, o_proj,
// residual, rmsnorm, gate/up GEMVs, SwiGLU, down GEMV, residual), each layer
// with its own BlockPool and PageTable, as Generator::forward_into drives them
// (src/models/generator.cpp:571-614).  Embedding, final norm, lm_head and
// sampling are not part of this build; the hidden state is fed back from layer
// to layer and from token to token.
//
// Weights are random bf16 N(0, 0.02) rows [out][in] behind a transpose view
// (the checkpoint layout of the reference's safetensors loader), norm gammas 1.
// Prints one JSON line.  Usage: bench_layer_stack [layers] [positions] [warmup]
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "stratakv/memory/block_pool.h"
#include "stratakv/memory/page_table.h"
#include "stratakv/models/transformer_block.h"
#include "stratakv/tensor.h"
#include "stratakv_amd.h"

using stratakv::DataType;
using stratakv::Device;
using stratakv::Tensor;
using stratakv::memory::BlockPool;
using stratakv::memory::PageTable;
using stratakv::models::TransformerBlock;

namespace {

void ok_or_die(int rc, const char* what) {
    if (rc != SKV_OK) throw std::runtime_error(std::string(what) + ": " + skv_last_error());
}

constexpr std::size_t kHidden = 2048, kInter = 5632, kHeads = 32, kKvHeads = 4;
constexpr int kBlockSize = 16, kPoolBlocks = 1024;  // per layer, as the reference CLI sizes it

void random_rows(stratakv::layers::Linear& layer, uint64_t seed) {
    const std::size_t in = layer.input_dim(), out = layer.output_dim();
    Tensor rows({out, in}, DataType::BF16, Device::GPU);
    ok_or_die(skv_fill_normal_scaled_bf16(static_cast<uint16_t*>(rows.raw_data()), in * out, seed, 0,
                                          0.02f, nullptr),
              "weight fill");
    layer.set_weight(rows.transpose_2d());
}

}  // namespace

int main(int argc, char** argv) {
    try {
        const int layers = argc > 1 ? std::atoi(argv[1]) : 22;
        const int positions = argc > 2 ? std::atoi(argv[2]) : 144;
        const int warmup = argc > 3 ? std::atoi(argv[3]) : 1;
        int devices = 0;
        if (skv_device_count(&devices) != SKV_OK || devices == 0) {
            std::fprintf(stderr, "bench_layer_stack: no GPU\n");
            return 77;
        }
        std::vector<std::unique_ptr<TransformerBlock>> blocks;
        for (int l = 0; l < layers; ++l) {
            auto b = std::make_unique<TransformerBlock>(kHidden, kInter, kHeads, kKvHeads, kPoolBlocks,
                                                        kBlockSize);
            const uint64_t s = 0x5EED1000u + 16u * static_cast<uint64_t>(l);
            random_rows(b->attention().query_projection(), s + 0);
            random_rows(b->attention().key_projection(), s + 1);
            random_rows(b->attention().value_projection(), s + 2);
            random_rows(b->attention().output_projection(), s + 3);
            random_rows(b->gate_proj(), s + 4);
            random_rows(b->up_proj(), s + 5);
            random_rows(b->down_proj(), s + 6);
            b->to(Device::GPU);
            blocks.push_back(std::move(b));
        }
        const std::size_t hd = kHidden / kHeads;
        Tensor x({1, kHidden}, DataType::FP32, Device::GPU);
        std::vector<float> x0(kHidden);
        for (std::size_t i = 0; i < kHidden; ++i) x0[i] = static_cast<float>((i * 7919) % 1000) / 1000.0f - 0.5f;

        void* e0 = nullptr;
        void* e1 = nullptr;
        ok_or_die(skv_event_create(&e0), "event");
        ok_or_die(skv_event_create(&e1), "event");
        double ms = 0.0, wall_ms = 0.0;
        for (int run = 0; run <= warmup; ++run) {  // warmup generations, then the timed one
            std::vector<std::unique_ptr<BlockPool>> pools;
            std::vector<PageTable> tables(layers);
            for (int l = 0; l < layers; ++l) {
                pools.push_back(std::make_unique<BlockPool>(kPoolBlocks, kBlockSize,
                                                            static_cast<int>(kKvHeads),
                                                            static_cast<int>(hd), Device::GPU));
                tables[l].allocate_sequence(0, *pools[l]);
            }
            ok_or_die(skv_memcpy_h2d(x.raw_data(), x0.data(), kHidden * sizeof(float), nullptr), "x");
            ok_or_die(skv_device_synchronize(), "sync");
            const auto t0 = std::chrono::steady_clock::now();
            ok_or_die(skv_event_record(e0, nullptr), "record");
            for (int p = 0; p < positions; ++p)
                for (int l = 0; l < layers; ++l)
                    blocks[l]->forward_into(x, x, 0, tables[l], *pools[l], true);
            ok_or_die(skv_event_record(e1, nullptr), "record");
            ok_or_die(skv_event_synchronize(e1), "sync");
            const auto t1 = std::chrono::steady_clock::now();
            float m = 0.0f;
            ok_or_die(skv_event_elapsed_ms(&m, e0, e1), "elapsed");
            ms = m;
            wall_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
        }
        std::vector<float> y(kHidden);
        ok_or_die(skv_memcpy_d2h(y.data(), x.raw_data(), kHidden * sizeof(float), nullptr), "y");
        bool finite = true;
        for (float v : y) finite = finite && std::isfinite(v);
        std::printf("{\"layers\": %d, \"positions\": %d, \"ms_per_generation\": %.4f, "
                    "\"host_wall_ms\": %.4f, \"tokens_per_s\": %.2f, \"us_per_layer_token\": %.3f, "
                    "\"finite\": %s}\n",
                    layers, positions, ms, wall_ms, positions / (ms / 1e3),
                    ms * 1e3 / (static_cast<double>(positions) * layers), finite ? "true" : "false");
        skv_event_destroy(e0);
        skv_event_destroy(e1);
        return finite ? 0 : 1;
    } catch (const std::exception& e) {
        std::fprintf(stderr, "bench_layer_stack: %s\n", e.what());
        return 1;
    }
}

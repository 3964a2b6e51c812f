// sampler.h -- the next-token choice, on the device.
//
// Interface of the reference's stratakv::generation::Sampler
// (include/stratakv/generation/sampler.h:9-34, src/generation/sampler.cpp):
// temperature 0 is greedy (first index of the maximum); otherwise the logits
// are divided by the temperature, filtered by top-k (0 = off) and top-p
// (1 = off), and one token is drawn from the softmax of what is kept, with the
// std::mt19937 stream seeded like the reference's (one generate_canonical
// draw per call, as std::discrete_distribution makes).  The choice itself
// runs on the GPU (skv_sample_f32); only the uniform draw is made on the host.
#pragma once

#include <cstdint>
#include <random>

#include "stratakv/tensor.h"

namespace stratakv {
namespace generation {

struct SamplerConfig {
    float temperature = 1.0f;
    int top_k = 0;
    float top_p = 1.0f;
};

class Sampler {
public:
    Sampler();
    explicit Sampler(SamplerConfig config);
    Sampler(SamplerConfig config, std::uint32_t seed);
    ~Sampler();
    Sampler(const Sampler&) = delete;
    Sampler& operator=(const Sampler&) = delete;
    Sampler(Sampler&& other) noexcept;
    Sampler& operator=(Sampler&& other) noexcept;

    // logits: [vocab] or [1, vocab] FP32 on the GPU (a CPU tensor is copied
    // to the GPU first).  Waits for the result.  Errors as the reference:
    // std::invalid_argument for bad shapes and non-finite (scaled) logits,
    // std::runtime_error for an empty filtered distribution.
    int sample(const Tensor& logits) const;

    // Queues the choice on `stream` without waiting: token_ids[index] (device)
    // receives the token; data errors set SKV_FLAG_* bits in *flags (device).
    void sample_into(const float* logits, int vocab, std::int32_t* token_ids, int index,
                     std::int32_t* flags, void* stream) const;

    const SamplerConfig& config() const noexcept { return config_; }

    // Extension: the host uniform stream (one draw per sampled step).  The
    // Generator saves it before each queued draw and puts it back to the state
    // after the EOS step's draw, so the stream advances exactly as the
    // reference's one-draw-per-step loop.
    std::mt19937 rng_state() const { return rng_; }
    void set_rng_state(const std::mt19937& state) const { rng_ = state; }

private:
    SamplerConfig config_;
    mutable std::mt19937 rng_;
    mutable std::int32_t* scratch_ = nullptr;  // device: [0] token, [1] flags
};

}  // namespace generation
}  // namespace stratakv

// sampler.cpp -- Sampler over the device token-choice kernels.
// Configuration rules and error messages: src/generation/sampler.cpp:12-56.
#include "stratakv/generation/sampler.h"

#include <climits>
#include <cmath>
#include <limits>
#include <optional>
#include <stdexcept>
#include <utility>
#include <vector>

#include "abi_check.h"

namespace stratakv {
namespace generation {
namespace {

void validate_config(const SamplerConfig& c) {
    if (!std::isfinite(c.temperature) || c.temperature < 0.0f)
        throw std::invalid_argument("Sampler: temperature must be finite and nonnegative");
    if (c.top_k < 0) throw std::invalid_argument("Sampler: top_k must be nonnegative");
    if (!std::isfinite(c.top_p) || c.top_p <= 0.0f || c.top_p > 1.0f)
        throw std::invalid_argument("Sampler: top_p must be in (0, 1]");
}

std::uint32_t fresh_seed() {
    std::random_device device;
    return device();
}

}  // namespace

Sampler::Sampler() : config_{0.0f, 0, 1.0f}, rng_(fresh_seed()) {}

Sampler::Sampler(SamplerConfig config) : config_(config), rng_(fresh_seed()) { validate_config(config_); }

Sampler::Sampler(SamplerConfig config, std::uint32_t seed) : config_(config), rng_(seed) {
    validate_config(config_);
}

Sampler::~Sampler() {
    if (scratch_ != nullptr) (void)skv_free(scratch_);
}

Sampler::Sampler(Sampler&& other) noexcept
    : config_(other.config_), rng_(other.rng_), scratch_(std::exchange(other.scratch_, nullptr)) {}

Sampler& Sampler::operator=(Sampler&& other) noexcept {
    if (this != &other) {
        if (scratch_ != nullptr) (void)skv_free(scratch_);
        config_ = other.config_;
        rng_ = other.rng_;
        scratch_ = std::exchange(other.scratch_, nullptr);
    }
    return *this;
}

void Sampler::sample_into(const float* logits, int vocab, std::int32_t* token_ids, int index,
                          std::int32_t* flags, void* stream) const {
    // std::discrete_distribution draws once per call, and not at all for a
    // single-entry distribution; greedy mode never draws.
    double u = 0.0;
    if (config_.temperature != 0.0f && vocab >= 2)
        u = std::generate_canonical<double, std::numeric_limits<double>::digits>(rng_);
    detail::check(skv_sample_f32(logits, vocab, config_.temperature, config_.top_k, config_.top_p, u,
                                 token_ids, index, flags, stream),
                  "Sampler::sample");
}

int Sampler::sample(const Tensor& logits) const {
    const auto& shape = logits.shape();
    if (!(shape.size() == 1 || (shape.size() == 2 && shape[0] == 1)))
        throw std::invalid_argument("Sampler: expected [vocab] or [1,vocab]");
    const std::size_t vocab = shape.back();
    if (vocab == 0 || vocab > static_cast<std::size_t>(INT_MAX) || logits.num_elements() != vocab ||
        !logits.raw_data())
        throw std::invalid_argument("Sampler: empty or invalid vocabulary/storage");
    // FP32 values on the device (BF16 logits widen exactly).
    std::optional<Tensor> staged;
    const Tensor* src = &logits;
    if (src->device() != Device::GPU) {
        staged.emplace(src->to(Device::GPU));
        src = &*staged;
    }
    std::optional<Tensor> widened;
    if (src->dtype() != DataType::FP32) {
        widened.emplace(std::vector<std::size_t>{vocab}, DataType::FP32, Device::GPU);
        detail::check(skv_convert_to_f32(src->raw_data(), SKV_DTYPE_BF16, vocab, static_cast<float*>(widened->raw_data()),
                                         nullptr, nullptr),
                      "Sampler::sample");
        src = &*widened;
    }
    if (scratch_ == nullptr) {
        void* p = nullptr;
        detail::check(skv_malloc(&p, 2 * sizeof(std::int32_t)), "Sampler::sample");
        scratch_ = static_cast<std::int32_t*>(p);
    }
    detail::check(skv_memset_d8(scratch_, 0, 2 * sizeof(std::int32_t), nullptr), "Sampler::sample");
    sample_into(static_cast<const float*>(src->raw_data()), static_cast<int>(vocab), scratch_, 0, scratch_ + 1,
                nullptr);
    std::int32_t result[2] = {0, 0};
    detail::check(skv_memcpy_d2h(result, scratch_, sizeof(result), nullptr), "Sampler::sample");
    if (result[1] & SKV_FLAG_NONFINITE_LOGITS) throw std::invalid_argument("Sampler: logits must all be finite");
    if (result[1] & SKV_FLAG_NONFINITE_SCALED) throw std::invalid_argument("Sampler: scaled logits are not finite");
    if (result[1] & SKV_FLAG_BAD_DISTRIBUTION) throw std::runtime_error("Sampler: invalid softmax distribution");
    return result[0];
}

}  // namespace generation
}  // namespace stratakv

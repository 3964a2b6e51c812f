// rmsnorm.h -- RMSNorm over the last dimension, fp32 gamma.
// Interface of the reference's stratakv::layers::RMSNorm
// (include/stratakv/layers/rmsnorm.h:10-39), epsilon 1e-5 by default.
#pragma once

#include <cstddef>

#include "stratakv/tensor.h"

namespace stratakv {
namespace layers {

class RMSNorm {
public:
    explicit RMSNorm(std::size_t hidden_dim, float epsilon = 1.0e-5f);
    RMSNorm(Tensor&& gamma, float epsilon = 1.0e-5f);

    RMSNorm(const RMSNorm&) = delete;
    RMSNorm& operator=(const RMSNorm&) = delete;
    RMSNorm(RMSNorm&&) noexcept = default;
    RMSNorm& operator=(RMSNorm&&) noexcept = default;
    ~RMSNorm() = default;

    // CPU: sum of squares accumulated in double (src/layers/rmsnorm.cpp:63-97).
    // GPU: skv_rmsnorm_f32.
    Tensor forward(const Tensor& input) const;
    void to(Device device);

    Tensor& gamma() noexcept { return gamma_; }
    const Tensor& gamma() const noexcept { return gamma_; }
    std::size_t hidden_dim() const noexcept { return hidden_dim_; }
    float epsilon() const noexcept { return epsilon_; }

private:
    std::size_t hidden_dim_;
    float epsilon_;
    Tensor gamma_;
};

}  // namespace layers
}  // namespace stratakv

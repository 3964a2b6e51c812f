// linear.h -- Y = X * W (+ bias), W logical [input_dim, output_dim].
//
// Interface of the reference's stratakv::layers::Linear
// (include/stratakv/layers/linear.h:16-57).  On the GPU, forward_into runs
// skv_linear_f32 (a GEMV for decode) over fp32 or bf16 weights stored either
// GEMM-ready [input_dim, output_dim] or as a transpose_2d() view over
// output-major [output_dim, input_dim] rows; on the CPU it is a plain loop.
#pragma once

#include <cstddef>
#include <optional>

#include "stratakv/tensor.h"

namespace stratakv {
namespace layers {

class Linear {
public:
    Linear(std::size_t input_dim, std::size_t output_dim, bool use_bias = false);
    Linear(Tensor&& weight_transposed, std::optional<Tensor> bias = std::nullopt);

    Linear(const Linear&) = delete;
    Linear& operator=(const Linear&) = delete;
    Linear(Linear&&) noexcept = default;
    Linear& operator=(Linear&&) noexcept = default;
    ~Linear() = default;

    Tensor forward(const Tensor& input) const;
    void forward_into(const Tensor& input, Tensor& output) const;
    void to(Device device);

    Tensor& weight() noexcept { return weight_; }
    const Tensor& weight() const noexcept { return weight_; }
    void set_weight(Tensor&& weight_transposed);
    Tensor* bias() noexcept { return bias_ ? &*bias_ : nullptr; }
    const Tensor* bias() const noexcept { return bias_ ? &*bias_ : nullptr; }
    std::size_t input_dim() const noexcept { return input_dim_; }
    std::size_t output_dim() const noexcept { return output_dim_; }

private:
    std::size_t input_dim_;
    std::size_t output_dim_;
    Tensor weight_;
    std::optional<Tensor> bias_;
};

}  // namespace layers
}  // namespace stratakv

// layers.cpp -- Linear, RMSNorm and the PagedAttention parameter holder.
// Linear follows src/layers/linear.cpp:30-163 (Y = X * W, W logical
// [input_dim, output_dim]); RMSNorm follows src/layers/rmsnorm.cpp:63-97
// (double-accumulated sum of squares on the CPU).
#include <cmath>
#include <stdexcept>
#include <string>
#include <utility>

#include "abi_check.h"
#include "stratakv/layers/attention.h"
#include "stratakv/layers/linear.h"
#include "stratakv/layers/rmsnorm.h"

namespace stratakv {
namespace layers {

Linear::Linear(std::size_t input_dim, std::size_t output_dim, bool use_bias)
    : input_dim_(input_dim), output_dim_(output_dim), weight_({input_dim, output_dim}) {
    if (input_dim == 0 || output_dim == 0)
        throw std::invalid_argument("Linear: input_dim and output_dim must be non-zero");
    if (use_bias) bias_.emplace(std::vector<std::size_t>{output_dim});
}

Linear::Linear(Tensor&& weight_transposed, std::optional<Tensor> bias)
    : input_dim_(weight_transposed.ndim() == 2 ? weight_transposed.shape()[0] : 0),
      output_dim_(weight_transposed.ndim() == 2 ? weight_transposed.shape()[1] : 0),
      weight_(std::move(weight_transposed)),
      bias_(std::move(bias)) {
    if (weight_.ndim() != 2) throw std::invalid_argument("Linear: weight must be rank-2");
    if (input_dim_ == 0 || output_dim_ == 0)
        throw std::invalid_argument("Linear: weight dimensions must be non-zero");
    if (bias_ && (bias_->ndim() != 1 || bias_->shape()[0] != output_dim_))
        throw std::invalid_argument("Linear: bias must have shape [output_dim]");
}

void Linear::set_weight(Tensor&& weight_transposed) {
    if (weight_transposed.ndim() != 2 || weight_transposed.shape()[0] != input_dim_ ||
        weight_transposed.shape()[1] != output_dim_)
        throw std::invalid_argument("Linear::set_weight: weight shape does not match layer");
    weight_ = std::move(weight_transposed);
}

void Linear::to(Device device) {
    if (weight_.device() == device && (!bias_ || bias_->device() == device)) return;
    weight_ = weight_.to(device);
    if (bias_) *bias_ = bias_->to(device);
}

Tensor Linear::forward(const Tensor& input) const {
    if (input.ndim() != 2)
        throw std::invalid_argument("Linear::forward: input must have shape [tokens, input_dim]");
    if (input.shape()[1] != input_dim_)
        throw std::invalid_argument("Linear::forward: input feature dimension is " +
                                    std::to_string(input.shape()[1]) + ", expected " +
                                    std::to_string(input_dim_));
    if (input.device() != weight_.device())
        throw std::invalid_argument("Linear::forward: input and weight must share a device");
    Tensor output({input.shape()[0], output_dim_}, DataType::FP32, input.device());
    forward_into(input, output);
    return output;
}

void Linear::forward_into(const Tensor& input, Tensor& output) const {
    if (input.ndim() != 2 || input.shape()[1] != input_dim_ || output.ndim() != 2 ||
        output.shape() != std::vector<std::size_t>{input.shape()[0], output_dim_} ||
        output.dtype() != DataType::FP32 || output.device() != input.device())
        throw std::invalid_argument("Linear::forward_into: input/output shape or device mismatch");
    if (input.dtype() != DataType::FP32)
        throw std::invalid_argument("Linear::forward_into: activations must be FP32");
    const std::size_t rows = input.shape()[0];
    if (input.device() == Device::GPU) {
        if (weight_.device() != Device::GPU || (bias_ && bias_->device() != Device::GPU))
            throw std::invalid_argument("Linear::forward_into: GPU input needs GPU-resident parameters");
        const int wdt = weight_.dtype() == DataType::BF16 ? SKV_DTYPE_BF16 : SKV_DTYPE_FP32;
        detail::check(skv_linear_f32(static_cast<const float*>(input.raw_data()), static_cast<int>(rows),
                                     weight_.raw_data(), wdt, static_cast<int64_t>(weight_.strides()[0]),
                                     static_cast<int64_t>(weight_.strides()[1]),
                                     static_cast<int>(input_dim_), static_cast<int>(output_dim_),
                                     bias_ ? static_cast<const float*>(bias_->raw_data()) : nullptr,
                                     static_cast<float*>(output.raw_data()), nullptr),
                      "Linear::forward_into");
        return;
    }
    if (weight_.device() != Device::CPU)
        throw std::invalid_argument("Linear::forward_into: input and weight must share a device");
    for (std::size_t r = 0; r < rows; ++r) {
        for (std::size_t n = 0; n < output_dim_; ++n) {
            float s = bias_ ? (*bias_)[n] : 0.0f;
            for (std::size_t k = 0; k < input_dim_; ++k)
                s += input[r * input_dim_ + k] * weight_[k * output_dim_ + n];
            output[r * output_dim_ + n] = s;
        }
    }
}

RMSNorm::RMSNorm(std::size_t hidden_dim, float epsilon)
    : hidden_dim_(hidden_dim), epsilon_(epsilon), gamma_({hidden_dim}) {
    if (hidden_dim == 0) throw std::invalid_argument("RMSNorm: hidden_dim must be non-zero");
    for (std::size_t i = 0; i < hidden_dim; ++i) gamma_[i] = 1.0f;
}

RMSNorm::RMSNorm(Tensor&& gamma, float epsilon)
    : hidden_dim_(gamma.ndim() == 1 ? gamma.shape()[0] : 0), epsilon_(epsilon), gamma_(std::move(gamma)) {
    if (hidden_dim_ == 0) throw std::invalid_argument("RMSNorm: gamma must be a non-empty vector");
}

void RMSNorm::to(Device device) {
    if (gamma_.device() != device) gamma_ = gamma_.to(device);
}

Tensor RMSNorm::forward(const Tensor& input) const {
    if (input.ndim() < 1 || input.shape().back() != hidden_dim_)
        throw std::invalid_argument("RMSNorm::forward: last dimension must equal hidden_dim");
    const std::size_t rows = input.num_elements() / hidden_dim_;
    Tensor output(input.shape(), DataType::FP32, input.device());
    if (input.device() == Device::GPU) {
        if (gamma_.device() != Device::GPU || input.dtype() != DataType::FP32)
            throw std::invalid_argument("RMSNorm::forward: GPU input needs FP32 data and GPU gamma");
        detail::check(skv_rmsnorm_f32(static_cast<const float*>(input.raw_data()),
                                      static_cast<float*>(output.raw_data()),
                                      static_cast<const float*>(gamma_.raw_data()), static_cast<int>(rows),
                                      static_cast<int>(hidden_dim_), epsilon_, nullptr),
                      "RMSNorm::forward");
        return output;
    }
    for (std::size_t r = 0; r < rows; ++r) {
        double sum = 0.0;
        for (std::size_t i = 0; i < hidden_dim_; ++i) {
            const double x = input[r * hidden_dim_ + i];
            sum += x * x;
        }
        const float inv = static_cast<float>(1.0 / std::sqrt(sum / static_cast<double>(hidden_dim_) +
                                                             static_cast<double>(epsilon_)));
        for (std::size_t i = 0; i < hidden_dim_; ++i)
            output[r * hidden_dim_ + i] = input[r * hidden_dim_ + i] * inv * gamma_[i];
    }
    return output;
}

PagedAttention::PagedAttention(std::size_t hidden_dim, std::size_t num_heads, int total_blocks,
                               int block_size, Device device)
    : PagedAttention(hidden_dim, num_heads, 0, total_blocks, block_size, device) {}

PagedAttention::PagedAttention(std::size_t hidden_dim, std::size_t num_heads, std::size_t num_kv_heads,
                               int total_blocks, int block_size, Device device)
    : hidden_dim_(hidden_dim),
      num_heads_(num_heads),
      num_kv_heads_(num_kv_heads == 0 ? num_heads : num_kv_heads),
      head_dim_(num_heads == 0 ? 0 : hidden_dim / num_heads),
      total_blocks_(total_blocks),
      block_size_(block_size),
      device_(device),
      q_proj_(hidden_dim == 0 ? 1 : hidden_dim, hidden_dim == 0 ? 1 : hidden_dim),
      k_proj_(hidden_dim == 0 ? 1 : hidden_dim, num_kv_heads_ * head_dim_ == 0 ? 1 : num_kv_heads_ * head_dim_),
      v_proj_(hidden_dim == 0 ? 1 : hidden_dim, num_kv_heads_ * head_dim_ == 0 ? 1 : num_kv_heads_ * head_dim_),
      out_proj_(hidden_dim == 0 ? 1 : hidden_dim, hidden_dim == 0 ? 1 : hidden_dim) {
    // Same preconditions as src/layers/attention.cpp:138-157.
    if (hidden_dim == 0 || num_heads == 0)
        throw std::invalid_argument("PagedAttention: hidden_dim and num_heads must be non-zero");
    if (hidden_dim % num_heads != 0)
        throw std::invalid_argument("PagedAttention: hidden_dim must be divisible by num_heads");
    if (num_kv_heads_ == 0 || num_heads_ % num_kv_heads_ != 0)
        throw std::invalid_argument("PagedAttention: num_kv_heads must divide num_heads");
    if (head_dim_ % 2 != 0)
        throw std::invalid_argument("PagedAttention: head dimension must be even for RoPE");
    if (total_blocks <= 0 || block_size <= 0)
        throw std::invalid_argument("PagedAttention: total_blocks and block_size must be positive");
}

Tensor PagedAttention::forward(const Tensor&, int, memory::PageTable&, memory::BlockPool&, bool) {
    throw std::runtime_error(
        "PagedAttention::forward: the CPU multi-token path is not part of this build; use "
        "TransformerBlock::forward_into on GPU tensors");
}

}  // namespace layers
}  // namespace stratakv

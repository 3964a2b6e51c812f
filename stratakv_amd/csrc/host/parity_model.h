// parity_model.h -- the host model behind STRATAKV_PARITY=1: every decoder
// layer, the final norm and the LM head restated on the CPU in double
// precision from host copies of the device weights, so the Generator can
// report how far each GPU layer is from it at every position.  The
// reference compares its GPU layers with its CPU layers the same way
// (src/generation/generator.cpp:33-36, 485-490, 581-613) and the ops of
// layer 0 on the first token (src/models/transformer_block.cpp:405-595).
//
// A diagnostic only: it never supplies a value to the GPU path.  Its K/V
// cache holds the rotated keys and the values rounded to bf16 (nearest-even),
// as this build's pools hold them, so its attention reads what the GPU's
// reads and the reported differences are the arithmetic's alone.
#pragma once

#include <cstddef>
#include <cstdint>
#include <vector>

#include "stratakv/layers/linear.h"
#include "stratakv/layers/rmsnorm.h"
#include "stratakv/models/transformer_block.h"
#include "stratakv/tensor.h"

namespace stratakv {
namespace detail {

// A projection's weights (and bias) copied to the host in their storage
// dtype; y = W x + b with element (o, i) widened exactly when read and the
// sums in double.
class HostLinear {
public:
    HostLinear() = default;
    explicit HostLinear(const layers::Linear& linear);
    std::vector<double> apply(const std::vector<double>& x) const;
    std::size_t input_dim() const noexcept { return in_; }
    std::size_t output_dim() const noexcept { return out_; }

private:
    double weight(std::size_t o, std::size_t i) const noexcept;
    std::size_t in_ = 0, out_ = 0;
    std::size_t stride_in_ = 0, stride_out_ = 0;   // element strides of input index i and output index o
    bool bf16_ = true;
    std::vector<std::uint16_t> w16_;
    std::vector<float> w32_;
    std::vector<double> bias_;
};

// One token's intermediate values in one layer.
struct HostLayerOps {
    std::vector<double> norm1, q, k, v, q_rot, k_rot, context, out_proj, residual, norm2, gate, up, act, down, output;
};

class ParityModel {
public:
    ParityModel(const std::vector<models::TransformerBlock>& blocks, const layers::RMSNorm& final_norm,
                const layers::Linear& lm_head, const Tensor& embeddings);
    // Empties every layer's cache (a new sequence at position 0).
    void reset();
    // The embedding row of `token`, widened exactly.
    std::vector<double> embedding(int token) const;
    // One token through layer `l` at that layer's next position; fills `ops`
    // when given.
    std::vector<double> layer(std::size_t l, const std::vector<double>& x, HostLayerOps* ops = nullptr);
    std::vector<double> final_norm(const std::vector<double>& x) const;
    std::vector<double> logits(const std::vector<double>& normed) const { return lm_head_.apply(normed); }
    std::size_t num_layers() const noexcept { return layers_.size(); }

private:
    struct Layer {
        std::vector<double> gamma1, gamma2;
        double eps1 = 0.0, eps2 = 0.0;
        HostLinear q, k, v, o, gate, up, down;
        std::vector<double> k_cache, v_cache;   // [position][num_kv_heads * head_dim], bf16-rounded
        int positions = 0;
    };
    std::vector<Layer> layers_;
    std::size_t hidden_ = 0, heads_ = 0, kv_heads_ = 0, head_dim_ = 0;
    std::vector<double> final_gamma_;
    double final_eps_ = 0.0;
    HostLinear lm_head_;
    const Tensor* embeddings_ = nullptr;
};

// Max |a - b| over the common length.
double max_abs_diff(const std::vector<float>& gpu, const std::vector<double>& cpu);

}  // namespace detail
}  // namespace stratakv

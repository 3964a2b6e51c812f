// transformer_block.cpp -- TransformerBlock::to / forward / forward_into.
// The GPU decode step follows src/models/transformer_block.cpp:334-613 of the
// reference sub-step for sub-step; the KV append and the paged decode are the
// hot path (skv_paged_attention_decode_append: append + decode in one launch); the other
// sub-steps run as fused projections (norm + q/k/v + RoPE, o_proj + residual,
// norm + gate/up + SwiGLU, down_proj + residual) when the weights are aligned
// output-major rows, else as the separate kernels of skv_layer_ops.hip.
#include "stratakv/models/transformer_block.h"

#include <cstring>

#include <cstdio>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "abi_check.h"
#include "prompt_gemm_api.h"

namespace stratakv {
namespace models {

TransformerBlock::TransformerBlock(std::size_t hidden_dim, std::size_t intermediate_dim,
                                   std::size_t num_heads, int total_blocks, int block_size,
                                   Device device)
    : TransformerBlock(hidden_dim, intermediate_dim, num_heads, 0, total_blocks, block_size, device) {}

TransformerBlock::TransformerBlock(std::size_t hidden_dim, std::size_t intermediate_dim,
                                   std::size_t num_heads, std::size_t num_kv_heads, int total_blocks,
                                   int block_size, Device device)
    : hidden_dim_(hidden_dim),
      norm1_(hidden_dim == 0 ? 1 : hidden_dim),
      attention_(hidden_dim, num_heads, num_kv_heads, total_blocks, block_size, device),
      norm2_(hidden_dim == 0 ? 1 : hidden_dim),
      gate_proj_(hidden_dim, intermediate_dim == 0 ? 1 : intermediate_dim),
      up_proj_(hidden_dim, intermediate_dim == 0 ? 1 : intermediate_dim),
      down_proj_(intermediate_dim == 0 ? 1 : intermediate_dim, hidden_dim) {
    if (hidden_dim == 0 || intermediate_dim == 0)
        throw std::invalid_argument("TransformerBlock: feature dimensions must be non-zero");
}

void TransformerBlock::to(Device device) {
    norm1_.to(device);
    attention_.query_projection().to(device);
    attention_.key_projection().to(device);
    attention_.value_projection().to(device);
    attention_.output_projection().to(device);
    norm2_.to(device);
    gate_proj_.to(device);
    up_proj_.to(device);
    down_proj_.to(device);
    if (device == Device::GPU) {
        const std::size_t kv_dim = attention_.num_kv_heads() * attention_.head_dim();
        const std::size_t inter = gate_proj_.output_dim();
        normalized_input_workspace_.emplace(std::vector<std::size_t>{1, hidden_dim_}, DataType::FP32, device);
        query_workspace_.emplace(std::vector<std::size_t>{1, hidden_dim_}, DataType::FP32, device);
        key_workspace_.emplace(std::vector<std::size_t>{1, kv_dim}, DataType::FP32, device);
        value_workspace_.emplace(std::vector<std::size_t>{1, kv_dim}, DataType::FP32, device);
        context_workspace_.emplace(std::vector<std::size_t>{1, hidden_dim_}, DataType::FP32, device);
        normalized_residual_workspace_.emplace(std::vector<std::size_t>{1, hidden_dim_}, DataType::FP32, device);
        gate_workspace_.emplace(std::vector<std::size_t>{1, inter}, DataType::FP32, device);
        up_workspace_.emplace(std::vector<std::size_t>{1, inter}, DataType::FP32, device);
        down_workspace_.emplace(std::vector<std::size_t>{1, hidden_dim_}, DataType::FP32, device);
        const std::size_t ws = skv_paged_attention_decode_workspace_bytes(
            static_cast<int>(attention_.num_heads()), static_cast<int>(attention_.num_kv_heads()),
            static_cast<int>(attention_.head_dim()));
        decode_workspace_.emplace(std::vector<std::size_t>{(ws + 3) / 4}, DataType::FP32, device);
    } else {
        normalized_input_workspace_.reset();
        query_workspace_.reset();
        key_workspace_.reset();
        value_workspace_.reset();
        context_workspace_.reset();
        normalized_residual_workspace_.reset();
        gate_workspace_.reset();
        up_workspace_.reset();
        down_workspace_.reset();
        decode_workspace_.reset();
    }
}

Tensor TransformerBlock::forward(const Tensor& hidden_states, int seq_id, memory::PageTable& page_table,
                                 memory::BlockPool& block_pool, bool append_tokens) {
    if (hidden_states.ndim() != 2 || hidden_states.shape()[1] != hidden_dim_)
        throw std::invalid_argument("TransformerBlock::forward: hidden_states must be [tokens, hidden_dim]");
    if (hidden_states.device() == Device::GPU) {
        Tensor result({1, hidden_dim_}, DataType::FP32, Device::GPU);
        forward_into(hidden_states, result, seq_id, page_table, block_pool, append_tokens);
        return result;
    }
    throw std::runtime_error(
        "TransformerBlock::forward: the CPU path is not part of this build; move the block and "
        "the hidden states to Device::GPU");
}

TransformerBlock::ParityRow TransformerBlock::parity_row(int row) const {
    detail::check(skv_stream_synchronize(stream_), "parity_row");
    const std::size_t q_dim = attention_.num_heads() * attention_.head_dim();
    const std::size_t kv_dim = attention_.num_kv_heads() * attention_.head_dim();
    const std::size_t inter = gate_proj_.output_dim();
    auto copy = [&](const std::optional<Tensor>& t, std::size_t dim) {
        std::vector<float> v;
        if (!t || row < 0 || static_cast<std::size_t>(row) * dim + dim > t->num_elements()) return v;
        v.resize(dim);
        detail::check(skv_memcpy_d2h(v.data(), static_cast<const float*>(t->raw_data()) + row * dim,
                                     dim * sizeof(float), nullptr),
                      "parity_row");
        return v;
    };
    ParityRow r;
    if (last_pass_prefill_ && pf_) {
        r.q = copy(pf_->queries, q_dim);
        r.k = copy(pf_->keys, kv_dim);
        r.v = copy(pf_->values, kv_dim);
        r.context = copy(pf_->context, q_dim);
        r.residual = copy(pf_->residual, hidden_dim_);
        r.act = copy(pf_->act, inter);
    } else if (row == 0) {
        r.q = copy(query_workspace_, q_dim);
        r.k = copy(key_workspace_, kv_dim);
        r.v = copy(value_workspace_, kv_dim);
        r.context = copy(context_workspace_, q_dim);
        r.residual = copy(down_workspace_, hidden_dim_);   // h = input + o_proj
        r.act = copy(gate_workspace_, inter);              // swiglu(gate, up)
    }
    return r;
}

// forward_into's device work with the position, context length and block
// table read on the device (see the header); no host bookkeeping, so the
// launches can be captured once and replayed per token.
bool TransformerBlock::forward_into_at(const Tensor& hidden_states, Tensor& output, const std::int32_t* step,
                                       const float* rope_cos_sin, int rope_positions, const int* device_table,
                                       int table_capacity, memory::BlockPool& block_pool) {
    last_pass_prefill_ = false;
    if (hidden_states.ndim() != 2 || hidden_states.shape()[0] != 1 || hidden_states.shape()[1] != hidden_dim_ ||
        output.shape() != hidden_states.shape() || output.device() != Device::GPU ||
        hidden_states.device() != Device::GPU || hidden_states.dtype() != DataType::FP32 ||
        output.dtype() != DataType::FP32)
        throw std::invalid_argument("TransformerBlock::forward_into_at: one FP32 GPU row in and out required");
    if (!step || !rope_cos_sin || rope_positions <= 0 || !device_table || table_capacity <= 0)
        throw std::invalid_argument("TransformerBlock::forward_into_at: invalid step state or block table");
    if (!query_workspace_ || !decode_workspace_ || block_pool.device() != Device::GPU ||
        block_pool.key_cache() == nullptr)
        throw std::runtime_error("TransformerBlock::forward_into_at: GPU workspace is not initialized");
    const layers::Linear& wq = attention_.query_projection();
    const layers::Linear& wk = attention_.key_projection();
    const layers::Linear& wv = attention_.value_projection();
    const layers::Linear& wo = attention_.output_projection();
    auto wdtype = [](const layers::Linear& l) {
        return l.weight().dtype() == DataType::BF16 ? SKV_DTYPE_BF16 : SKV_DTYPE_FP32;
    };
    auto stride_k = [](const layers::Linear& l) { return static_cast<int64_t>(l.weight().strides()[0]); };
    auto stride_n = [](const layers::Linear& l) { return static_cast<int64_t>(l.weight().strides()[1]); };
    auto cfp = [](const Tensor& t) { return static_cast<const float*>(t.raw_data()); };
    auto fp = [](Tensor& t) { return static_cast<float*>(t.raw_data()); };
    auto bias_of = [&](const layers::Linear& l) { return l.bias() ? cfp(*l.bias()) : nullptr; };
    // Every projection must take its fused kernel (checked before anything is
    // launched): the same-dtype and same-layout conditions forward_into tests,
    // and the fused kernels' layout rules (output-major 16-byte aligned rows,
    // at least one wave-wide load long, inputs staged whole in LDS).
    auto fusable = [&](const layers::Linear& l) {
        const int esz = wdtype(l) == SKV_DTYPE_BF16 ? 2 : 4;
        const std::size_t K = l.input_dim();
        return stride_k(l) == 1 && K >= static_cast<std::size_t>(esz == 2 ? 512 : 256) && K <= 8192 &&
               reinterpret_cast<std::uintptr_t>(l.weight().raw_data()) % 16 == 0 &&
               (stride_n(l) * esz) % 16 == 0 && static_cast<std::size_t>(stride_n(l)) >= K;
    };
    if (!(wdtype(wq) == wdtype(wk) && wdtype(wq) == wdtype(wv) && stride_k(wq) == stride_k(wk) &&
          stride_k(wq) == stride_k(wv) && wdtype(gate_proj_) == wdtype(up_proj_) &&
          stride_k(gate_proj_) == stride_k(up_proj_)))
        return false;
    const layers::Linear* const projections[] = {&wq, &wk, &wv, &wo, &gate_proj_, &up_proj_, &down_proj_};
    for (const layers::Linear* l : projections)
        if (!fusable(*l)) return false;

    const int head_dim = static_cast<int>(attention_.head_dim());
    const int num_heads = static_cast<int>(attention_.num_heads());
    const int num_kv_heads = static_cast<int>(attention_.num_kv_heads());
    const int hidden = static_cast<int>(hidden_dim_);
    const int inter = static_cast<int>(gate_proj_.output_dim());
    void* s = stream_;
    Tensor& queries = *query_workspace_;
    Tensor& keys = *key_workspace_;
    Tensor& values = *value_workspace_;
    Tensor& context = *context_workspace_;
    Tensor& gate = *gate_workspace_;
    Tensor& down = *down_workspace_;
    Tensor& ws = *decode_workspace_;
    const int64_t qkv_strides[3] = {stride_n(wq), stride_n(wk), stride_n(wv)};
    detail::check(skv_fused_qkv_at_f32(cfp(hidden_states), cfp(norm1_.gamma()), norm1_.epsilon(),
                                       wq.weight().raw_data(), wk.weight().raw_data(), wv.weight().raw_data(),
                                       wdtype(wq), stride_k(wq), qkv_strides, bias_of(wq), bias_of(wk),
                                       bias_of(wv), hidden, num_heads, num_kv_heads, head_dim, step,
                                       rope_cos_sin, rope_positions, fp(queries), fp(keys), fp(values), s),
                  "forward_into_at: fused rmsnorm + q/k/v + rope");
    detail::check(skv_paged_decode_append(cfp(queries), SKV_DTYPE_FP32, cfp(keys), cfp(values), SKV_DTYPE_FP32,
                                          block_pool.key_cache(), block_pool.value_cache(),
                                          block_pool.total_blocks(), device_table, table_capacity, step + 1, 1,
                                          num_heads, num_kv_heads, head_dim, block_pool.block_size(),
                                          1.0f / std::sqrt(static_cast<float>(head_dim)), fp(context),
                                          ws.raw_data(), ws.num_elements() * ws.element_size(), s),
                  "forward_into_at: KV append + paged attention");
    detail::check(skv_linear_residual_f32(cfp(context), wo.weight().raw_data(), wdtype(wo), stride_k(wo),
                                          stride_n(wo), static_cast<int>(wo.input_dim()),
                                          static_cast<int>(wo.output_dim()), bias_of(wo), cfp(hidden_states),
                                          fp(down), s),
                  "forward_into_at: fused o_proj + residual");
    detail::check(skv_fused_gate_up_swiglu_f32(cfp(down), cfp(norm2_.gamma()), norm2_.epsilon(),
                                               gate_proj_.weight().raw_data(), up_proj_.weight().raw_data(),
                                               wdtype(gate_proj_), stride_k(gate_proj_), stride_n(gate_proj_),
                                               stride_n(up_proj_), bias_of(gate_proj_), bias_of(up_proj_), hidden,
                                               inter, fp(gate), s),
                  "forward_into_at: fused rmsnorm + gate/up + swiglu");
    detail::check(skv_linear_residual_f32(cfp(gate), down_proj_.weight().raw_data(), wdtype(down_proj_),
                                          stride_k(down_proj_), stride_n(down_proj_), inter, hidden,
                                          bias_of(down_proj_), cfp(down), fp(output), s),
                  "forward_into_at: fused down_proj + residual");
    return true;
}

void TransformerBlock::forward_into(const Tensor& hidden_states, Tensor& output, int seq_id,
                                    memory::PageTable& page_table, memory::BlockPool& block_pool,
                                    bool append_tokens) {
    last_pass_prefill_ = false;
    // Validation in the order and with the messages of
    // src/models/transformer_block.cpp:338-394.
    if (hidden_states.ndim() != 2 || hidden_states.shape()[1] != hidden_dim_ ||
        output.device() != hidden_states.device() || output.shape() != hidden_states.shape() ||
        output.dtype() != DataType::FP32)
        throw std::invalid_argument("TransformerBlock::forward_into: output shape or device mismatch");
    if (output.device() != Device::GPU)
        throw std::runtime_error(
            "TransformerBlock::forward_into: the CPU path is not part of this build; use GPU tensors");
    if (hidden_states.shape()[0] != 1)
        throw std::invalid_argument("TransformerBlock::forward_into: GPU decode requires one token");
    if (hidden_states.dtype() != DataType::FP32)
        throw std::runtime_error("TransformerBlock::forward_into: hidden_states is not FP32");
    if (norm1_.gamma().dtype() != DataType::FP32 || norm2_.gamma().dtype() != DataType::FP32 ||
        norm1_.gamma().device() != Device::GPU || norm2_.gamma().device() != Device::GPU)
        throw std::runtime_error("TransformerBlock::forward_into: RMSNorm weights are not on GPU");
    if (attention_.query_projection().weight().device() != Device::GPU ||
        attention_.key_projection().weight().device() != Device::GPU ||
        attention_.value_projection().weight().device() != Device::GPU ||
        attention_.output_projection().weight().device() != Device::GPU ||
        gate_proj_.weight().device() != Device::GPU || up_proj_.weight().device() != Device::GPU ||
        down_proj_.weight().device() != Device::GPU)
        throw std::runtime_error("TransformerBlock::forward_into: projection weights are not on GPU");
    if (block_pool.device() != Device::GPU || block_pool.key_cache() == nullptr ||
        block_pool.value_cache() == nullptr ||
        block_pool.num_kv_heads() != static_cast<int>(attention_.num_kv_heads()) ||
        block_pool.head_dim() != static_cast<int>(attention_.head_dim()))
        throw std::invalid_argument(
            "TransformerBlock::forward_into: GPU BlockPool configuration does not match attention");
    if (!page_table.has_sequence(seq_id))
        throw std::runtime_error("TransformerBlock::forward_into: seq_id is not registered");
    if (!normalized_input_workspace_ || !query_workspace_ || !key_workspace_ || !value_workspace_ ||
        !context_workspace_ || !normalized_residual_workspace_ || !gate_workspace_ ||
        !up_workspace_ || !down_workspace_ || !decode_workspace_)
        throw std::runtime_error("TransformerBlock::forward_into: GPU workspace is not initialized");

    const memory::SequenceState& initial_state = page_table.get_state(seq_id);
    if (initial_state.sequence_length <= 0 && !append_tokens)
        throw std::invalid_argument("TransformerBlock::forward_into: cannot decode without context");
    const int logical_position = initial_state.sequence_length;
    if (append_tokens) page_table.append_token(seq_id, block_pool);
    const memory::SequenceState& state = page_table.get_state(seq_id);
    const int context_len = state.sequence_length;
    const int position = append_tokens ? logical_position : context_len - 1;
    const int block_size = block_pool.block_size();
    const int head_dim = static_cast<int>(attention_.head_dim());
    const int num_heads = static_cast<int>(attention_.num_heads());
    const int num_kv_heads = static_cast<int>(attention_.num_kv_heads());
    const int hidden = static_cast<int>(hidden_dim_);
    const int inter = static_cast<int>(gate_proj_.output_dim());
    if (position / block_size >= static_cast<int>(state.physical_blocks.size()))
        throw std::runtime_error("TransformerBlock::forward_into: no KV page for decode position");
    void* s = stream_;

    auto fp = [](Tensor& t) { return static_cast<float*>(t.raw_data()); };
    auto cfp = [](const Tensor& t) { return static_cast<const float*>(t.raw_data()); };
    auto linear = [&](const layers::Linear& layer, const Tensor& x, Tensor& y, const char* what) {
        const Tensor& w = layer.weight();
        detail::check(skv_linear_f32(cfp(x), 1, w.raw_data(),
                                     w.dtype() == DataType::BF16 ? SKV_DTYPE_BF16 : SKV_DTYPE_FP32,
                                     static_cast<int64_t>(w.strides()[0]), static_cast<int64_t>(w.strides()[1]),
                                     static_cast<int>(layer.input_dim()), static_cast<int>(layer.output_dim()),
                                     layer.bias() ? cfp(*layer.bias()) : nullptr, fp(y), s),
                      what);
    };
    Tensor& normalized_input = *normalized_input_workspace_;
    Tensor& queries = *query_workspace_;
    Tensor& keys = *key_workspace_;
    Tensor& values = *value_workspace_;
    Tensor& context = *context_workspace_;
    Tensor& normalized_residual = *normalized_residual_workspace_;
    Tensor& gate = *gate_workspace_;
    Tensor& up = *up_workspace_;
    Tensor& down = *down_workspace_;

    auto wdtype = [](const layers::Linear& l) {
        return l.weight().dtype() == DataType::BF16 ? SKV_DTYPE_BF16 : SKV_DTYPE_FP32;
    };
    auto stride_k = [](const layers::Linear& l) { return static_cast<int64_t>(l.weight().strides()[0]); };
    auto stride_n = [](const layers::Linear& l) { return static_cast<int64_t>(l.weight().strides()[1]); };
    auto bias_of = [&](const layers::Linear& l) { return l.bias() ? cfp(*l.bias()) : nullptr; };
    // A fused call returns SKV_ERR_UNSUPPORTED (doing nothing) for weights that
    // are not aligned output-major rows; the separate kernels then run.
    auto fused = [](int rc, const char* what) {
        if (rc == SKV_ERR_UNSUPPORTED) return false;
        detail::check(rc, what);
        return true;
    };
    const layers::Linear& wq = attention_.query_projection();
    const layers::Linear& wk = attention_.key_projection();
    const layers::Linear& wv = attention_.value_projection();
    const layers::Linear& wo = attention_.output_projection();
    const bool same_dtype = wdtype(wq) == wdtype(wk) && wdtype(wq) == wdtype(wv) &&
                            stride_k(wq) == stride_k(wk) && stride_k(wq) == stride_k(wv);

    // Input RMSNorm, q/k/v projections and RoPE at `position`.
    const int64_t qkv_strides[3] = {stride_n(wq), stride_n(wk), stride_n(wv)};
    if (!(same_dtype &&
          fused(skv_fused_qkv_f32(cfp(hidden_states), cfp(norm1_.gamma()), norm1_.epsilon(),
                                  wq.weight().raw_data(), wk.weight().raw_data(), wv.weight().raw_data(),
                                  wdtype(wq), stride_k(wq), qkv_strides, bias_of(wq), bias_of(wk),
                                  bias_of(wv), hidden, num_heads, num_kv_heads, head_dim, position,
                                  fp(queries), fp(keys), fp(values), s),
                "forward_into: fused rmsnorm + q/k/v + rope"))) {
        detail::check(skv_rmsnorm_f32(cfp(hidden_states), fp(normalized_input), cfp(norm1_.gamma()), 1,
                                      hidden, norm1_.epsilon(), s),
                      "forward_into: input rmsnorm");
        linear(wq, normalized_input, queries, "forward_into: q_proj");
        linear(wk, normalized_input, keys, "forward_into: k_proj");
        linear(wv, normalized_input, values, "forward_into: v_proj");
        detail::check(skv_rope_f32(fp(queries), num_heads, head_dim, position, s), "forward_into: rope q");
        detail::check(skv_rope_f32(fp(keys), num_kv_heads, head_dim, position, s), "forward_into: rope k");
    }

    // The paged-KV hot path: device block table (only new block ids are
    // uploaded), then one launch that appends this token's K/V rows at
    // `position` (= context_len - 1) and decodes over the whole context.
    const int* table = page_table.get_device_block_table(seq_id, s);
    Tensor& ws = *decode_workspace_;
    detail::check(skv_paged_attention_decode_append(
                      cfp(queries), cfp(keys), cfp(values), SKV_DTYPE_FP32, block_pool.key_cache(),
                      block_pool.value_cache(), block_pool.total_blocks(), table, fp(context),
                      context_len, block_size, num_heads, num_kv_heads, head_dim,
                      1.0f / std::sqrt(static_cast<float>(head_dim)), ws.raw_data(),
                      ws.num_elements() * ws.element_size(), s),
                  "forward_into: KV append + paged attention");
    // The blocks that attention read: every block of the context.
    attention_.last_blocks_visited_ = std::min<std::size_t>(
        state.physical_blocks.size(), static_cast<std::size_t>((context_len + block_size - 1) / block_size));

    // o_proj + residual: reads hidden_states before output is written
    // (aliasing-safe).  down holds h = hidden + attention output.
    if (!fused(skv_linear_residual_f32(cfp(context), wo.weight().raw_data(), wdtype(wo), stride_k(wo),
                                       stride_n(wo), static_cast<int>(wo.input_dim()),
                                       static_cast<int>(wo.output_dim()), bias_of(wo),
                                       cfp(hidden_states), fp(down), s),
               "forward_into: fused o_proj + residual")) {
        linear(wo, context, down, "forward_into: o_proj");
        detail::check(skv_add_f32(fp(down), cfp(hidden_states), hidden, s), "forward_into: residual");
    }
    // Post-attention RMSNorm, gate/up projections and SwiGLU.
    const bool ffn_same = wdtype(gate_proj_) == wdtype(up_proj_) && stride_k(gate_proj_) == stride_k(up_proj_);
    if (!(ffn_same &&
          fused(skv_fused_gate_up_swiglu_f32(cfp(down), cfp(norm2_.gamma()), norm2_.epsilon(),
                                             gate_proj_.weight().raw_data(), up_proj_.weight().raw_data(),
                                             wdtype(gate_proj_), stride_k(gate_proj_), stride_n(gate_proj_),
                                             stride_n(up_proj_), bias_of(gate_proj_), bias_of(up_proj_),
                                             hidden, inter, fp(gate), s),
                "forward_into: fused rmsnorm + gate/up + swiglu"))) {
        detail::check(skv_rmsnorm_f32(cfp(down), fp(normalized_residual), cfp(norm2_.gamma()), 1, hidden,
                                      norm2_.epsilon(), s),
                      "forward_into: post-attention rmsnorm");
        linear(gate_proj_, normalized_residual, gate, "forward_into: gate_proj");
        linear(up_proj_, normalized_residual, up, "forward_into: up_proj");
        detail::check(skv_swiglu_f32(fp(gate), cfp(up), inter, s), "forward_into: swiglu");
    }
    // down_proj + residual straight into output (hidden_states is not read any more).
    if (!fused(skv_linear_residual_f32(cfp(gate), down_proj_.weight().raw_data(), wdtype(down_proj_),
                                       stride_k(down_proj_), stride_n(down_proj_), inter, hidden,
                                       bias_of(down_proj_), cfp(down), fp(output), s),
               "forward_into: fused down_proj + residual")) {
        linear(down_proj_, gate, context, "forward_into: down_proj");
        detail::check(skv_add_f32(fp(down), cfp(context), hidden, s), "forward_into: residual");
        detail::check(skv_memcpy_d2d(output.raw_data(), down.raw_data(), hidden_dim_ * sizeof(float), s),
                      "forward_into: output copy");
    }
}

TransformerBlock::PrefillGemmUse TransformerBlock::prefill_gemm_use(int rows) const noexcept {
    PrefillGemmUse use;
    const detail::PromptGemmApi* api = rows >= kPrefillGemmRows ? detail::prompt_gemm_api() : nullptr;
    if (api == nullptr) return use;
    auto takes = [](const layers::Linear& l) {
        return l.weight().dtype() == DataType::BF16 && l.weight().strides()[0] == 1 && l.input_dim() % 8 == 0 &&
               l.input_dim() <= 8192;
    };
    const layers::Linear& wq = attention_.query_projection();
    const layers::Linear& wk = attention_.key_projection();
    const layers::Linear& wv = attention_.value_projection();
    const int hidden = static_cast<int>(hidden_dim_);
    const int inter = static_cast<int>(gate_proj_.output_dim());
    const int q_dim = static_cast<int>(attention_.num_heads() * attention_.head_dim());
    const int kv_dim = static_cast<int>(attention_.num_kv_heads() * attention_.head_dim());
    use.qkv = takes(wq) && takes(wk) && takes(wv);
    use.o = takes(attention_.output_projection());
    use.gate_up = takes(gate_proj_) && takes(up_proj_);
    use.down = takes(down_proj_);
    use.ffn = use.gate_up && use.down;
    auto need = [&](bool on, int in, int outs) {
        if (on) use.bytes = std::max(use.bytes, api->workspace_bytes(rows, in, outs));
    };
    need(use.qkv, hidden, q_dim + 2 * kv_dim);
    need(use.o, q_dim, hidden);
    // The feed-forward call's workspace also serves gate/up and down_proj as
    // separate calls, should it refuse the chunk.
    need(use.ffn, std::max(hidden, inter), std::max(2 * inter, hidden));
    need(use.gate_up, hidden, 2 * inter);
    need(use.down, inter, hidden);
    return use;
}

int TransformerBlock::prefill_chunk_rows() const noexcept {
    // fp32 scratch per token: q, k, v, context, residual, act, normalised
    // input; plus the library GEMMs' workspace of the chunk.
    const std::size_t q_dim = attention_.num_heads() * attention_.head_dim();
    const std::size_t kv_dim = attention_.num_kv_heads() * attention_.head_dim();
    const std::size_t row_bytes = 4 * (2 * q_dim + 2 * kv_dim + 2 * hidden_dim_ + gate_proj_.output_dim());
    int rows = kPrefillChunk;
    while (rows > kPrefillMinChunk &&
           row_bytes * static_cast<std::size_t>(rows) + prefill_gemm_use(rows).bytes > kPrefillScratchBudget)
        rows -= 64;
    return std::max(rows, kPrefillMinChunk);
}

void TransformerBlock::ensure_prefill_workspace(int rows) {
    if (!pf_) pf_ = std::make_shared<PrefillScratch>();
    const std::size_t q_dim = attention_.num_heads() * attention_.head_dim();
    const std::size_t kv_dim = attention_.num_kv_heads() * attention_.head_dim();
    const std::size_t inter = gate_proj_.output_dim();
    const std::size_t dims[4] = {hidden_dim_, q_dim, kv_dim, inter};
    const bool same_shape = std::equal(dims, dims + 4, pf_->dims);
    if (same_shape && rows <= pf_->rows) return;
    const std::size_t r = static_cast<std::size_t>(same_shape ? rows : std::max(rows, pf_->rows));
    auto make = [&](std::optional<Tensor>& t, std::size_t dim) {
        t.emplace(std::vector<std::size_t>{r, dim}, DataType::FP32, Device::GPU);
    };
    make(pf_->queries, q_dim);
    make(pf_->keys, kv_dim);
    make(pf_->values, kv_dim);
    make(pf_->context, q_dim);
    make(pf_->residual, hidden_dim_);
    make(pf_->act, inter);
    make(pf_->normalized, hidden_dim_);
    pf_->up.reset();
    pf_->down.reset();
    if (!pf_->meta) pf_->meta.emplace(std::vector<std::size_t>{4}, DataType::FP32, Device::GPU);
    pf_->rows = static_cast<int>(r);
    std::copy(dims, dims + 4, pf_->dims);
}

void* TransformerBlock::prefill_gemm_workspace(std::size_t bytes) {
    std::optional<Tensor>& b = pf_->gemm;
    if (!b || b->num_elements() * sizeof(float) < bytes)
        b.emplace(std::vector<std::size_t>{(bytes + sizeof(float) - 1) / sizeof(float)}, DataType::FP32,
                  Device::GPU);
    return b->raw_data();
}

void TransformerBlock::prefill_into(const Tensor& hidden_states, Tensor& output, int seq_id,
                                    memory::PageTable& page_table, memory::BlockPool& block_pool) {
    if (hidden_states.ndim() != 2 || hidden_states.shape()[1] != hidden_dim_ || hidden_states.shape()[0] == 0 ||
        output.device() != hidden_states.device() || output.shape() != hidden_states.shape() ||
        output.dtype() != DataType::FP32 || hidden_states.dtype() != DataType::FP32)
        throw std::invalid_argument("TransformerBlock::prefill_into: output shape, dtype or device mismatch");
    if (output.device() != Device::GPU)
        throw std::runtime_error("TransformerBlock::prefill_into: GPU tensors required");
    if (norm1_.gamma().dtype() != DataType::FP32 || norm2_.gamma().dtype() != DataType::FP32 ||
        norm1_.gamma().device() != Device::GPU || norm2_.gamma().device() != Device::GPU)
        throw std::runtime_error("TransformerBlock::prefill_into: RMSNorm weights are not on GPU");
    if (attention_.query_projection().weight().device() != Device::GPU ||
        attention_.key_projection().weight().device() != Device::GPU ||
        attention_.value_projection().weight().device() != Device::GPU ||
        attention_.output_projection().weight().device() != Device::GPU ||
        gate_proj_.weight().device() != Device::GPU || up_proj_.weight().device() != Device::GPU ||
        down_proj_.weight().device() != Device::GPU)
        throw std::runtime_error("TransformerBlock::prefill_into: projection weights are not on GPU");
    if (block_pool.device() != Device::GPU || block_pool.key_cache() == nullptr ||
        block_pool.value_cache() == nullptr ||
        block_pool.num_kv_heads() != static_cast<int>(attention_.num_kv_heads()) ||
        block_pool.head_dim() != static_cast<int>(attention_.head_dim()))
        throw std::invalid_argument(
            "TransformerBlock::prefill_into: GPU BlockPool configuration does not match attention");
    if (!page_table.has_sequence(seq_id))
        throw std::runtime_error("TransformerBlock::prefill_into: seq_id is not registered");

    const int tokens = static_cast<int>(hidden_states.shape()[0]);
    const int block_size = block_pool.block_size();
    const int head_dim = static_cast<int>(attention_.head_dim());
    const int num_heads = static_cast<int>(attention_.num_heads());
    const int num_kv_heads = static_cast<int>(attention_.num_kv_heads());
    const int hidden = static_cast<int>(hidden_dim_);
    const int inter = static_cast<int>(gate_proj_.output_dim());
    const int q_dim = num_heads * head_dim;
    const int chunk = prefill_chunk_rows();
    ensure_prefill_workspace(std::min(tokens, chunk));
    const std::size_t ws_rows = static_cast<std::size_t>(pf_->rows);
    auto fallback_buffer = [&](std::optional<Tensor>& t, std::size_t dim) {
        if (!t) t.emplace(std::vector<std::size_t>{ws_rows, dim}, DataType::FP32, Device::GPU);
        return static_cast<float*>(t->raw_data());
    };
    void* s = stream_;

    auto fp = [](Tensor& t) { return static_cast<float*>(t.raw_data()); };
    auto cfp = [](const Tensor& t) { return static_cast<const float*>(t.raw_data()); };
    auto wdtype = [](const layers::Linear& l) {
        return l.weight().dtype() == DataType::BF16 ? SKV_DTYPE_BF16 : SKV_DTYPE_FP32;
    };
    auto stride_k = [](const layers::Linear& l) { return static_cast<int64_t>(l.weight().strides()[0]); };
    auto stride_n = [](const layers::Linear& l) { return static_cast<int64_t>(l.weight().strides()[1]); };
    auto bias_of = [&](const layers::Linear& l) { return l.bias() ? cfp(*l.bias()) : nullptr; };
    auto fused = [](int rc, const char* what) {
        if (rc == SKV_ERR_UNSUPPORTED) return false;
        detail::check(rc, what);
        return true;
    };
    auto linear = [&](const layers::Linear& layer, const float* x, int rows, float* y, const char* what) {
        detail::check(skv_linear_f32(x, rows, layer.weight().raw_data(), wdtype(layer), stride_k(layer),
                                     stride_n(layer), static_cast<int>(layer.input_dim()),
                                     static_cast<int>(layer.output_dim()), bias_of(layer), y, s),
                      what);
    };
    const layers::Linear& wq = attention_.query_projection();
    const layers::Linear& wk = attention_.key_projection();
    const layers::Linear& wv = attention_.value_projection();
    const layers::Linear& wo = attention_.output_projection();
    const bool same_dtype = wdtype(wq) == wdtype(wk) && wdtype(wq) == wdtype(wv) &&
                            stride_k(wq) == stride_k(wk) && stride_k(wq) == stride_k(wv);
    const bool ffn_same = wdtype(gate_proj_) == wdtype(up_proj_) && stride_k(gate_proj_) == stride_k(up_proj_);
    const int64_t qkv_strides[3] = {stride_n(wq), stride_n(wk), stride_n(wv)};
    float* q = fp(*pf_->queries);
    float* k = fp(*pf_->keys);
    float* v = fp(*pf_->values);
    float* ctx = fp(*pf_->context);
    float* h = fp(*pf_->residual);
    float* act = fp(*pf_->act);
    auto* meta = static_cast<std::int32_t*>(pf_->meta->raw_data());

    last_pass_prefill_ = true;
    for (int c0 = 0; c0 < tokens; c0 += chunk) {
        const int n = std::min(chunk, tokens - c0);
        const float* x = cfp(hidden_states) + static_cast<std::size_t>(c0) * hidden;
        float* y = fp(output) + static_cast<std::size_t>(c0) * hidden;
        const int p0 = page_table.get_state(seq_id).sequence_length;
        for (int i = 0; i < n; ++i) page_table.append_token(seq_id, block_pool);
        const memory::SequenceState& state = page_table.get_state(seq_id);
        const int nblocks = static_cast<int>(state.physical_blocks.size());
        const std::int32_t meta_h[4] = {p0, 0, n, p0 + n};
        detail::check(skv_write_i32(meta, meta_h, 4, s), "prefill_into: chunk metadata");
        // Each projection: the matrix-core entry point for long chunks, else
        // (or when it does not take the shape) the rows kernels, else the
        // separate kernels.
        const bool mm = n >= kPrefillMmRows;
        // From kPrefillGemmRows tokens the projections whose weights the
        // library GEMMs take run there (one workspace sized for the widest of
        // those): the 2,048-token prompt of the TinyLlama shape took 14.8 ms
        // so against 15.2 ms with q/k/v and o_proj on the matrix-core kernels
        // and 17.2 ms with all four there.
        const PrefillGemmUse use = prefill_gemm_use(n);
        const detail::PromptGemmApi* api = use.bytes > 0 ? detail::prompt_gemm_api() : nullptr;
        const std::size_t gemm_bytes = use.bytes;
        void* gemm_ws = api != nullptr ? prefill_gemm_workspace(gemm_bytes) : nullptr;
        // Input RMSNorm, q/k/v projections and RoPE at p0 + row.
        auto qkv = [&](auto entry, float* scratch) {
            return entry(x, n, cfp(norm1_.gamma()), norm1_.epsilon(), wq.weight().raw_data(), wk.weight().raw_data(),
                         wv.weight().raw_data(), wdtype(wq), stride_k(wq), qkv_strides, bias_of(wq), bias_of(wk),
                         bias_of(wv), hidden, num_heads, num_kv_heads, head_dim, p0, q, k, v, scratch, s);
        };
        auto qkv_gemm_entry = [&](const float* xx, int rows, const float* g, float e, const void* a, const void* b,
                                  const void* c, int dt, int64_t sk, const int64_t* sn, const float* ba,
                                  const float* bb, const float* bc, int hd_, int nh, int nkv, int hdim, int pos,
                                  float* qq, float* kk, float* vv, float* scratch, void* st) {
            return api->fused_qkv(xx, rows, g, e, a, b, c, dt, sk, sn, ba, bb, bc, hd_, nh, nkv, hdim, pos, qq, kk, vv,
                                  scratch, gemm_ws, gemm_bytes, st);
        };
        if (!(same_dtype &&
              ((use.qkv && fused(qkv(qkv_gemm_entry, fp(*pf_->normalized)), "prefill_into: q/k/v as library GEMMs")) ||
               (mm && fused(qkv(skv_fused_qkv_mm_f32, fp(*pf_->normalized)), "prefill_into: q/k/v on the matrix cores")) ||
               fused(qkv(skv_fused_qkv_rows_f32, fp(*pf_->normalized)), "prefill_into: fused rmsnorm + q/k/v + rope")))) {
            float* xn = fp(*pf_->normalized);
            detail::check(skv_rmsnorm_f32(x, xn, cfp(norm1_.gamma()), n, hidden, norm1_.epsilon(), s),
                          "prefill_into: input rmsnorm");
            linear(wq, xn, n, q, "prefill_into: q_proj");
            linear(wk, xn, n, k, "prefill_into: k_proj");
            linear(wv, xn, n, v, "prefill_into: v_proj");
            detail::check(skv_rope_rows_f32(q, n, num_heads, head_dim, p0, s), "prefill_into: rope q");
            detail::check(skv_rope_rows_f32(k, n, num_kv_heads, head_dim, p0, s), "prefill_into: rope k");
        }

        // The chunk's K/V rows into the pools (fp32 rounded to bf16 like the
        // decode path), then causal attention over the whole context.
        const int* table = page_table.get_device_block_table(seq_id, s);
        detail::check(skv_kv_append(k, v, SKV_DTYPE_FP32, block_pool.key_cache(), block_pool.value_cache(),
                                    block_pool.total_blocks(), table, nblocks, meta, nullptr, 1, n, num_kv_heads,
                                    head_dim, block_size, s),
                      "prefill_into: KV append");
        detail::check(skv_paged_prefill(q, SKV_DTYPE_FP32, block_pool.key_cache(), block_pool.value_cache(),
                                        block_pool.total_blocks(), table, nblocks, meta + 1, meta + 3, 1, n,
                                        num_heads, num_kv_heads, head_dim, block_size,
                                        1.0f / std::sqrt(static_cast<float>(head_dim)), ctx, s),
                      "prefill_into: paged prefill attention");
        attention_.last_blocks_visited_ = static_cast<std::size_t>(nblocks);

        // o_proj + residual (reads x before y is written: aliasing-safe).
        if (!((use.o && fused(api->linear_residual(ctx, n, wo.weight().raw_data(), wdtype(wo), stride_k(wo),
                                                   stride_n(wo), q_dim, hidden, bias_of(wo), x, h, gemm_ws,
                                                   gemm_bytes, s),
                            "prefill_into: o_proj as a library GEMM")) ||
              (mm && fused(skv_linear_residual_mm_f32(ctx, n, wo.weight().raw_data(), wdtype(wo), stride_k(wo),
                                                      stride_n(wo), q_dim, hidden, bias_of(wo), x, h, s),
                           "prefill_into: o_proj on the matrix cores")) ||
              fused(skv_linear_residual_rows_f32(ctx, n, wo.weight().raw_data(), wdtype(wo), stride_k(wo),
                                                 stride_n(wo), q_dim, hidden, bias_of(wo), x, h, s),
                    "prefill_into: fused o_proj + residual"))) {
            linear(wo, ctx, n, h, "prefill_into: o_proj");
            detail::check(skv_add_f32(h, x, n * hidden, s), "prefill_into: residual");
        }
        // The feed-forward half as one library-GEMM call (the SwiGLU output
        // goes straight to down_proj as its split operand), else in two steps.
        if (!(use.ffn && ffn_same && stride_k(down_proj_) == stride_k(gate_proj_) &&
              wdtype(down_proj_) == wdtype(gate_proj_) &&
              fused(api->ffn_swiglu(h, n, cfp(norm2_.gamma()), norm2_.epsilon(), gate_proj_.weight().raw_data(),
                                    up_proj_.weight().raw_data(), down_proj_.weight().raw_data(), wdtype(gate_proj_),
                                    stride_k(gate_proj_), stride_n(gate_proj_), stride_n(up_proj_),
                                    stride_n(down_proj_), bias_of(gate_proj_), bias_of(up_proj_),
                                    bias_of(down_proj_), hidden, inter, y, fp(*pf_->normalized), gemm_ws,
                                    gemm_bytes, s),
                    "prefill_into: FFN as library GEMMs"))) {
            // Post-attention RMSNorm, gate/up and SwiGLU.
            auto gate_up = [&](auto entry, float* scratch) {
                return entry(h, n, cfp(norm2_.gamma()), norm2_.epsilon(), gate_proj_.weight().raw_data(),
                             up_proj_.weight().raw_data(), wdtype(gate_proj_), stride_k(gate_proj_), stride_n(gate_proj_),
                             stride_n(up_proj_), bias_of(gate_proj_), bias_of(up_proj_), hidden, inter, act, scratch, s);
            };
            // The library-GEMM entry point in the shape of the others (workspace bound here).
            auto gate_up_gemm_entry = [&](const float* xx, int rows, const float* g, float e, const void* a,
                                          const void* b, int dt, int64_t sk, int64_t sa, int64_t sb, const float* ba,
                                          const float* bb, int in, int out, float* y_, float* scratch, void* st) {
                return api->fused_gate_up_swiglu(xx, rows, g, e, a, b, dt, sk, sa, sb, ba, bb, in, out, y_, scratch,
                                                 gemm_ws, gemm_bytes, st);
            };
            if (!(ffn_same &&
                  ((use.gate_up && fused(gate_up(gate_up_gemm_entry, fp(*pf_->normalized)),
                                         "prefill_into: gate/up as library GEMMs")) ||
                   (mm && fused(gate_up(skv_fused_gate_up_swiglu_mm_f32, fp(*pf_->normalized)),
                                "prefill_into: gate/up on the matrix cores")) ||
                   fused(gate_up(skv_fused_gate_up_swiglu_rows_f32, fp(*pf_->normalized)),
                         "prefill_into: fused rmsnorm + gate/up + swiglu")))) {
                float* hn = fp(*pf_->normalized);
                float* up = fallback_buffer(pf_->up, static_cast<std::size_t>(inter));
                detail::check(skv_rmsnorm_f32(h, hn, cfp(norm2_.gamma()), n, hidden, norm2_.epsilon(), s),
                              "prefill_into: post-attention rmsnorm");
                linear(gate_proj_, hn, n, act, "prefill_into: gate_proj");
                linear(up_proj_, hn, n, up, "prefill_into: up_proj");
                detail::check(skv_swiglu_f32(act, up, n * inter, s), "prefill_into: swiglu");
            }
            // down_proj + residual into the output rows.
            if (!((use.down && fused(api->linear_residual(act, n, down_proj_.weight().raw_data(), wdtype(down_proj_),
                                                          stride_k(down_proj_), stride_n(down_proj_), inter, hidden,
                                                          bias_of(down_proj_), h, y, gemm_ws, gemm_bytes, s),
                                "prefill_into: down_proj as a library GEMM")) ||
                  (mm && fused(skv_linear_residual_mm_f32(act, n, down_proj_.weight().raw_data(), wdtype(down_proj_),
                                                          stride_k(down_proj_), stride_n(down_proj_), inter, hidden,
                                                          bias_of(down_proj_), h, y, s),
                               "prefill_into: down_proj on the matrix cores")) ||
                  fused(skv_linear_residual_rows_f32(act, n, down_proj_.weight().raw_data(), wdtype(down_proj_),
                                                     stride_k(down_proj_), stride_n(down_proj_), inter, hidden,
                                                     bias_of(down_proj_), h, y, s),
                        "prefill_into: fused down_proj + residual"))) {
                float* d = fallback_buffer(pf_->down, hidden_dim_);
                linear(down_proj_, act, n, d, "prefill_into: down_proj");
                detail::check(skv_add_f32(h, d, n * hidden, s), "prefill_into: residual");
                detail::check(skv_memcpy_d2d(y, h, static_cast<std::size_t>(n) * hidden * sizeof(float), s),
                              "prefill_into: output copy");
            }
        }
    }
}

}  // namespace models
}  // namespace stratakv

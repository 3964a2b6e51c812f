// parity_model.cpp -- the host model of STRATAKV_PARITY=1 (see the header).
// Arithmetic of the reference's CPU layer (src/models/transformer_block.cpp:
// 275-332, src/layers/attention.cpp:96-135, 153-342), in double.
#include "parity_model.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <thread>

#include "abi_check.h"

namespace stratakv {
namespace detail {
namespace {

// The bytes a tensor's elements occupy in its storage (its strides' span),
// copied to the host.
std::vector<unsigned char> storage_bytes(const Tensor& t, std::size_t* span_out) {
    std::size_t span = t.num_elements() == 0 ? 0 : 1;
    for (std::size_t d = 0; d < t.ndim() && span > 0; ++d) span += (t.shape()[d] - 1) * t.strides()[d];
    std::vector<unsigned char> out(span * t.element_size());
    if (!out.empty()) {
        if (t.device() == Device::GPU)
            check(skv_memcpy_d2h(out.data(), t.raw_data(), out.size(), nullptr), "parity model: weight copy");
        else
            std::memcpy(out.data(), t.raw_data(), out.size());
    }
    *span_out = span;
    return out;
}

double widen_bf16(std::uint16_t b) {
    const std::uint32_t bits = static_cast<std::uint32_t>(b) << 16;
    float f;
    std::memcpy(&f, &bits, sizeof f);
    return f;
}

// A 1-D tensor (gamma, bias) as doubles.
std::vector<double> host_values(const Tensor& t) {
    std::size_t span = 0;
    const std::vector<unsigned char> raw = storage_bytes(t, &span);
    std::vector<double> v(t.num_elements());
    const std::size_t stride = t.ndim() == 0 ? 1 : t.strides().back();
    for (std::size_t i = 0; i < v.size(); ++i) {
        if (t.dtype() == DataType::BF16) {
            std::uint16_t b;
            std::memcpy(&b, raw.data() + 2 * i * stride, 2);
            v[i] = widen_bf16(b);
        } else {
            float f;
            std::memcpy(&f, raw.data() + 4 * i * stride, 4);
            v[i] = f;
        }
    }
    return v;
}

// x -> float -> bf16 by round-to-nearest-even -> double: the value an fp32
// K/V row element keeps in a bf16 pool.
double round_bf16(double x) {
    const float f = static_cast<float>(x);
    std::uint32_t bits;
    std::memcpy(&bits, &f, sizeof bits);
    if ((bits & 0x7F800000u) == 0x7F800000u) return f;   // inf / NaN kept
    bits = (bits + 0x7FFFu + ((bits >> 16) & 1u)) & 0xFFFF0000u;
    float r;
    std::memcpy(&r, &bits, sizeof r);
    return r;
}

std::vector<double> rmsnorm(const std::vector<double>& x, const std::vector<double>& gamma, double eps) {
    double ss = 0.0;
    for (double v : x) ss += v * v;
    const double scale = 1.0 / std::sqrt(ss / static_cast<double>(x.size()) + eps);
    std::vector<double> y(x.size());
    for (std::size_t i = 0; i < x.size(); ++i) y[i] = x[i] * scale * gamma[i];
    return y;
}

// Split-half RoPE at `position`: pair i of each head is (i, i + head_dim / 2),
// inverse frequency 10000^(-2i / head_dim) rounded to float.
void rope(std::vector<double>& x, std::size_t heads, std::size_t head_dim, int position) {
    const std::size_t half = head_dim / 2;
    for (std::size_t i = 0; i < half; ++i) {
        const float inv = static_cast<float>(std::pow(10000.0, -2.0 * static_cast<double>(i) / head_dim));
        const double angle = static_cast<double>(position) * static_cast<double>(inv);
        const double c = std::cos(angle), s = std::sin(angle);
        for (std::size_t h = 0; h < heads; ++h) {
            double& a = x[h * head_dim + i];
            double& b = x[h * head_dim + i + half];
            const double a0 = a, b0 = b;
            a = a0 * c - b0 * s;
            b = a0 * s + b0 * c;
        }
    }
}

}  // namespace

HostLinear::HostLinear(const layers::Linear& linear) : in_(linear.input_dim()), out_(linear.output_dim()) {
    const Tensor& w = linear.weight();
    if (w.ndim() != 2 || w.shape()[0] != in_ || w.shape()[1] != out_)
        throw std::invalid_argument("parity model: unexpected projection weight shape");
    stride_in_ = w.strides()[0];
    stride_out_ = w.strides()[1];
    bf16_ = w.dtype() == DataType::BF16;
    std::size_t span = 0;
    const std::vector<unsigned char> raw = storage_bytes(w, &span);
    if (bf16_) {
        w16_.resize(span);
        std::memcpy(w16_.data(), raw.data(), raw.size());
    } else {
        w32_.resize(span);
        std::memcpy(w32_.data(), raw.data(), raw.size());
    }
    if (linear.bias() != nullptr) bias_ = host_values(*linear.bias());
}

double HostLinear::weight(std::size_t o, std::size_t i) const noexcept {
    const std::size_t at = i * stride_in_ + o * stride_out_;
    return bf16_ ? widen_bf16(w16_[at]) : static_cast<double>(w32_[at]);
}

std::vector<double> HostLinear::apply(const std::vector<double>& x) const {
    std::vector<double> y(out_);
    auto rows = [&](std::size_t first, std::size_t step) {
        for (std::size_t o = first; o < out_; o += step) {
            double acc = bias_.empty() ? 0.0 : bias_[o];
            for (std::size_t i = 0; i < in_; ++i) acc += weight(o, i) * x[i];
            y[o] = acc;
        }
    };
    const unsigned hw = std::max(1u, std::thread::hardware_concurrency());
    const unsigned threads = in_ * out_ >= (std::size_t{1} << 20) ? std::min(16u, hw) : 1u;
    if (threads == 1) {
        rows(0, 1);
        return y;
    }
    std::vector<std::thread> pool;
    for (unsigned t = 0; t < threads; ++t) pool.emplace_back(rows, t, threads);
    for (auto& th : pool) th.join();
    return y;
}

ParityModel::ParityModel(const std::vector<models::TransformerBlock>& blocks, const layers::RMSNorm& final_norm,
                         const layers::Linear& lm_head, const Tensor& embeddings)
    : lm_head_(lm_head), embeddings_(&embeddings) {
    if (blocks.empty()) throw std::invalid_argument("parity model: no layers");
    const layers::PagedAttention& a0 = blocks.front().attention();
    heads_ = a0.num_heads();
    kv_heads_ = a0.num_kv_heads();
    head_dim_ = a0.head_dim();
    hidden_ = blocks.front().input_norm().gamma().num_elements();
    for (const auto& b : blocks) {
        Layer L;
        L.gamma1 = host_values(b.input_norm().gamma());
        L.eps1 = b.input_norm().epsilon();
        L.gamma2 = host_values(b.post_attention_norm().gamma());
        L.eps2 = b.post_attention_norm().epsilon();
        L.q = HostLinear(b.attention().query_projection());
        L.k = HostLinear(b.attention().key_projection());
        L.v = HostLinear(b.attention().value_projection());
        L.o = HostLinear(b.attention().output_projection());
        L.gate = HostLinear(b.gate_proj());
        L.up = HostLinear(b.up_proj());
        L.down = HostLinear(b.down_proj());
        layers_.push_back(std::move(L));
    }
    final_gamma_ = host_values(final_norm.gamma());
    final_eps_ = final_norm.epsilon();
}

void ParityModel::reset() {
    for (auto& L : layers_) {
        L.k_cache.clear();
        L.v_cache.clear();
        L.positions = 0;
    }
}

std::vector<double> ParityModel::embedding(int token) const {
    const Tensor& e = *embeddings_;
    if (token < 0 || e.ndim() != 2 || static_cast<std::size_t>(token) >= e.shape()[0])
        throw std::invalid_argument("parity model: token outside the embedding table");
    const std::size_t row_elems = e.shape()[1];
    const std::size_t es = e.element_size();
    std::vector<unsigned char> raw(row_elems * es);
    const auto* src = static_cast<const unsigned char*>(e.raw_data()) +
                      static_cast<std::size_t>(token) * e.strides()[0] * es;
    if (e.device() == Device::GPU)
        check(skv_memcpy_d2h(raw.data(), src, raw.size(), nullptr), "parity model: embedding row");
    else
        std::memcpy(raw.data(), src, raw.size());
    std::vector<double> x(row_elems);
    for (std::size_t i = 0; i < row_elems; ++i) {
        if (e.dtype() == DataType::BF16) {
            std::uint16_t b;
            std::memcpy(&b, raw.data() + 2 * i, 2);
            x[i] = widen_bf16(b);
        } else {
            float f;
            std::memcpy(&f, raw.data() + 4 * i, 4);
            x[i] = f;
        }
    }
    return x;
}

std::vector<double> ParityModel::layer(std::size_t l, const std::vector<double>& x, HostLayerOps* ops) {
    Layer& L = layers_.at(l);
    const int position = L.positions;
    const std::size_t kv_dim = kv_heads_ * head_dim_;
    HostLayerOps local;
    HostLayerOps& r = ops != nullptr ? *ops : local;
    r.norm1 = rmsnorm(x, L.gamma1, L.eps1);
    r.q = L.q.apply(r.norm1);
    r.k = L.k.apply(r.norm1);
    r.v = L.v.apply(r.norm1);
    r.q_rot = r.q;
    r.k_rot = r.k;
    rope(r.q_rot, heads_, head_dim_, position);
    rope(r.k_rot, kv_heads_, head_dim_, position);
    for (std::size_t i = 0; i < kv_dim; ++i) {
        L.k_cache.push_back(round_bf16(r.k_rot[i]));
        L.v_cache.push_back(round_bf16(r.v[i]));
    }
    L.positions = position + 1;
    // Two-pass softmax over positions 0 .. position (src/layers/attention.cpp:263-337).
    const std::size_t group = heads_ / kv_heads_;
    const double scale = 1.0 / std::sqrt(static_cast<double>(head_dim_));
    r.context.assign(heads_ * head_dim_, 0.0);
    std::vector<double> s(static_cast<std::size_t>(L.positions));
    for (std::size_t h = 0; h < heads_; ++h) {
        const std::size_t kvh = h / group;
        double mx = -INFINITY;
        for (int t = 0; t < L.positions; ++t) {
            const double* kr = L.k_cache.data() + static_cast<std::size_t>(t) * kv_dim + kvh * head_dim_;
            double d = 0.0;
            for (std::size_t e = 0; e < head_dim_; ++e) d += r.q_rot[h * head_dim_ + e] * kr[e];
            s[t] = d * scale;
            mx = std::max(mx, s[t]);
        }
        double den = 0.0;
        for (int t = 0; t < L.positions; ++t) den += (s[t] = std::exp(s[t] - mx));
        for (int t = 0; t < L.positions; ++t) {
            const double* vr = L.v_cache.data() + static_cast<std::size_t>(t) * kv_dim + kvh * head_dim_;
            for (std::size_t e = 0; e < head_dim_; ++e) r.context[h * head_dim_ + e] += s[t] / den * vr[e];
        }
    }
    r.out_proj = L.o.apply(r.context);
    r.residual.resize(x.size());
    for (std::size_t i = 0; i < x.size(); ++i) r.residual[i] = x[i] + r.out_proj[i];
    r.norm2 = rmsnorm(r.residual, L.gamma2, L.eps2);
    r.gate = L.gate.apply(r.norm2);
    r.up = L.up.apply(r.norm2);
    r.act.resize(r.gate.size());
    for (std::size_t i = 0; i < r.act.size(); ++i) r.act[i] = r.gate[i] / (1.0 + std::exp(-r.gate[i])) * r.up[i];
    r.down = L.down.apply(r.act);
    r.output.resize(x.size());
    for (std::size_t i = 0; i < x.size(); ++i) r.output[i] = r.residual[i] + r.down[i];
    return r.output;
}

std::vector<double> ParityModel::final_norm(const std::vector<double>& x) const {
    return rmsnorm(x, final_gamma_, final_eps_);
}

double max_abs_diff(const std::vector<float>& gpu, const std::vector<double>& cpu) {
    double m = 0.0;
    const std::size_t n = std::min(gpu.size(), cpu.size());
    for (std::size_t i = 0; i < n; ++i) m = std::max(m, std::fabs(static_cast<double>(gpu[i]) - cpu[i]));
    return m;
}

}  // namespace detail
}  // namespace stratakv

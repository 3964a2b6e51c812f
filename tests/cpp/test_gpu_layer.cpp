// test_gpu_layer.cpp -- GPU tests of the C++ host layer through the C ABI:
//  * PageTable::get_device_block_table (incremental uploads, switching
//    sequences) and DeviceBatch (incremental batched tables);
//  * BlockPool device pools and their deep copy;
//  * TransformerBlock::forward_into against a float64 CPU restatement of the
//    decoder layer (src/models/transformer_block.cpp:334-613) over 40 tokens
//    crossing block boundaries: the appended K/V rows must be the bf16
//    rounding of the reference rows, the attention is the oracle's over the
//    device pool's own bits, and every layer output must match; plus
//    append_tokens=false and input/output aliasing;
//  * TransformerBlock::prefill_into (several tokens per call, chunked) against
//    the same float64 layer with causal attention per token, then decode
//    steps on the cache it wrote.
// Exit status 77 when no GPU is visible (the reference's skip convention).
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

#include "oracle.h"
#include "stratakv/memory/block_pool.h"
#include "stratakv/memory/page_table.h"
#include "stratakv/models/transformer_block.h"
#include "stratakv/tensor.h"
#include "stratakv_amd.h"

using stratakv::DataType;
using stratakv::Device;
using stratakv::Tensor;
using stratakv::memory::BlockPool;
using stratakv::memory::DeviceBatch;
using stratakv::memory::PageTable;

namespace {

int failures = 0;

void check(bool ok, const std::string& what) {
    if (!ok) {
        std::fprintf(stderr, "FAIL: %s\n", what.c_str());
        ++failures;
    }
}

void ok_or_die(int rc, const char* what) {
    if (rc != SKV_OK) throw std::runtime_error(std::string(what) + ": " + skv_last_error());
}

template <typename T>
std::vector<T> download(const void* dev, std::size_t n) {
    std::vector<T> h(n);
    ok_or_die(skv_memcpy_d2h(h.data(), dev, n * sizeof(T), nullptr), "download");
    return h;
}

void device_tables() {
    BlockPool pool(64, 4, 2, 64, Device::GPU);
    PageTable pt;
    pt.allocate_sequence(0, pool);
    pt.allocate_sequence(1, pool);
    for (int step = 0; step < 30; ++step) {
        pt.append_token(0, pool);
        if (step % 3 == 0) pt.append_token(1, pool);
        const int sid = step % 5 == 0 ? 1 : 0;  // switch the staged sequence now and then
        const int* d = pt.get_device_block_table(sid);
        const auto& blocks = pt.get_state(sid).physical_blocks;
        check(download<int>(d, blocks.size()) == blocks, "device block table step " + std::to_string(step));
    }
    // Batched tables: three sequences, incremental syncs.
    DeviceBatch batch(4, 32);
    pt.allocate_sequence(2, pool);
    batch.bind(pt, {2, 0, 1});
    for (int step = 0; step < 20; ++step) {
        pt.append_token(2, pool);
        pt.append_token(0, pool);
        if (step % 4 == 0) pt.append_token(1, pool);
        batch.sync(pt);
        ok_or_die(skv_device_synchronize(), "sync");
        const auto tables = download<int32_t>(batch.tables(), 4 * 32);
        const auto lens = download<int32_t>(batch.context_lens(), 3);
        const auto pos = download<int32_t>(batch.positions(), 3);
        const int ids[3] = {2, 0, 1};
        for (int i = 0; i < 3; ++i) {
            const auto& st = pt.get_state(ids[i]);
            bool same = lens[i] == st.sequence_length && pos[i] == st.sequence_length - 1;
            for (std::size_t k = 0; k < st.physical_blocks.size(); ++k)
                same = same && tables[i * 32 + k] == st.physical_blocks[k];
            check(same, "DeviceBatch row " + std::to_string(i) + " step " + std::to_string(step));
        }
    }
    // A bound seq_id freed and allocated again between syncs, with at least as
    // many blocks as were uploaded: its block went to another sequence, so the
    // row must be re-uploaded whole (stale ids would send the fused append
    // into a block the other sequence owns).
    {
        BlockPool p2(16, 4, 2, 64, Device::GPU);
        PageTable t2;
        t2.allocate_sequence(7, p2);  // block 0
        DeviceBatch b2(2, 8);
        b2.bind(t2, {7});
        const int old_first = t2.get_state(7).physical_blocks[0];
        t2.free_sequence(7, p2);      // block 0 back on top of the free stack
        t2.allocate_sequence(8, p2);  // takes block 0
        t2.allocate_sequence(7, p2);  // a different block
        for (int k = 0; k < 4; ++k) t2.append_token(7, p2);
        const auto& st = t2.get_state(7);
        check(st.physical_blocks[0] != old_first, "re-allocated sequence got a different block");
        b2.sync(t2);
        ok_or_die(skv_device_synchronize(), "sync");
        const auto row = download<int32_t>(b2.tables(), st.physical_blocks.size());
        const auto len = download<int32_t>(b2.context_lens(), 1);
        check(std::vector<int>(row.begin(), row.end()) == st.physical_blocks && len[0] == st.sequence_length,
              "DeviceBatch re-uploads the row of a re-allocated seq_id");
    }
}

void pool_copy() {
    BlockPool a(8, 16, 4, 64, Device::GPU);
    const std::size_t n = a.total_blocks() * a.block_elements();
    ok_or_die(skv_fill_normal_bf16(a.key_cache(), n, 7, 0, nullptr), "fill");
    ok_or_die(skv_fill_normal_bf16(a.value_cache(), n, 8, 0, nullptr), "fill");
    BlockPool b(a);
    check(b.key_cache() != a.key_cache(), "copy owns new storage");
    check(download<uint16_t>(b.key_cache(), n) == download<uint16_t>(a.key_cache(), n) &&
              download<uint16_t>(b.value_cache(), n) == download<uint16_t>(a.value_cache(), n),
          "pool copy is a deep device copy");
}

// ---------------------------------------------------------------------------
// Float64 restatement of one decoder layer.
// ---------------------------------------------------------------------------
struct HostLayer {
    int H, I, Hq, Hkv, hd;
    std::vector<double> g1, g2;                  // gammas
    std::vector<double> wq, wk, wv, wo;          // logical [in][out]
    std::vector<double> wg, wu, wd;
};

std::vector<double> matvec(const std::vector<double>& x, const std::vector<double>& w, int in, int out) {
    std::vector<double> y(out, 0.0);
    for (int k = 0; k < in; ++k)
        for (int n = 0; n < out; ++n) y[n] += x[k] * w[static_cast<std::size_t>(k) * out + n];
    return y;
}

std::vector<double> rmsnorm(const std::vector<double>& x, const std::vector<double>& g) {
    double s = 0.0;
    for (double v : x) s += v * v;
    const double inv = 1.0 / std::sqrt(s / x.size() + 1e-5);
    std::vector<double> y(x.size());
    for (std::size_t i = 0; i < x.size(); ++i) y[i] = x[i] * inv * g[i];
    return y;
}

void rope(std::vector<double>& x, int heads, int hd, int pos) {
    const int half = hd / 2;
    for (int h = 0; h < heads; ++h)
        for (int i = 0; i < half; ++i) {
            const float inv = static_cast<float>(std::pow(10000.0, -2.0 * i / static_cast<double>(hd)));
            const double ang = static_cast<double>(pos) * static_cast<double>(inv);
            const double c = std::cos(ang), s = std::sin(ang);
            double& a = x[h * hd + i];
            double& b = x[h * hd + i + half];
            const double a0 = a, b0 = b;
            a = a0 * c - b0 * s;
            b = a0 * s + b0 * c;
        }
}

uint16_t bf16_of(double v) { return oracle_f32_to_bf16_rne(static_cast<float>(v)); }

// Fills a block's weights (bf16 checkpoint rows behind a transpose view for
// the attention projections, fp32 GEMM-ready FFN) and the same values as
// float64 into `ref`.
void build_layer(stratakv::models::TransformerBlock& block, HostLayer& ref, std::mt19937& rng) {
    const int H = ref.H;
    std::normal_distribution<float> nd(0.0f, 1.0f);
    auto gamma = [&](stratakv::layers::RMSNorm& norm, std::vector<double>& g) {
        g.resize(H);
        for (int i = 0; i < H; ++i) {
            const float v = 1.0f + 0.1f * nd(rng);
            norm.gamma()[i] = v;
            g[i] = v;
        }
    };
    gamma(block.input_norm(), ref.g1);
    gamma(block.post_attention_norm(), ref.g2);
    auto bf16_rows = [&](stratakv::layers::Linear& layer, std::vector<double>& w) {
        const int in = static_cast<int>(layer.input_dim()), out = static_cast<int>(layer.output_dim());
        Tensor rows({static_cast<std::size_t>(out), static_cast<std::size_t>(in)}, DataType::BF16);
        w.assign(static_cast<std::size_t>(in) * out, 0.0);
        for (int n = 0; n < out; ++n)
            for (int k = 0; k < in; ++k) {
                rows[static_cast<std::size_t>(n) * in + k] = 0.05f * nd(rng);
                w[static_cast<std::size_t>(k) * out + n] = rows[static_cast<std::size_t>(n) * in + k];
            }
        layer.set_weight(rows.transpose_2d());
    };
    bf16_rows(block.attention().query_projection(), ref.wq);
    bf16_rows(block.attention().key_projection(), ref.wk);
    bf16_rows(block.attention().value_projection(), ref.wv);
    bf16_rows(block.attention().output_projection(), ref.wo);
    auto fp32_cols = [&](stratakv::layers::Linear& layer, std::vector<double>& w) {
        const std::size_t n = layer.input_dim() * layer.output_dim();
        w.resize(n);
        for (std::size_t i = 0; i < n; ++i) {
            const float v = 0.04f * nd(rng);
            layer.weight()[i] = v;
            w[i] = v;
        }
    };
    fp32_cols(block.gate_proj(), ref.wg);
    fp32_cols(block.up_proj(), ref.wu);
    fp32_cols(block.down_proj(), ref.wd);
}

// The float64 layer output of one token at `pos`, attending through `table`
// over the first `len` positions of the pools as the device holds them.
std::vector<double> ref_layer_token(const HostLayer& ref, const std::vector<double>& xd, int pos,
                                    const std::vector<uint16_t>& kp, const std::vector<uint16_t>& vp, int total,
                                    const std::vector<int32_t>& table, int32_t len, int bs) {
    const int H = ref.H, I = ref.I, Hq = ref.Hq, Hkv = ref.Hkv, hd = ref.hd;
    std::vector<double> n1 = rmsnorm(xd, ref.g1);
    std::vector<double> q = matvec(n1, ref.wq, H, H);
    rope(q, Hq, hd, pos);
    std::vector<float> qf(q.begin(), q.end()), ctx(H);
    check(oracle_paged_decode_f32(qf.data(), kp.data(), vp.data(), total, table.data(),
                                  static_cast<int>(table.size()), &len, 1, Hq, Hkv, hd, bs,
                                  1.0f / std::sqrt(static_cast<float>(hd)), ctx.data()) == 0,
          "oracle attention");
    std::vector<double> c(ctx.begin(), ctx.end());
    std::vector<double> o = matvec(c, ref.wo, H, H);
    std::vector<double> h(H);
    for (int i = 0; i < H; ++i) h[i] = xd[i] + o[i];
    std::vector<double> n2 = rmsnorm(h, ref.g2);
    std::vector<double> g = matvec(n2, ref.wg, H, I), u = matvec(n2, ref.wu, H, I);
    for (int i = 0; i < I; ++i) g[i] = g[i] / (1.0 + std::exp(-g[i])) * u[i];
    std::vector<double> d = matvec(g, ref.wd, I, H);
    std::vector<double> y(H);
    for (int i = 0; i < H; ++i) y[i] = h[i] + d[i];
    return y;
}

void transformer_block_parity() {
    const int H = 512, I = 768, Hq = 8, Hkv = 2, hd = H / Hq, bs = 16, total = 12, T = 40;
    std::mt19937 rng(2024);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    stratakv::models::TransformerBlock block(H, I, Hq, Hkv, total, bs);
    HostLayer ref{H, I, Hq, Hkv, hd, {}, {}, {}, {}, {}, {}, {}, {}, {}};
    build_layer(block, ref, rng);
    block.to(Device::GPU);

    BlockPool pool(total, bs, Hkv, hd, Device::GPU);
    ok_or_die(skv_fill_u16(pool.key_cache(), total * pool.block_elements(), 0xFFFF, nullptr), "poison");
    ok_or_die(skv_fill_u16(pool.value_cache(), total * pool.block_elements(), 0xFFFF, nullptr), "poison");
    PageTable pt;
    pt.allocate_sequence(0, pool);
    pt.allocate_sequence(1, pool);  // interleave: sequence 0's pages are non-contiguous

    Tensor x_dev({1, static_cast<std::size_t>(H)}, DataType::FP32, Device::GPU);
    Tensor y_dev({1, static_cast<std::size_t>(H)}, DataType::FP32, Device::GPU);
    double worst = 0.0, worst_kv = 0.0;
    auto run_step = [&](bool append, bool alias) {
        std::vector<float> x(H);
        for (float& v : x) v = nd(rng);
        ok_or_die(skv_memcpy_h2d(x_dev.raw_data(), x.data(), H * sizeof(float), nullptr), "upload");
        const int pos = append ? pt.get_state(0).sequence_length : pt.get_state(0).sequence_length - 1;
        if (alias) block.forward_into(x_dev, x_dev, 0, pt, pool, append);
        else block.forward_into(x_dev, y_dev, 0, pt, pool, append);
        if (append && pt.get_state(0).sequence_length % bs == 1) pt.append_token(1, pool);
        ok_or_die(skv_device_synchronize(), "sync");
        const std::vector<float> y = download<float>(alias ? x_dev.raw_data() : y_dev.raw_data(), H);

        // Reference, with the K/V pools as the device holds them.
        std::vector<double> xd(x.begin(), x.end());
        std::vector<double> n1 = rmsnorm(xd, ref.g1);
        std::vector<double> q = matvec(n1, ref.wq, H, H);
        std::vector<double> k = matvec(n1, ref.wk, H, Hkv * hd);
        std::vector<double> v = matvec(n1, ref.wv, H, Hkv * hd);
        rope(q, Hq, hd, pos);
        rope(k, Hkv, hd, pos);
        const std::size_t pool_n = total * pool.block_elements();
        std::vector<uint16_t> kp = download<uint16_t>(pool.key_cache(), pool_n);
        std::vector<uint16_t> vp = download<uint16_t>(pool.value_cache(), pool_n);
        const auto& st = pt.get_state(0);
        const std::size_t row = (static_cast<std::size_t>(st.physical_blocks[pos / bs]) * bs + pos % bs) * Hkv * hd;
        for (int e = 0; e < Hkv * hd; ++e) {
            // The appended rows are the bf16 rounding of the fp32 K/V (one bf16 ulp of slack).
            const double gk = oracle_bf16_to_f32(kp[row + e]), gv = oracle_bf16_to_f32(vp[row + e]);
            worst_kv = std::max(worst_kv, std::fabs(gk - oracle_bf16_to_f32(bf16_of(k[e]))) / (std::fabs(k[e]) + 1e-3));
            worst_kv = std::max(worst_kv, std::fabs(gv - oracle_bf16_to_f32(bf16_of(v[e]))) / (std::fabs(v[e]) + 1e-3));
        }
        std::vector<float> qf(q.begin(), q.end()), ctx(H);
        const int32_t len = st.sequence_length;
        std::vector<int32_t> table(st.physical_blocks.begin(), st.physical_blocks.end());
        check(oracle_paged_decode_f32(qf.data(), kp.data(), vp.data(), total, table.data(),
                                      static_cast<int>(table.size()), &len, 1, Hq, Hkv, hd, bs,
                                      1.0f / std::sqrt(static_cast<float>(hd)), ctx.data()) == 0,
              "oracle attention");
        std::vector<double> c(ctx.begin(), ctx.end());
        std::vector<double> o = matvec(c, ref.wo, H, H);
        std::vector<double> h(H);
        for (int i = 0; i < H; ++i) h[i] = xd[i] + o[i];
        std::vector<double> n2 = rmsnorm(h, ref.g2);
        std::vector<double> g = matvec(n2, ref.wg, H, I), u = matvec(n2, ref.wu, H, I);
        for (int i = 0; i < I; ++i) g[i] = g[i] / (1.0 + std::exp(-g[i])) * u[i];
        std::vector<double> d = matvec(g, ref.wd, I, H);
        for (int i = 0; i < H; ++i) {
            const double want = h[i] + d[i];
            const double err = std::fabs(y[i] - want);
            worst = std::max(worst, err / (1e-3 + 1e-3 * std::fabs(want)));
        }
        return y;
    };
    for (int t = 0; t < T; ++t) run_step(true, false);
    check(pt.get_state(0).sequence_length == T, "forward_into appended every token");
    check(pt.get_state(0).physical_blocks.size() == 3 &&
              pt.get_state(0).physical_blocks[1] != pt.get_state(0).physical_blocks[0] + 1,
          "sequence pages are non-contiguous");
    run_step(false, false);  // append_tokens = false: rewrite the last slot, same length
    check(pt.get_state(0).sequence_length == T, "append_tokens=false keeps the length");
    run_step(false, true);   // aliased input/output
    check(worst <= 1.0, "forward_into matches the float64 layer (worst error / bound = " + std::to_string(worst) + ")");
    check(worst_kv <= 1.0 / 64, "appended K/V are the bf16 rounding of the rows (" + std::to_string(worst_kv) + ")");
    std::printf("forward_into: worst error/bound %.3g, worst K/V rel diff %.3g\n", worst, worst_kv);

    // Validation mirrors the reference's exceptions.
    Tensor cpu_x({1, static_cast<std::size_t>(H)});
    Tensor cpu_y({1, static_cast<std::size_t>(H)});
    bool threw = false;
    try {
        block.forward_into(cpu_x, cpu_y, 0, pt, pool);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    check(threw, "CPU tensors are rejected");
    threw = false;
    try {
        block.forward_into(x_dev, y_dev, 9, pt, pool);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    check(threw, "unknown sequence is rejected");
    BlockPool wrong(4, bs, Hkv + 1, hd, Device::GPU);
    threw = false;
    try {
        block.forward_into(x_dev, y_dev, 0, pt, wrong);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    check(threw, "mismatched pool geometry is rejected");
}

// TransformerBlock::prefill_into: several tokens per call (a 2,100-token prompt
// = two internal chunks, then a second 21-token chunk with aliased
// input/output), then decode steps through forward_into on the cache the
// prefill wrote.  Every output row against the float64 layer with causal
// attention over the pools as the device holds them; the prefill's K/V rows
// against the bf16 rounding of the float64 K/V.
void prefill_parity() {
    const int H = 512, I = 768, Hq = 8, Hkv = 2, hd = H / Hq, bs = 16, total = 140;
    std::mt19937 rng(77);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    stratakv::models::TransformerBlock block(H, I, Hq, Hkv, total, bs);
    HostLayer ref{H, I, Hq, Hkv, hd, {}, {}, {}, {}, {}, {}, {}, {}, {}};
    build_layer(block, ref, rng);
    block.to(Device::GPU);
    BlockPool pool(total, bs, Hkv, hd, Device::GPU);
    ok_or_die(skv_fill_u16(pool.key_cache(), total * pool.block_elements(), 0xFFFF, nullptr), "poison");
    ok_or_die(skv_fill_u16(pool.value_cache(), total * pool.block_elements(), 0xFFFF, nullptr), "poison");
    PageTable pt;
    pt.allocate_sequence(3, pool);
    const std::size_t pool_n = total * pool.block_elements();
    double worst = 0.0, worst_kv = 0.0;
    std::vector<std::vector<double>> inputs;  // every token's layer input, by position

    // Runs `n` new tokens (prefill_into when prefill, else forward_into per
    // token) and checks their outputs and appended K/V.
    auto run = [&](int n, bool prefill, bool alias) {
        const int p0 = pt.get_state(3).sequence_length;
        std::vector<float> x(static_cast<std::size_t>(n) * H);
        for (float& v : x) v = nd(rng);
        for (int t = 0; t < n; ++t) inputs.emplace_back(x.begin() + t * H, x.begin() + (t + 1) * H);
        std::vector<float> y;
        if (prefill) {
            Tensor xd({static_cast<std::size_t>(n), static_cast<std::size_t>(H)}, DataType::FP32, Device::GPU);
            Tensor yd({static_cast<std::size_t>(n), static_cast<std::size_t>(H)}, DataType::FP32, Device::GPU);
            ok_or_die(skv_memcpy_h2d(xd.raw_data(), x.data(), x.size() * sizeof(float), nullptr), "upload");
            if (alias) block.prefill_into(xd, xd, 3, pt, pool);
            else block.prefill_into(xd, yd, 3, pt, pool);
            ok_or_die(skv_device_synchronize(), "sync");
            y = download<float>(alias ? xd.raw_data() : yd.raw_data(), x.size());
        } else {
            Tensor xd({1, static_cast<std::size_t>(H)}, DataType::FP32, Device::GPU);
            for (int t = 0; t < n; ++t) {
                ok_or_die(skv_memcpy_h2d(xd.raw_data(), x.data() + t * H, H * sizeof(float), nullptr), "upload");
                block.forward_into(xd, xd, 3, pt, pool, true);
                ok_or_die(skv_device_synchronize(), "sync");
                const std::vector<float> yt = download<float>(xd.raw_data(), H);
                y.insert(y.end(), yt.begin(), yt.end());
            }
        }
        const auto& st = pt.get_state(3);
        check(st.sequence_length == p0 + n, "every token appended");
        const std::vector<uint16_t> kp = download<uint16_t>(pool.key_cache(), pool_n);
        const std::vector<uint16_t> vp = download<uint16_t>(pool.value_cache(), pool_n);
        const std::vector<int32_t> table(st.physical_blocks.begin(), st.physical_blocks.end());
        for (int t = 0; t < n; ++t) {
            const int pos = p0 + t;
            const std::vector<double>& xt = inputs[pos];
            // Appended K/V: the bf16 rounding of the float64 rows (one bf16 ulp of slack).
            std::vector<double> n1 = rmsnorm(xt, ref.g1);
            std::vector<double> k = matvec(n1, ref.wk, H, Hkv * hd), v = matvec(n1, ref.wv, H, Hkv * hd);
            rope(k, Hkv, hd, pos);
            const std::size_t row = (static_cast<std::size_t>(table[pos / bs]) * bs + pos % bs) * Hkv * hd;
            for (int e = 0; e < Hkv * hd; ++e) {
                const double gk = oracle_bf16_to_f32(kp[row + e]), gv = oracle_bf16_to_f32(vp[row + e]);
                worst_kv = std::max(worst_kv, std::fabs(gk - oracle_bf16_to_f32(bf16_of(k[e]))) / (std::fabs(k[e]) + 1e-3));
                worst_kv = std::max(worst_kv, std::fabs(gv - oracle_bf16_to_f32(bf16_of(v[e]))) / (std::fabs(v[e]) + 1e-3));
            }
            const std::vector<double> want = ref_layer_token(ref, xt, pos, kp, vp, total, table, pos + 1, bs);
            for (int i = 0; i < H; ++i)
                worst = std::max(worst, std::fabs(y[static_cast<std::size_t>(t) * H + i] - want[i]) /
                                            (1e-3 + 1e-3 * std::fabs(want[i])));
        }
    };
    check(block.prefill_chunk_rows() == 2048, "prefill chunk of this layer: 2,048 tokens");
    run(2100, true, false);  // prompt: 2,048 + 52 tokens inside prefill_into
    run(21, true, true);     // a later chunk, input and output aliased
    run(2, false, false);    // decode on the prefilled cache
    check(pt.get_state(3).sequence_length == 2123, "prefill + decode length");
    check(worst <= 1.0, "prefill_into matches the float64 layer (worst error / bound = " + std::to_string(worst) + ")");
    check(worst_kv <= 1.0 / 64, "prefill K/V are the bf16 rounding of the rows (" + std::to_string(worst_kv) + ")");
    std::printf("prefill_into: worst error/bound %.3g, worst K/V rel diff %.3g\n", worst, worst_kv);

    bool threw = false;
    try {
        Tensor xd({2, static_cast<std::size_t>(H)}, DataType::FP32, Device::GPU);
        Tensor yd({3, static_cast<std::size_t>(H)}, DataType::FP32, Device::GPU);
        block.prefill_into(xd, yd, 3, pt, pool);
    } catch (const std::invalid_argument&) {
        threw = true;
    }
    check(threw, "prefill_into rejects mismatched shapes");
    threw = false;
    try {
        Tensor xd({2, static_cast<std::size_t>(H)}, DataType::FP32, Device::GPU);
        block.prefill_into(xd, xd, 8, pt, pool);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    check(threw, "prefill_into rejects an unknown sequence");
}

}  // namespace

int main() {
    int n = 0;
    if (skv_device_count(&n) != SKV_OK || n < 1) {
        std::printf("test_gpu_layer: no GPU, skipped\n");
        return 77;
    }
    try {
        device_tables();
        pool_copy();
        transformer_block_parity();
        prefill_parity();
    } catch (const std::exception& e) {
        std::fprintf(stderr, "FAIL: unexpected exception %s\n", e.what());
        return 1;
    }
    if (failures) {
        std::fprintf(stderr, "%d check(s) failed\n", failures);
        return 1;
    }
    std::printf("test_gpu_layer: all checks passed\n");
    return 0;
}

// skv_model_ops.hip -- the model boundary on either side of the decode path:
// checkpoint tensors decoded on the device, the embedding lookup, and the
// choice of the next token from the logits (greedy argmax and the
// temperature / top-k / top-p sampler).  Token ids are read from and written
// to device memory, so a generation loop can queue step after step without
// waiting for the host.
//
// Reference behaviour followed (StrataKV source tree):
//   checkpoint decode   src/io/safetensors.cpp:98-104 (BF16 widen), :219-250
//                       (half_to_float), :610-681 and src/cuda/gemm_cuda.cu:74-83
//                       (fp32 -> bf16 by truncation), src/generation/generator.cpp:265-290
//                       (non-finite weights are rejected)
//   embedding lookup    src/cuda/gemm_cuda.cu:286-300, src/generation/generator.cpp:531-552
//   greedy token        src/generation/sampler.cpp:57-62 (first index of the maximum)
//   sampler             src/generation/sampler.cpp:71-147
#include "skv_common.h"

#include <cmath>

namespace skv {

// ---------------------------------------------------------------------------
// Checkpoint element decode.  All three source types are little-endian.
// ---------------------------------------------------------------------------

// IEEE binary16 -> binary32, exact for every input (subnormals normalised,
// infinities and NaN payloads carried over bit for bit).
__device__ __forceinline__ uint32_t half_to_f32_bits(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t mant = h & 0x3FFu;
    if (exp == 0x1Fu) return sign | 0x7F800000u | (mant << 13);
    if (exp != 0) return sign | ((exp + 112u) << 23) | (mant << 13);
    if (mant == 0) return sign;
    // Subnormal: mant * 2^-24.  Shift the leading one up to bit 10.
    const int shift = __builtin_clz(mant) - 21;           // 1..10
    const uint32_t m = (mant << shift) & 0x3FFu;
    return sign | (static_cast<uint32_t>(113 - shift) << 23) | (m << 13);
}

__device__ __forceinline__ uint32_t source_f32_bits(const void* src, int dtype, size_t i) {
    if (dtype == SKV_DTYPE_FP32) return static_cast<const uint32_t*>(src)[i];
    const uint32_t h = static_cast<const uint16_t*>(src)[i];
    return dtype == SKV_DTYPE_BF16 ? h << 16 : half_to_f32_bits(h);
}

__device__ __forceinline__ bool finite_bits(uint32_t b) {
    return (b & 0x7F800000u) != 0x7F800000u;
}

// dst_kind 0: bf16 bits, upper half of the fp32 value (truncation);
// dst_kind 1: fp32 bits; dst NULL: check only.
__global__ void convert_kernel(const void* __restrict__ src, int src_dtype, size_t count,
                               void* __restrict__ dst, int dst_kind, int32_t* __restrict__ nonfinite) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    bool bad = false;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride) {
        const uint32_t b = source_f32_bits(src, src_dtype, i);
        bad |= !finite_bits(b);
        if (dst != nullptr) {
            if (dst_kind == 0) static_cast<uint16_t*>(dst)[i] = static_cast<uint16_t>(b >> 16);
            else static_cast<uint32_t*>(dst)[i] = b;
        }
    }
    if (nonfinite != nullptr && __any(bad) && (threadIdx.x & 63) == 0) atomicOr(nonfinite, 1);
}

int launch_convert(const void* src, int src_dtype, size_t count, void* dst, int dst_kind,
                   int32_t* nonfinite, void* stream, const char* what) {
    SKV_REQUIRE(src != nullptr, "%s: NULL source", what);
    SKV_REQUIRE(src_dtype == SKV_DTYPE_BF16 || src_dtype == SKV_DTYPE_FP32 || src_dtype == SKV_DTYPE_F16,
                "%s: unknown source dtype %d", what, src_dtype);
    if (count == 0) return SKV_OK;
    const size_t blocks = std::min<size_t>(cdiv<size_t>(count, 256), 8192);
    convert_kernel<<<static_cast<unsigned>(blocks), 256, 0, static_cast<hipStream_t>(stream)>>>(
        src, src_dtype, count, dst, dst_kind, nonfinite);
    return check_launch(what);
}

// ---------------------------------------------------------------------------
// Embedding lookup: out[i] = table[ids[index] * hidden + i] widened to fp32.
// An id outside [0, vocab) gives zeros and sets bit SKV_FLAG_BAD_TOKEN.
// ---------------------------------------------------------------------------
// Row blockIdx.y: out[y][i] = table[ids[index + y]][i].  index_at (device,
// may be null) is added to index and flag_at (device, may be null) selects
// the flag word, for launches captured once and replayed per token.
__global__ void embedding_kernel(const void* __restrict__ table, int dtype, int vocab, int hidden,
                                 const int32_t* __restrict__ ids, int index, float* __restrict__ out,
                                 int32_t* __restrict__ flags, const int32_t* __restrict__ index_at,
                                 const int32_t* __restrict__ flag_at) {
    if (index_at != nullptr) index += *index_at;
    if (flags != nullptr && flag_at != nullptr) flags += *flag_at;
    const int id = ids[index + static_cast<int>(blockIdx.y)];
    out += static_cast<size_t>(blockIdx.y) * static_cast<size_t>(hidden);
    const bool ok = id >= 0 && id < vocab;
    if (!ok && threadIdx.x == 0 && blockIdx.x == 0 && flags != nullptr) atomicOr(flags, SKV_FLAG_BAD_TOKEN);
    const size_t row = static_cast<size_t>(ok ? id : 0) * static_cast<size_t>(hidden);
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x)
        out[i] = ok ? __uint_as_float(source_f32_bits(table, dtype, row + i)) : 0.0f;
}

// ---------------------------------------------------------------------------
// Block-wide helpers for the 1024-thread token-choice kernels.
// ---------------------------------------------------------------------------
constexpr int kPickThreads = 1024;
constexpr int kPickWaves = kPickThreads / 64;

struct PickShared {
    int32_t hist_cnt[256];
    double hist_sum[256];
    double wave_d[kPickWaves];
    float wave_f[kPickWaves];
    int32_t wave_i[kPickWaves];
    int32_t wave_j[kPickWaves];
    int32_t sel_bin;
    int32_t sel_below;          // count strictly above the selected bin (top-k)
    double sel_above;           // mass strictly above the selected bin (top-p)
    int32_t found;
    int32_t winner;
};

__device__ __forceinline__ double wave_sum_d(double x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}
__device__ __forceinline__ int wave_sum_i(int x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}
__device__ __forceinline__ int wave_min_i(int x) {
    for (int o = 32; o > 0; o >>= 1) x = min(x, __shfl_xor(x, o, 64));
    return x;
}

__device__ double block_sum_d(double x, PickShared& sh) {
    x = wave_sum_d(x);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh.wave_d[w] = x;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < kPickWaves; ++i) t += sh.wave_d[i];   // same order in every thread
    return t;
}
__device__ int block_sum_i(int x, PickShared& sh) {
    x = wave_sum_i(x);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh.wave_i[w] = x;
    __syncthreads();
    int t = 0;
    for (int i = 0; i < kPickWaves; ++i) t += sh.wave_i[i];
    return t;
}
__device__ int block_min_i(int x, PickShared& sh) {
    x = wave_min_i(x);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh.wave_i[w] = x;
    __syncthreads();
    int t = sh.wave_i[0];
    for (int i = 1; i < kPickWaves; ++i) t = min(t, sh.wave_i[i]);
    return t;
}
__device__ float block_max_f(float x, PickShared& sh) {
    x = wave_max(x);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh.wave_f[w] = x;
    __syncthreads();
    float t = sh.wave_f[0];
    for (int i = 1; i < kPickWaves; ++i) t = fmaxf(t, sh.wave_f[i]);
    return t;
}
// Exclusive prefix over threads in thread order (int and double).
__device__ int block_excl_scan_i(int x, PickShared& sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int inc = x;
    for (int o = 1; o < 64; o <<= 1) {
        const int u = __shfl_up(inc, o, 64);
        if (lane >= o) inc += u;
    }
    __syncthreads();
    if (lane == 63) sh.wave_i[w] = inc;
    __syncthreads();
    int base = 0;
    for (int i = 0; i < w; ++i) base += sh.wave_i[i];
    return base + inc - x;
}
__device__ double block_excl_scan_d(double x, PickShared& sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    double inc = x;
    for (int o = 1; o < 64; o <<= 1) {
        const double u = __shfl_up(inc, o, 64);
        if (lane >= o) inc += u;
    }
    __syncthreads();
    if (lane == 63) sh.wave_d[w] = inc;
    __syncthreads();
    double base = 0.0;
    for (int i = 0; i < w; ++i) base += sh.wave_d[i];
    return base + inc - x;
}

// ---------------------------------------------------------------------------
// Greedy: ids[out_index] = the first index of the maximum logit (strict >
// scan, src/generation/sampler.cpp:57-62).  A non-finite logit sets
// SKV_FLAG_NONFINITE_LOGITS (the reference aborts on one,
// src/generation/generator.cpp:720-732).
// ---------------------------------------------------------------------------
// VEC: logits 16-byte aligned; each thread reads float4s, kArgmaxBatch of
// them in flight (unconditional, clamped), then a scalar tail.  Every thread
// scans its own elements in increasing index, so the first index of the
// maximum wins as in the scalar loop.
constexpr int kArgmaxBatch = 8;

template <bool VEC>
__global__ __launch_bounds__(kPickThreads) void argmax_kernel(const float* __restrict__ logits, int n,
                                                             int32_t* __restrict__ ids, int out_index,
                                                             int32_t* __restrict__ flags,
                                                             const int32_t* __restrict__ index_at,
                                                             const int32_t* __restrict__ flag_at) {
    __shared__ PickShared sh;
    float best = -INFINITY;
    int bi = n;                      // "none": loses every comparison
    bool bad = false;
    auto consider = [&](float v, int i) {
        bad |= !(fabsf(v) <= 3.402823466e38f);
        if (bi == n || v > best) { best = v; bi = i; }
    };
    int tail = 0;
    if constexpr (VEC) {
        const int n4 = n / 4;
        const float4* l4 = reinterpret_cast<const float4*>(logits);
        for (int b0 = threadIdx.x; b0 < n4; b0 += kPickThreads * kArgmaxBatch) {
            float4 v[kArgmaxBatch];
#pragma unroll
            for (int u = 0; u < kArgmaxBatch; ++u) v[u] = l4[min(b0 + u * kPickThreads, n4 - 1)];
#pragma unroll
            for (int u = 0; u < kArgmaxBatch; ++u) {
                const int q = b0 + u * kPickThreads;
                if (q < n4) {
                    consider(v[u].x, 4 * q);
                    consider(v[u].y, 4 * q + 1);
                    consider(v[u].z, 4 * q + 2);
                    consider(v[u].w, 4 * q + 3);
                }
            }
        }
        tail = 4 * n4;
    }
    for (int i = tail + static_cast<int>(threadIdx.x); i < n; i += kPickThreads) consider(logits[i], i);
    // Reduce (value, index): larger value wins, equal values -> smaller index.
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (oi != n && (bi == n || ov > best || (ov == best && oi < bi))) { best = ov; bi = oi; }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) { sh.wave_f[w] = best; sh.wave_j[w] = bi; }
    const int any_bad = __syncthreads_or(bad);
    if (threadIdx.x == 0) {
        float b = sh.wave_f[0];
        int j = sh.wave_j[0];
        for (int i = 1; i < kPickWaves; ++i) {
            const int oi = sh.wave_j[i];
            if (oi != n && (j == n || sh.wave_f[i] > b || (sh.wave_f[i] == b && oi < j))) { b = sh.wave_f[i]; j = oi; }
        }
        // index_at / flag_at (device, may be null): the output index and flag
        // word of launches captured once and replayed per token.
        ids[out_index + (index_at != nullptr ? *index_at : 0)] = j == n ? 0 : j;
        if (any_bad && flags != nullptr) atomicOr(flags + (flag_at != nullptr ? *flag_at : 0), SKV_FLAG_NONFINITE_LOGITS);
    }
}

// ---------------------------------------------------------------------------
// Sampler (src/generation/sampler.cpp:71-147), one workgroup.
//
// 1. v_i = logits_i / T; every logit and every v_i must be finite.
// 2. top-k (0 < k < n): keep the k first elements of the order (v desc,
//    index asc).  A 4-pass 8-bit radix select on an order-preserving key of
//    v finds the k-th value; among elements equal to it the lowest indices
//    are kept.
// 3. w_i = exp(v_i - max) over the kept elements, total = sum w.
// 4. top-p (< 1): in the order (w desc, index asc) an element is kept while
//    the probability mass before it is below top_p.  A radix select on the
//    bits of w (non-negative floats order like their bits) with per-bin mass
//    finds the crossing weight; its ties are kept in index order.
// 5. p_i = w_i / sum(kept w) as float, then the categorical draw of
//    std::discrete_distribution: cp = running sum of p_i / sum(p) in double in
//    index order (cp of the last element forced to 1), result = the first i
//    with cp_i >= u.  `u` is the caller's draw of generate_canonical<double, 53>
//    from the sampler's mt19937 stream.
// Masses are summed in double and in a different order than the reference's
// sequential float loops, so a result can differ only when a top-p or
// categorical boundary lies within rounding of u or top_p.
// Each thread owns a contiguous index range, so scans over threads are scans
// over indices.
// ---------------------------------------------------------------------------
struct SampleArgs {
    const float* logits;
    int n;
    float temperature;
    int top_k;
    float top_p;
    double u;
    int32_t* ids;
    int out_index;
    int32_t* flags;
};

// Monotone map of a finite float onto uint32 (-0 and +0 map together).
__device__ __forceinline__ uint32_t order_key(float v) {
    const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// Wave 0 picks the bin of a radix pass: scanning bins from 255 down, the
// first bin b whose cumulative count (from the top) reaches `need`.
// Returns via sh.sel_bin / sh.sel_below.
__device__ void pick_bin_count(PickShared& sh, int need) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        int c[4], local = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) { c[e] = sh.hist_cnt[255 - 4 * lane - e]; local += c[e]; }
        int inc = local;
        for (int o = 1; o < 64; o <<= 1) {
            const int u = __shfl_up(inc, o, 64);
            if (lane >= o) inc += u;
        }
        int above = inc - local;   // count in bins above this lane's 4 bins
        int bin = -1, below = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (bin < 0 && above + c[e] >= need) { bin = 255 - 4 * lane - e; below = above; }
            above += c[e];
        }
        const int first = wave_min_i(bin >= 0 ? lane : 64);
        if (lane == first) { sh.sel_bin = bin; sh.sel_below = below; }
    }
    __syncthreads();
}

// The same on masses: first bin (from the top) where the mass above it plus
// its own mass reaches `target`; sh.found = 0 when no bin does.  With
// `refine` (a pass inside a bin that did reach the target, whose sub-bin sums
// may round a little lower) the lowest non-empty bin is taken instead.
__device__ void pick_bin_mass(PickShared& sh, double target, bool refine) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        double c[4], local = 0.0;
#pragma unroll
        for (int e = 0; e < 4; ++e) { c[e] = sh.hist_sum[255 - 4 * lane - e]; local += c[e]; }
        double inc = local;
        for (int o = 1; o < 64; o <<= 1) {
            const double u = __shfl_up(inc, o, 64);
            if (lane >= o) inc += u;
        }
        double above = inc - local;
        int bin = -1, low = -1;
        double before = 0.0, low_before = 0.0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (bin < 0 && above + c[e] >= target) { bin = 255 - 4 * lane - e; before = above; }
            if (c[e] > 0.0) { low = 255 - 4 * lane - e; low_before = above; }
            above += c[e];
        }
        const int first = wave_min_i(bin >= 0 ? lane : 64);
        const int last = -wave_min_i(low >= 0 ? -lane : 1);   // highest lane with a non-empty bin
        if (first < 64) {
            if (lane == 0) sh.found = 1;
            if (lane == first) { sh.sel_bin = bin; sh.sel_above = before; }
        } else if (refine && last >= 0) {
            if (lane == 0) sh.found = 1;
            if (lane == last) { sh.sel_bin = low; sh.sel_above = low_before; }
        } else if (lane == 0) {
            sh.found = 0;
        }
    }
    __syncthreads();
}

__global__ __launch_bounds__(kPickThreads) void sample_kernel(SampleArgs a) {
    __shared__ PickShared sh;
    const int n = a.n;
    const int chunk = cdiv(n, kPickThreads);
    const int i0 = min(n, static_cast<int>(threadIdx.x) * chunk);
    const int i1 = min(n, i0 + chunk);
    const float T = a.temperature;

    // 1. scaled values, finiteness, maximum
    bool bad_logit = false, bad_scaled = false;
    float vmax = -INFINITY;
    for (int i = i0; i < i1; ++i) {
        const float x = a.logits[i];
        const float v = x / T;
        bad_logit |= !(fabsf(x) <= 3.402823466e38f);
        bad_scaled |= !(fabsf(v) <= 3.402823466e38f);
        vmax = fmaxf(vmax, v);
    }
    const int any_logit = __syncthreads_or(bad_logit);
    const int any_scaled = __syncthreads_or(bad_scaled);
    if (any_logit || any_scaled) {
        if (threadIdx.x == 0) {
            if (a.flags != nullptr)
                atomicOr(a.flags, any_logit ? SKV_FLAG_NONFINITE_LOGITS : SKV_FLAG_NONFINITE_SCALED);
            a.ids[a.out_index] = 0;
        }
        return;
    }
    const float M = block_max_f(vmax, sh);

    // 2. top-k threshold key K and the number of its ties to keep
    const bool topk = a.top_k > 0 && a.top_k < n;
    uint32_t K = 0;            // keep key > K, and the first `tie_keep` ties of key == K
    int tie_keep = 0, tie_base = 0;
    if (topk) {
        uint32_t prefix = 0, mask = 0;
        int need = a.top_k;
        for (int pass = 0; pass < 4; ++pass) {
            const int shift = 24 - 8 * pass;
            for (int b = threadIdx.x; b < 256; b += kPickThreads) sh.hist_cnt[b] = 0;
            __syncthreads();
            for (int i = i0; i < i1; ++i) {
                const uint32_t key = order_key(a.logits[i] / T);
                if ((key & mask) == prefix) atomicAdd(&sh.hist_cnt[(key >> shift) & 255u], 1);
            }
            __syncthreads();
            pick_bin_count(sh, need);
            need -= sh.sel_below;
            prefix |= static_cast<uint32_t>(sh.sel_bin) << shift;
            mask |= 255u << shift;
            __syncthreads();
        }
        K = prefix;
        tie_keep = need;
        int ties = 0;
        for (int i = i0; i < i1; ++i) ties += order_key(a.logits[i] / T) == K;
        tie_base = block_excl_scan_i(ties, sh);
    }
    // kept_k(i, tie_rank): the top-k filter for element i whose rank among
    // the K-ties (in index order) is tie_rank.
    auto kept_k = [&](uint32_t key, int tie_rank) {
        return !topk || key > K || (key == K && tie_rank < tie_keep);
    };

    // 3. weights over the top-k set and their total
    double tot = 0.0;
    {
        int tr = tie_base;
        for (int i = i0; i < i1; ++i) {
            const float v = a.logits[i] / T;
            const uint32_t key = order_key(v);
            if (kept_k(key, tr)) tot += static_cast<double>(expf(v - M));
            tr += key == K;
        }
    }
    const float total = static_cast<float>(block_sum_d(tot, sh));
    if (!(total > 0.0f) || !(total <= 3.402823466e38f)) {
        if (threadIdx.x == 0) {
            if (a.flags != nullptr) atomicOr(a.flags, SKV_FLAG_BAD_DISTRIBUTION);
            a.ids[a.out_index] = 0;
        }
        return;
    }

    // 4. top-p: crossing weight W and how many of its ties stay
    const bool topp = a.top_p < 1.0f;
    uint32_t W = 0;
    int wtie_keep = 0, wtie_base = 0;
    bool topp_cut = false;
    if (topp) {
        uint32_t prefix = 0, mask = 0;
        double above = 0.0;
        const double target = static_cast<double>(a.top_p);
        bool found = true;
        for (int pass = 0; pass < 4 && found; ++pass) {
            const int shift = 24 - 8 * pass;
            for (int b = threadIdx.x; b < 256; b += kPickThreads) sh.hist_sum[b] = 0.0;
            __syncthreads();
            int tr = tie_base;
            for (int i = i0; i < i1; ++i) {
                const float v = a.logits[i] / T;
                const uint32_t key = order_key(v);
                if (kept_k(key, tr)) {
                    const float w = expf(v - M);
                    const uint32_t wb = __float_as_uint(w);
                    if ((wb & mask) == prefix)
                        atomicAdd(&sh.hist_sum[(wb >> shift) & 255u], static_cast<double>(w / total));
                }
                tr += key == K;
            }
            __syncthreads();
            pick_bin_mass(sh, target - above, pass > 0);
            found = sh.found != 0;
            if (found) {
                above += sh.sel_above;
                prefix |= static_cast<uint32_t>(sh.sel_bin) << shift;
                mask |= 255u << shift;
            }
            __syncthreads();
        }
        if (found) {
            topp_cut = true;
            W = prefix;
            // ties of W in index order: the tie of rank r has mass
            // above + r * q before it and stays while that is below top_p.
            const double q = static_cast<double>(__uint_as_float(W) / total);
            const double room = target - above;          // > 0
            wtie_keep = q > 0.0 ? static_cast<int>(ceil(room / q)) : 0x7FFFFFFF;
            int ties = 0, tr = tie_base;
            for (int i = i0; i < i1; ++i) {
                const float v = a.logits[i] / T;
                const uint32_t key = order_key(v);
                if (kept_k(key, tr) && __float_as_uint(expf(v - M)) == W) ++ties;
                tr += key == K;
            }
            wtie_base = block_excl_scan_i(ties, sh);
        }
    }

    // 5. final weights, total, and the categorical draw in index order
    auto final_weight = [&](int i, int& tr, int& wr) -> float {
        const float v = a.logits[i] / T;
        const uint32_t key = order_key(v);
        float w = 0.0f;
        if (kept_k(key, tr)) {
            w = expf(v - M);
            if (topp_cut) {
                const uint32_t wb = __float_as_uint(w);
                if (wb == W) {
                    if (wr >= wtie_keep) w = 0.0f;
                    ++wr;
                } else if (wb < W) {
                    w = 0.0f;
                }
            }
        }
        tr += key == K;
        return w;
    };
    double tot2 = 0.0;
    {
        int tr = tie_base, wr = wtie_base;
        for (int i = i0; i < i1; ++i) tot2 += static_cast<double>(final_weight(i, tr, wr));
    }
    const float total2 = static_cast<float>(block_sum_d(tot2, sh));
    double psum = 0.0;
    {
        int tr = tie_base, wr = wtie_base;
        for (int i = i0; i < i1; ++i) psum += static_cast<double>(final_weight(i, tr, wr) / total2);
    }
    const double S = block_sum_d(psum, sh);
    double local = 0.0;
    {
        int tr = tie_base, wr = wtie_base;
        for (int i = i0; i < i1; ++i) local += static_cast<double>(final_weight(i, tr, wr) / total2) / S;
    }
    double cp = block_excl_scan_d(local, sh);
    int cand = n - 1;
    {
        int tr = tie_base, wr = wtie_base;
        for (int i = i0; i < i1; ++i) {
            cp += static_cast<double>(final_weight(i, tr, wr) / total2) / S;
            if (cp >= a.u) { cand = i; break; }
        }
    }
    const int pick = block_min_i(cand, sh);
    if (threadIdx.x == 0) a.ids[a.out_index] = pick;
}

}  // namespace skv

using namespace skv;

extern "C" int skv_convert_to_bf16(const void* src, int src_dtype, size_t count, uint16_t* dst,
                                   int32_t* nonfinite, void* stream) {
    SKV_REQUIRE(dst != nullptr || count == 0, "skv_convert_to_bf16: NULL destination");
    return launch_convert(src, src_dtype, count, dst, 0, nonfinite, stream, "skv_convert_to_bf16");
}

extern "C" int skv_convert_to_f32(const void* src, int src_dtype, size_t count, float* dst,
                                  int32_t* nonfinite, void* stream) {
    SKV_REQUIRE(dst != nullptr || count == 0, "skv_convert_to_f32: NULL destination");
    return launch_convert(src, src_dtype, count, dst, 1, nonfinite, stream, "skv_convert_to_f32");
}

extern "C" int skv_check_finite(const void* src, int src_dtype, size_t count, int32_t* nonfinite,
                                void* stream) {
    SKV_REQUIRE(nonfinite != nullptr, "skv_check_finite: NULL flag");
    return launch_convert(src, src_dtype, count, nullptr, 0, nonfinite, stream, "skv_check_finite");
}

namespace {
int embedding_rows(const char* fn, const void* table, int table_dtype, int vocab, int hidden,
                   const int32_t* token_ids, int first_index, int rows, float* out, int32_t* flags, void* stream,
                   const int32_t* index_at = nullptr, const int32_t* flag_at = nullptr) {
    SKV_REQUIRE(table && token_ids && out, "%s: NULL pointer", fn);
    SKV_REQUIRE(table_dtype == SKV_DTYPE_BF16 || table_dtype == SKV_DTYPE_FP32 || table_dtype == SKV_DTYPE_F16,
                "%s: unknown table dtype %d", fn, table_dtype);
    SKV_REQUIRE(vocab > 0 && hidden > 0 && first_index >= 0 && rows > 0 && rows <= 65535 &&
                    first_index <= INT32_MAX - rows,
                "%s: invalid dimensions", fn);
    const dim3 grid(static_cast<unsigned>(std::min(cdiv(hidden, 256), 64)), static_cast<unsigned>(rows));
    embedding_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
        table, table_dtype, vocab, hidden, token_ids, first_index, out, flags, index_at, flag_at);
    return check_launch(fn);
}
}  // namespace

extern "C" int skv_embedding_f32(const void* table, int table_dtype, int vocab, int hidden,
                                 const int32_t* token_ids, int index, float* out, int32_t* flags,
                                 void* stream) {
    return embedding_rows("skv_embedding_f32", table, table_dtype, vocab, hidden, token_ids, index, 1, out, flags,
                          stream);
}

extern "C" int skv_embedding_at_f32(const void* table, int table_dtype, int vocab, int hidden,
                                    const int32_t* token_ids, const int32_t* index_at, float* out, int32_t* flags,
                                    const int32_t* flag_at, void* stream) {
    SKV_REQUIRE(index_at != nullptr, "skv_embedding_at_f32: NULL index");
    return embedding_rows("skv_embedding_at_f32", table, table_dtype, vocab, hidden, token_ids, 0, 1, out, flags,
                          stream, index_at, flag_at);
}

extern "C" int skv_embedding_rows_f32(const void* table, int table_dtype, int vocab, int hidden,
                                      const int32_t* token_ids, int first_index, int rows, float* out,
                                      int32_t* flags, void* stream) {
    return embedding_rows("skv_embedding_rows_f32", table, table_dtype, vocab, hidden, token_ids, first_index, rows,
                          out, flags, stream);
}

namespace {
int launch_argmax(const float* logits, int n, int32_t* ids, int index, int32_t* flags, hipStream_t s,
                  const int32_t* index_at = nullptr, const int32_t* flag_at = nullptr) {
    if (aligned16(logits))
        argmax_kernel<true><<<1, kPickThreads, 0, s>>>(logits, n, ids, index, flags, index_at, flag_at);
    else argmax_kernel<false><<<1, kPickThreads, 0, s>>>(logits, n, ids, index, flags, index_at, flag_at);
    return check_launch("argmax_kernel");
}
}  // namespace

extern "C" int skv_argmax_f32(const float* logits, int n, int32_t* token_ids, int index, int32_t* flags,
                              void* stream) {
    SKV_REQUIRE(logits && token_ids, "skv_argmax_f32: NULL pointer");
    SKV_REQUIRE(n > 0 && index >= 0, "skv_argmax_f32: invalid dimensions");
    return launch_argmax(logits, n, token_ids, index, flags, static_cast<hipStream_t>(stream));
}

extern "C" int skv_argmax_at_f32(const float* logits, int n, int32_t* token_ids, const int32_t* index_at,
                                 int32_t* flags, const int32_t* flag_at, void* stream) {
    SKV_REQUIRE(logits && token_ids && index_at, "skv_argmax_at_f32: NULL pointer");
    SKV_REQUIRE(n > 0, "skv_argmax_at_f32: invalid dimensions");
    return launch_argmax(logits, n, token_ids, 0, flags, static_cast<hipStream_t>(stream), index_at, flag_at);
}

extern "C" int skv_sample_f32(const float* logits, int n, float temperature, int top_k, float top_p,
                              double uniform, int32_t* token_ids, int index, int32_t* flags, void* stream) {
    SKV_REQUIRE(logits && token_ids, "skv_sample_f32: NULL pointer");
    SKV_REQUIRE(n > 0 && index >= 0, "skv_sample_f32: invalid dimensions");
    // Sampler configuration rules of src/generation/sampler.cpp:13-22.
    SKV_REQUIRE(std::isfinite(temperature) && temperature >= 0.0f,
                "Sampler: temperature must be finite and nonnegative");
    SKV_REQUIRE(top_k >= 0, "Sampler: top_k must be nonnegative");
    SKV_REQUIRE(std::isfinite(top_p) && top_p > 0.0f && top_p <= 1.0f, "Sampler: top_p must be in (0, 1]");
    SKV_REQUIRE(uniform >= 0.0 && uniform < 1.0, "skv_sample_f32: uniform must be in [0, 1)");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (temperature == 0.0f) {
        return launch_argmax(logits, n, token_ids, index, flags, s);
    }
    SampleArgs a{logits, n, temperature, top_k, top_p, uniform, token_ids, index, flags};
    sample_kernel<<<1, kPickThreads, 0, s>>>(a);
    return check_launch("skv_sample_f32");
}

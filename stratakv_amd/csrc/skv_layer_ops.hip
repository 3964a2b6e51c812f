// skv_layer_ops.hip -- the non-attention sub-steps of a decoder layer's
// decode step (TransformerBlock::forward_into): RMSNorm, the projections as
// GEMV over bf16 or fp32 weights, split-half RoPE, SwiGLU and the residual
// add.  They exist so the drop-in forward_into runs end to end on the GPU;
// the GEMV streams the weights with 16-byte loads (it is most of a layer's
// time); the others are simple elementwise kernels.
//
// Reference behaviour followed (StrataKV sources):
//   rmsnorm  src/cuda/gemm_cuda.cu:172-202 (sum of squares, 1/sqrt(mean + eps))
//   linear   src/layers/linear.cpp:113-163 (Y = X * W, W logical [in, out],
//            GEMM-ready or a transpose view over output-major rows)
//   rope     src/layers/attention.cpp:96-135 (split-half pairs, inverse
//            frequency 10000^(-2i/hd) rounded to float, angle in double)
//   swiglu   src/models/transformer_block.cpp:315-323 (overflow-safe sigmoid)
#include "skv_common.h"

#include <algorithm>
#include <cmath>

namespace skv {

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ in,
                                                      float* __restrict__ out,
                                                      const float* __restrict__ gamma, int n,
                                                      float eps) {
    __shared__ float red[4];
    const int row = blockIdx.x;
    const float* x = in + static_cast<int64_t>(row) * n;
    float* y = out + static_cast<int64_t>(row) * n;
    float s = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) s = fmaf(x[i], x[i], s);
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    const float total = (red[0] + red[1]) + (red[2] + red[3]);
    const float inv = 1.0f / sqrtf(total / static_cast<float>(n) + eps);
    for (int i = threadIdx.x; i < n; i += 256) y[i] = x[i] * inv * gamma[i];
}

template <bool BF16W>
__device__ __forceinline__ float weight_at(const void* w, int64_t idx) {
    if constexpr (BF16W) return bf16_to_f32(static_cast<const uint16_t*>(w)[idx]);
    else return static_cast<const float*>(w)[idx];
}

// 16 bytes of weights -> 8 (bf16) or 4 (fp32) floats.
template <bool BF16W>
__device__ __forceinline__ void widen16(const uint4& q, float* f) {
    if constexpr (BF16W) {
        f[0] = bf16_lo(q.x); f[1] = bf16_hi(q.x); f[2] = bf16_lo(q.y); f[3] = bf16_hi(q.y);
        f[4] = bf16_lo(q.z); f[5] = bf16_hi(q.z); f[6] = bf16_lo(q.w); f[7] = bf16_hi(q.w);
    } else {
        f[0] = __uint_as_float(q.x); f[1] = __uint_as_float(q.y);
        f[2] = __uint_as_float(q.z); f[3] = __uint_as_float(q.w);
    }
}

constexpr int kGemvRowsPerWave = 2;    // output rows per wavefront
constexpr int kGemvUnroll = 4;         // 16-byte loads per row in flight
constexpr int kGemvMaxLdsK = 8192;     // x staged in LDS up to this many inputs

// Output-major weights (stride_k == 1, 16-byte aligned rows): output n is the
// dot product of x with the contiguous row n.  One wavefront per 2 rows, 16
// bytes per lane per load with 4 loads per row issued together (8 KiB in
// flight per wavefront); x is staged once per workgroup in LDS.  Further rows
// of x (tokens) read the weights again, from L2.
template <bool BF16W>
__global__ __launch_bounds__(256) void gemv_rows_vec_kernel(const float* __restrict__ x, int rows,
                                                            const void* __restrict__ w,
                                                            int64_t stride_n, int K, int N,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ y) {
    constexpr int EPL = BF16W ? 8 : 4;           // elements per 16-byte load
    constexpr int STEP = 64 * EPL;               // elements per wave-wide load
    extern __shared__ float x_s[];               // [rows][K] when it fits
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int n0 = wave * kGemvRowsPerWave;
    const bool lds_x = static_cast<int64_t>(rows) * K <= kGemvMaxLdsK;
    if (lds_x) {
        for (int i = threadIdx.x; i < rows * K; i += 256) x_s[i] = x[i];
        __syncthreads();
    }
    if (n0 >= N) return;
    const int nrows = min(kGemvRowsPerWave, N - n0);
    const char* wb = static_cast<const char*>(w);
    const int64_t esz = BF16W ? 2 : 4;
    for (int r = 0; r < rows; ++r) {
        const float* xr = lds_x ? x_s + static_cast<int64_t>(r) * K : x + static_cast<int64_t>(r) * K;
        float acc[kGemvRowsPerWave] = {};
        int k0 = 0;
        // Main part: kGemvUnroll full wave-wide steps, every load unconditional.
        for (; k0 + kGemvUnroll * STEP <= K; k0 += kGemvUnroll * STEP) {
            uint4 q[kGemvRowsPerWave][kGemvUnroll];
#pragma unroll
            for (int j = 0; j < kGemvRowsPerWave; ++j) {
                const int n = n0 + min(j, nrows - 1);
#pragma unroll
                for (int u = 0; u < kGemvUnroll; ++u)
                    q[j][u] = *reinterpret_cast<const uint4*>(
                        wb + (static_cast<int64_t>(n) * stride_n + k0 + u * STEP + lane * EPL) * esz);
            }
#pragma unroll
            for (int u = 0; u < kGemvUnroll; ++u) {
                float xv[EPL];
#pragma unroll
                for (int e = 0; e < EPL; ++e) xv[e] = xr[k0 + u * STEP + lane * EPL + e];
#pragma unroll
                for (int j = 0; j < kGemvRowsPerWave; ++j) {
                    float f[EPL];
                    widen16<BF16W>(q[j][u], f);
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[j] = fmaf(xv[e], f[e], acc[j]);
                }
            }
        }
        // Tail: whole 16-byte chunks, then single elements.
        for (int k = k0 + lane * EPL; k + EPL <= K; k += STEP) {
#pragma unroll
            for (int j = 0; j < kGemvRowsPerWave; ++j) {
                if (j >= nrows) break;
                float f[EPL];
                widen16<BF16W>(*reinterpret_cast<const uint4*>(
                                   wb + (static_cast<int64_t>(n0 + j) * stride_n + k) * esz), f);
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[j] = fmaf(xr[k + e], f[e], acc[j]);
            }
        }
        const int kt = K - K % EPL;
        for (int k = kt + lane; k < K; k += 64)
            for (int j = 0; j < nrows; ++j)
                acc[j] = fmaf(xr[k], weight_at<BF16W>(w, static_cast<int64_t>(n0 + j) * stride_n + k), acc[j]);
#pragma unroll
        for (int j = 0; j < kGemvRowsPerWave; ++j) {
            const float v = wave_sum(acc[j]);
            if (lane == 0 && j < nrows)
                y[static_cast<int64_t>(r) * N + n0 + j] = v + (bias ? bias[n0 + j] : 0.0f);
        }
    }
}

// Output-major weights without 16-byte alignment: one wavefront per output,
// lanes over k.
template <bool BF16W>
__global__ __launch_bounds__(256) void gemv_rows_kernel(const float* __restrict__ x, int rows,
                                                        const void* __restrict__ w,
                                                        int64_t stride_n, int K, int N,
                                                        const float* __restrict__ bias,
                                                        float* __restrict__ y) {
    const int wave = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int lane = threadIdx.x & 63;
    if (wave >= rows * N) return;
    const int r = wave / N, n = wave - r * N;
    const float* xr = x + static_cast<int64_t>(r) * K;
    const int64_t base = static_cast<int64_t>(n) * stride_n;
    float s = 0.0f;
    for (int k = lane; k < K; k += 64) s = fmaf(xr[k], weight_at<BF16W>(w, base + k), s);
    s = wave_sum(s);
    if (lane == 0) y[static_cast<int64_t>(r) * N + n] = s + (bias ? bias[n] : 0.0f);
}

// GEMM-ready weights (stride_n == 1): threads over outputs, loop over k; the
// 4 wavefronts of a workgroup split k and meet in LDS.
template <bool BF16W>
__global__ __launch_bounds__(256) void gemv_cols_kernel(const float* __restrict__ x, int rows,
                                                        const void* __restrict__ w,
                                                        int64_t stride_k, int K, int N,
                                                        const float* __restrict__ bias,
                                                        float* __restrict__ y) {
    __shared__ float part[4][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int n = blockIdx.x * 64 + lane;
    const int r = blockIdx.y;
    const float* xr = x + static_cast<int64_t>(r) * K;
    const int kq = cdiv(K, 4);
    const int kb = wv * kq, ke = min(K, kb + kq);
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    if (n < N) {
        int k = kb;
        for (; k + 4 <= ke; k += 4) {
            const float w0 = weight_at<BF16W>(w, static_cast<int64_t>(k) * stride_k + n);
            const float w1 = weight_at<BF16W>(w, static_cast<int64_t>(k + 1) * stride_k + n);
            const float w2 = weight_at<BF16W>(w, static_cast<int64_t>(k + 2) * stride_k + n);
            const float w3 = weight_at<BF16W>(w, static_cast<int64_t>(k + 3) * stride_k + n);
            s0 = fmaf(xr[k], w0, s0);
            s1 = fmaf(xr[k + 1], w1, s1);
            s2 = fmaf(xr[k + 2], w2, s2);
            s3 = fmaf(xr[k + 3], w3, s3);
        }
        for (; k < ke; ++k) s0 = fmaf(xr[k], weight_at<BF16W>(w, static_cast<int64_t>(k) * stride_k + n), s0);
    }
    part[wv][lane] = (s0 + s1) + (s2 + s3);
    __syncthreads();
    if (wv == 0 && n < N)
        y[static_cast<int64_t>(r) * N + n] =
            ((part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane])) + (bias ? bias[n] : 0.0f);
}

__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ x, int heads, int hd,
                                                   int position) {
    const int half = hd / 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= heads * half) return;
    const int h = i / half, pair = i - h * half;
    const float inv = static_cast<float>(pow(10000.0, -2.0 * pair / static_cast<double>(hd)));
    const double angle = static_cast<double>(position) * static_cast<double>(inv);
    const float c = static_cast<float>(cos(angle));
    const float s = static_cast<float>(sin(angle));
    float* p = x + static_cast<int64_t>(h) * hd;
    const float a = p[pair], b = p[pair + half];
    p[pair] = a * c - b * s;
    p[pair + half] = a * s + b * c;
}

__global__ __launch_bounds__(256) void swiglu_kernel(float* __restrict__ gate,
                                                     const float* __restrict__ up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float g = gate[i];
    const float sig = g >= 0.0f ? 1.0f / (1.0f + expf(-g)) : expf(g) / (1.0f + expf(g));
    gate[i] = g * sig * up[i];
}

__global__ __launch_bounds__(256) void add_kernel(float* __restrict__ t, const float* __restrict__ s,
                                                  int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) t[i] += s[i];
}

}  // namespace skv

using namespace skv;

extern "C" int skv_rmsnorm_f32(const float* input, float* output, const float* gamma, int rows,
                               int hidden, float epsilon, void* stream) {
    SKV_REQUIRE(input && output && gamma && rows > 0 && hidden > 0,
                "skv_rmsnorm_f32: invalid pointers or sizes");
    rmsnorm_kernel<<<rows, 256, 0, static_cast<hipStream_t>(stream)>>>(input, output, gamma, hidden,
                                                                        epsilon);
    return check_launch("rmsnorm_kernel");
}

extern "C" int skv_linear_f32(const float* x, int rows, const void* weight, int weight_dtype,
                              int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                              const float* bias, float* y, void* stream) {
    SKV_REQUIRE(x && weight && y && rows > 0 && in_dim > 0 && out_dim > 0,
                "skv_linear_f32: invalid pointers or sizes");
    SKV_REQUIRE(weight_dtype == SKV_DTYPE_BF16 || weight_dtype == SKV_DTYPE_FP32,
                "skv_linear_f32: unknown weight dtype %d", weight_dtype);
    SKV_REQUIRE((stride_k == 1 && stride_n >= in_dim) || (stride_n == 1 && stride_k >= out_dim),
                "skv_linear_f32: weight strides (%lld, %lld) are neither output- nor input-major",
                static_cast<long long>(stride_k), static_cast<long long>(stride_n));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool bf16 = weight_dtype == SKV_DTYPE_BF16;
    const int64_t esz = bf16 ? 2 : 4;
    if (stride_k == 1 && aligned16(weight) && (stride_n * esz) % 16 == 0 && rows <= 64) {
        const unsigned grid = static_cast<unsigned>(cdiv(out_dim, 4 * kGemvRowsPerWave));
        const bool lds_x = static_cast<int64_t>(rows) * in_dim <= kGemvMaxLdsK;
        const size_t lds = lds_x ? sizeof(float) * static_cast<size_t>(rows) * in_dim : 0;
        if (bf16) gemv_rows_vec_kernel<true><<<grid, 256, lds, s>>>(x, rows, weight, stride_n, in_dim, out_dim, bias, y);
        else gemv_rows_vec_kernel<false><<<grid, 256, lds, s>>>(x, rows, weight, stride_n, in_dim, out_dim, bias, y);
    } else if (stride_k == 1) {
        const int64_t threads = static_cast<int64_t>(rows) * out_dim * 64;
        const unsigned grid = static_cast<unsigned>(cdiv<int64_t>(threads, 256));
        if (bf16) gemv_rows_kernel<true><<<grid, 256, 0, s>>>(x, rows, weight, stride_n, in_dim, out_dim, bias, y);
        else gemv_rows_kernel<false><<<grid, 256, 0, s>>>(x, rows, weight, stride_n, in_dim, out_dim, bias, y);
    } else {
        const dim3 grid(static_cast<unsigned>(cdiv(out_dim, 64)), static_cast<unsigned>(rows));
        if (bf16) gemv_cols_kernel<true><<<grid, 256, 0, s>>>(x, rows, weight, stride_k, in_dim, out_dim, bias, y);
        else gemv_cols_kernel<false><<<grid, 256, 0, s>>>(x, rows, weight, stride_k, in_dim, out_dim, bias, y);
    }
    return check_launch("gemv_kernel");
}

extern "C" int skv_rope_f32(float* x, int heads, int head_dim, int position, void* stream) {
    SKV_REQUIRE(x && heads > 0 && head_dim > 0 && head_dim % 2 == 0 && position >= 0,
                "skv_rope_f32: invalid pointers or sizes");
    const int n = heads * (head_dim / 2);
    rope_kernel<<<cdiv(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(x, heads, head_dim,
                                                                          position);
    return check_launch("rope_kernel");
}

extern "C" int skv_swiglu_f32(float* gate, const float* up, int n, void* stream) {
    SKV_REQUIRE(gate && up && n > 0, "skv_swiglu_f32: invalid pointers or sizes");
    swiglu_kernel<<<cdiv(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(gate, up, n);
    return check_launch("swiglu_kernel");
}

extern "C" int skv_add_f32(float* target, const float* source, int n, void* stream) {
    SKV_REQUIRE(target && source && n > 0, "skv_add_f32: invalid pointers or sizes");
    add_kernel<<<cdiv(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(target, source, n);
    return check_launch("add_kernel");
}

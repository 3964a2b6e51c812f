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
#include "skv_prompt_gemm.h"

#include <algorithm>
#include <cmath>

namespace skv {

// Loads of 256-thread loops over n elements, 8 per thread in flight: element
// i0 + 256 u of chunk i0 (clamped into range, so every load is issued
// unconditionally; callers ignore the clamped lanes).
constexpr int kChunk = 8;

__device__ __forceinline__ void load_chunk(const float* src, int i0, int n, float (&v)[kChunk]) {
#pragma unroll
    for (int u = 0; u < kChunk; ++u) v[u] = src[min(i0 + 256 * u, n - 1)];
}

// Copies n floats into LDS (256 threads).
__device__ __forceinline__ void stage_to_lds(const float* src, float* dst, int n) {
    for (int i0 = threadIdx.x; i0 < n; i0 += 256 * kChunk) {
        float v[kChunk];
        load_chunk(src, i0, n, v);
#pragma unroll
        for (int u = 0; u < kChunk; ++u)
            if (i0 + 256 * u < n) dst[i0 + 256 * u] = v[u];
    }
}

// 1 / sqrt(mean(x^2) + eps) of n values (256 threads, `red` = 4 floats of
// LDS): thread t sums x[t], x[t + 256], ... in that order with fma, then the
// wavefront and the 4 wavefronts are reduced.  rmsnorm_kernel and the fused
// projections use this same order, so they normalise to the same bits.
template <typename Get>
__device__ __forceinline__ float rms_inverse(Get get, int n, float eps, float* red) {
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) {
        const float v = get(i);
        ss = fmaf(v, v, ss);
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float total = (red[0] + red[1]) + (red[2] + red[3]);
    return 1.0f / sqrtf(total / static_cast<float>(n) + eps);
}

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* __restrict__ in,
                                                      float* __restrict__ out,
                                                      const float* __restrict__ gamma, int n,
                                                      float eps) {
    extern __shared__ float xg_s[];  // [2][n]: the row and gamma
    __shared__ float red[4];
    const int row = blockIdx.x;
    const float* x = in + static_cast<int64_t>(row) * n;
    float* y = out + static_cast<int64_t>(row) * n;
    stage_to_lds(x, xg_s, n);
    stage_to_lds(gamma, xg_s + n, n);
    __syncthreads();
    const float inv = rms_inverse([&](int i) { return xg_s[i]; }, n, eps, red);
    for (int i = threadIdx.x; i < n; i += 256) y[i] = xg_s[i] * inv * xg_s[n + i];
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

// Weight rows are read once per call (streamed): 16-byte loads with the
// non-temporal hint, which keeps them from displacing reused lines in L2.
__device__ __forceinline__ uint4 load_stream16(const char* p) {
    typedef uint32_t u32x4s_t __attribute__((ext_vector_type(4)));
    const u32x4s_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4s_t*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}

// Dot products of x (K floats, LDS or global) with two output-major weight
// rows (byte pointers, 16-byte aligned, K elements each; r1 may repeat r0), by
// one wavefront: 16 bytes per lane per load, fp32 accumulation, then a wave
// reduction.  The first min(NU, K / STEP) loads of each row are issued by the
// constructor, before x is needed (callers stage x meanwhile); the rest follow
// NU at a time.  Each lane accumulates its elements in increasing k whatever
// NU is, so every caller computes a row with exactly the same arithmetic and
// fused and separate projections give the same bits.
// FULL: the caller guarantees K >= STEP, so the constructor issues its loads
// without a branch (a branch around them makes the compiler's wait counts
// after it assume the worst and wait for the weights before anything else).
template <bool BF16W, int NU = kGemvUnroll, bool FULL = false>
struct PairPrefetch {
    static constexpr int EPL = BF16W ? 8 : 4;    // elements per 16-byte load
    static constexpr int STEP = 64 * EPL;        // elements per wave-wide load
    static constexpr int64_t ESZ = BF16W ? 2 : 4;
    const char* rows[2];
    uint4 q[2][NU];
    int npre;                                    // steps issued by the constructor

    __device__ __forceinline__ PairPrefetch(const char* r0, const char* r1, int K, int lane) {
        rows[0] = r0;
        rows[1] = r1;
        npre = min(NU, K / STEP);
        // Every one of the NU loads is issued (steps past npre repeat step
        // npre - 1, in bounds, and are never accumulated), so all of them are
        // in flight together.
        if (FULL || npre > 0) {
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    q[j][u] = load_stream16(rows[j] + (min(u, npre - 1) * STEP + lane * EPL) * ESZ);
        }
    }

    __device__ __forceinline__ void accumulate(const float* xr, int k0, int lane, int n, float (&acc)[2]) const {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            if (u >= n) continue;
            float xv[EPL];
#pragma unroll
            for (int e = 0; e < EPL; ++e) xv[e] = xr[k0 + u * STEP + lane * EPL + e];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float f[EPL];
                widen16<BF16W>(q[j][u], f);
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[j] = fmaf(xv[e], f[e], acc[j]);
            }
        }
    }

    // Rows held whole by the constructor (K == npre * STEP): the dot products
    // with another input, with finish()'s arithmetic; the registers are kept.
    __device__ __forceinline__ void dot_resident(const float* xr, int lane, float& out0, float& out1) const {
        float acc[2] = {0.0f, 0.0f};
        accumulate(xr, 0, lane, npre, acc);
        out0 = wave_sum(acc[0]);
        out1 = wave_sum(acc[1]);
    }

    __device__ __forceinline__ void finish(const float* xr, int K, int lane, float& out0, float& out1) {
        float acc[2] = {0.0f, 0.0f};
        accumulate(xr, 0, lane, npre, acc);
        int k0 = npre * STEP;
        for (; k0 + NU * STEP <= K; k0 += NU * STEP) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int u = 0; u < NU; ++u)
                    q[j][u] = load_stream16(rows[j] + (k0 + u * STEP + lane * EPL) * ESZ);
            accumulate(xr, k0, lane, NU, acc);
        }
        for (int k = k0 + lane * EPL; k + EPL <= K; k += STEP) {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                float f[EPL];
                widen16<BF16W>(load_stream16(rows[j] + k * ESZ), f);
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[j] = fmaf(xr[k + e], f[e], acc[j]);
            }
        }
        for (int k = K - K % EPL + lane; k < K; k += 64)
#pragma unroll
            for (int j = 0; j < 2; ++j)
                acc[j] = fmaf(xr[k], weight_at<BF16W>(rows[j], k), acc[j]);
        out0 = wave_sum(acc[0]);
        out1 = wave_sum(acc[1]);
    }
};

template <bool BF16W>
__device__ __forceinline__ void gemv_pair(const float* xr, const char* r0, const char* r1, int K,
                                          int lane, float& out0, float& out1) {
    PairPrefetch<BF16W> pf(r0, r1, K, lane);
    pf.finish(xr, K, lane, out0, out1);
}

// Output-major weights (stride_k == 1, 16-byte aligned rows): output n is the
// dot product of x with the contiguous row n.  One wavefront per 2 rows
// (gemv_pair: 8 KiB in flight per wavefront); x is staged once per workgroup
// in LDS.  Further rows of x (tokens) read the weights again, from L2.
template <bool BF16W>
__global__ __launch_bounds__(256) void gemv_rows_vec_kernel(const float* __restrict__ x, int rows,
                                                            const void* __restrict__ w,
                                                            int64_t stride_n, int K, int N,
                                                            const float* __restrict__ bias,
                                                            float* __restrict__ y) {
    extern __shared__ float x_s[];               // [rows][K] when it fits
    const int lane = threadIdx.x & 63;
    const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int n0 = min(wave * kGemvRowsPerWave, N - 1);  // waves past N redo row N-1, store nothing
    const int n1 = min(n0 + 1, N - 1);
    const char* wb = static_cast<const char*>(w);
    const int64_t rb = stride_n * (BF16W ? 2 : 4);
    const bool lds_x = static_cast<int64_t>(rows) * K <= kGemvMaxLdsK;
    const int nx = rows * K;
    // Issue order: the first chunk of x, then the weights (see fused_gemv_kernel).
    float xv[kChunk];
    if (lds_x) load_chunk(x, threadIdx.x, nx, xv);
    PairPrefetch<BF16W> pf(wb + n0 * rb, wb + n1 * rb, K, lane);
    if (lds_x) {
#pragma unroll
        for (int u = 0; u < kChunk; ++u)
            if (threadIdx.x + 256 * u < nx) x_s[threadIdx.x + 256 * u] = xv[u];
        if (nx > 256 * kChunk) stage_to_lds(x + 256 * kChunk, x_s + 256 * kChunk, nx - 256 * kChunk);
        __syncthreads();
    }
    if (wave * kGemvRowsPerWave >= N) return;
    for (int r = 0; r < rows; ++r) {
        const float* xr = lds_x ? x_s + static_cast<int64_t>(r) * K : x + static_cast<int64_t>(r) * K;
        float a0, a1;
        if (r == 0) pf.finish(xr, K, lane, a0, a1);
        else gemv_pair<BF16W>(xr, wb + n0 * rb, wb + n1 * rb, K, lane, a0, a1);
        if (lane == 0) {
            y[static_cast<int64_t>(r) * N + n0] = a0 + (bias ? bias[n0] : 0.0f);
            if (n1 != n0) y[static_cast<int64_t>(r) * N + n1] = a1 + (bias ? bias[n1] : 0.0f);
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

// cos and sin of pair `pair` of a head_dim-hd head at `position`: inverse
// frequency 10000^(-2 pair / hd) rounded to float, angle in double.
// cos / sin of the rotation of pair `pair` at `position`: the inverse
// frequency 10000^(-2 pair / hd) in double, rounded to float, the angle in
// double (src/layers/attention.cpp:96-135).  Computed on the host, with the
// same double routines as the reference's CPU path, once per (hd, position),
// and handed to the kernels in their arguments (2 KiB at most): the kernels
// never evaluate double transcendentals.
constexpr int kMaxRopePairs = 256;   // head_dim <= 512
struct RopeTable {
    float cs[2 * kMaxRopePairs];     // [pair][cos, sin]
};

const RopeTable& rope_table(int hd, int position) {
    thread_local RopeTable table;
    thread_local int cached_hd = -1, cached_pos = -1;
    if (hd != cached_hd || position != cached_pos) {
        for (int i = 0; i < hd / 2; ++i) {
            const float inv = static_cast<float>(std::pow(10000.0, -2.0 * i / static_cast<double>(hd)));
            const double angle = static_cast<double>(position) * static_cast<double>(inv);
            table.cs[2 * i] = static_cast<float>(std::cos(angle));
            table.cs[2 * i + 1] = static_cast<float>(std::sin(angle));
        }
        cached_hd = hd;
        cached_pos = position;
    }
    return table;
}

// Inverse frequencies 10000^(-2i/hd) rounded to float, as the reference's
// rope_inv_freq_ (and rope_table above) hold them.
const RopeTable& rope_inv_freq(int hd) {
    thread_local RopeTable table;
    thread_local int cached_hd = -1;
    if (hd != cached_hd) {
        for (int i = 0; i < hd / 2; ++i)
            table.cs[i] = static_cast<float>(std::pow(10000.0, -2.0 * i / static_cast<double>(hd)));
        cached_hd = hd;
    }
    return table;
}

// cos and sin of position * inv (angle in double, rounded to float): the
// values rope_table computes on the host, for kernels that rotate several
// positions.
__device__ __forceinline__ void rope_cos_sin(int position, float inv, float& c, float& s) {
    const double angle = static_cast<double>(position) * static_cast<double>(inv);
    c = static_cast<float>(cos(angle));
    s = static_cast<float>(sin(angle));
}

__device__ __forceinline__ float swiglu_of(float g, float u) {
    const float sig = g >= 0.0f ? 1.0f / (1.0f + expf(-g)) : expf(g) / (1.0f + expf(g));
    return g * sig * u;
}

// One rotation, with the rounding spelled out (one product, one fused
// multiply-add per output) so that every kernel that rotates gives the same
// bits whatever the compiler would contract.
__device__ __forceinline__ void rotate_pair(float& a, float& b, float c, float s) {
    const float a0 = a, b0 = b;
    a = fmaf(a0, c, -(b0 * s));
    b = fmaf(a0, s, b0 * c);
}

__global__ __launch_bounds__(256) void rope_kernel(float* __restrict__ x, int heads, int hd,
                                                   RopeTable rt) {
    const int half = hd / 2;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= heads * half) return;
    const int h = i / half, pair = i - h * half;
    const float c = rt.cs[2 * pair], s = rt.cs[2 * pair + 1];
    float* p = x + static_cast<int64_t>(h) * hd;
    float a = p[pair], b = p[pair + half];
    rotate_pair(a, b, c, s);
    p[pair] = a;
    p[pair + half] = b;
}

// Rows of `heads` head vectors, row r at position first + r (prompt prefill).
__global__ __launch_bounds__(256) void rope_rows_kernel(float* __restrict__ x, int rows, int heads, int hd,
                                                        int first, RopeTable inv) {
    const int half = hd / 2;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(rows) * heads * half) return;
    const int r = static_cast<int>(i / (heads * half));
    const int rem = static_cast<int>(i - static_cast<int64_t>(r) * heads * half);
    const int h = rem / half, pair = rem - h * half;
    float c, s;
    rope_cos_sin(first + r, inv.cs[pair], c, s);
    float* p = x + (static_cast<int64_t>(r) * heads + h) * hd;
    float a = p[pair], b = p[pair + half];
    rotate_pair(a, b, c, s);
    p[pair] = a;
    p[pair + half] = b;
}

__global__ __launch_bounds__(256) void swiglu_kernel(float* __restrict__ gate,
                                                     const float* __restrict__ up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    gate[i] = swiglu_of(gate[i], up[i]);
}

__global__ __launch_bounds__(256) void add_kernel(float* __restrict__ t, const float* __restrict__ s,
                                                  int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) t[i] += s[i];
}

// ---------------------------------------------------------------------------
// Fused projections of the decode step (single token).  Each workgroup stages
// the input in LDS, RMS-normalised on the way when gamma is given (the same
// reduction and rounding as rmsnorm_kernel), and every wavefront computes two
// output rows with gemv_pair; the epilogue then applies what the separate
// kernels would, to the same values:
//   QKV       q, k, v projections of the normalised input; with position >= 0
//             a wavefront of q or k takes rows (i, i + hd/2) of one head and
//             rotates them (rope_kernel's arithmetic) before storing;
//   GATE_UP   gate row n and up row n of the normalised input -> swiglu;
//   RESIDUAL  y = W x + residual (o_proj and down_proj with their residual add);
//   LINEAR    y = W x (+ bias): skv_linear_f32 of one row (the same rows and
//             arithmetic as gemv_rows_vec_kernel, staged without branches).
// Bias, when present, is added before the rotation, as Linear::forward_into
// does before the RoPE step.
// ---------------------------------------------------------------------------
enum FusedMode : int { FUSED_QKV = 0, FUSED_GATE_UP = 1, FUSED_RESIDUAL = 2, FUSED_LINEAR = 3 };

struct FusedGemv {
    const float* x;
    const float* gamma;       // nullptr: no normalisation
    float eps;
    int K;
    const void* w[3];
    int64_t row_bytes[3];     // byte stride between output rows
    const float* bias[3];
    int n[3];                 // output rows per matrix
    float* y[3];
    int head_dim;             // QKV
    int position;             // QKV: RoPE position, < 0 = none
    const float* residual;    // RESIDUAL
    RopeTable rope;           // QKV with position >= 0: cos/sin of `position` (one token),
                              // or the inverse frequencies (fused_gemv_rows_kernel)
    int rows;                 // tokens (fused_gemv_rows_kernel; x, y, residual row-major)
    // QKV of one token at a position held in device memory (launches captured
    // once and replayed per token): the position is *position_at, clamped to
    // [0, rope_positions), and its cos/sin pairs are read from rope_dev
    // ([rope_positions][head_dim / 2][cos, sin], rope_table's values).
    const int32_t* position_at;
    const float* rope_dev;
    int rope_positions;
};

// The two rows of work item `item` (one wavefront): matrix ma row ra and
// matrix mb row rb; an item past the end computes a valid row (live = false)
// and stores nothing.  QKV with RoPE pairs rows (i, i + hd/2) of one head.
struct FusedRowPair {
    int ma, mb, ra, rb, seg, p;
    bool live, rope;
};

// `item` must be wave-uniform (the callers pass the wave index through
// readfirstlane), so the matrix choice and the row pointers are scalar values
// and the weight addresses never wait on a vector load of the arguments.
// Kernel-argument arrays are indexed only with constants and the element
// chosen by compares: an index computed at run time makes the compiler read
// the argument buffer at that point, one dependent scalar round trip each
// (the buffer is cold in the scalar cache at every launch).
template <typename T>
__device__ __forceinline__ T pick3(const T (&a)[3], int i) {
    return i == 0 ? a[0] : (i == 1 ? a[1] : a[2]);
}

template <int MODE>
__device__ __forceinline__ FusedRowPair fused_row_pair(const FusedGemv& f, int item) {
    FusedRowPair r{0, 0, 0, 0, 0, item, true, false};
    if constexpr (MODE == FUSED_QKV) {
        const int h0 = f.n[0] / 2, h01 = h0 + f.n[1] / 2, h012 = h01 + f.n[2] / 2;
        r.live = item < h012;
        const int it = r.live ? item : h012 - 1;   // past the end: the last pair of v
        r.seg = (it >= h0 ? 1 : 0) + (it >= h01 ? 1 : 0);
        r.p = it - (r.seg == 0 ? 0 : (r.seg == 1 ? h0 : h01));
        const int hd = f.head_dim, half = hd / 2;
        r.rope = r.seg < 2 && f.position >= 0;
        r.ma = r.mb = r.seg;
        r.ra = r.rope ? (r.p / half) * hd + r.p % half : 2 * r.p;
        r.rb = r.rope ? r.ra + half : 2 * r.p + 1;
    } else if constexpr (MODE == FUSED_GATE_UP) {
        r.live = item < f.n[0];
        r.ra = r.rb = min(item, f.n[0] - 1);
        r.mb = 1;
    } else {
        r.live = 2 * item < f.n[0];
        r.ra = min(2 * item, f.n[0] - 1);
        r.rb = min(r.ra + 1, f.n[0] - 1);
    }
    return r;
}

__device__ __forceinline__ const char* fused_row_ptr(const FusedGemv& f, int m, int r) {
    return static_cast<const char*>(pick3(f.w, m)) + static_cast<int64_t>(r) * pick3(f.row_bytes, m);
}

template <bool BF16W, int MODE, int NU, int XU, bool NORM, bool DEVPOS = false>
__global__ __launch_bounds__(256) void fused_gemv_kernel(FusedGemv f) {
    extern __shared__ float x_s[];  // [256 XU] input, normalised when NORM (padding past K unused)
    __shared__ float red[4];
    const int t = threadIdx.x, lane = t & 63;
    const int K = f.K;
    const FusedRowPair rp = fused_row_pair<MODE>(f, blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(t >> 6));
    const int ma = rp.ma, mb = rp.mb, ra = rp.ra, rb = rp.rb, seg = rp.seg, p = rp.p;
    const bool live = rp.live, rope = rp.rope;
    // Loads in issue order: all of x (and gamma), XU per thread (K <= 256 XU),
    // the epilogue's operands, then this wavefront's weights.  Everything up to
    // the dot products is straight-line code on registers and unconditional
    // LDS stores (elements past K land in padding), so the waits before it
    // count only the x and gamma loads and the weights stay in flight through
    // the normalisation.  The epilogue operands (bias, residual, RoPE
    // cos/sin) are requested here, before the barrier (a memory fence the
    // compiler does not move loads across), not after the dot products.
    float xv[XU], gv[XU];
#pragma unroll
    for (int u = 0; u < XU; ++u) xv[u] = f.x[min(t + 256 * u, K - 1)];
    if constexpr (NORM)
#pragma unroll
        for (int u = 0; u < XU; ++u) gv[u] = f.gamma[min(t + 256 * u, K - 1)];
    const float* bias_a = pick3(f.bias, ma);
    const float* bias_b = pick3(f.bias, mb);
    const float ba = bias_a != nullptr ? bias_a[ra] : 0.0f;
    const float bb = bias_b != nullptr ? bias_b[rb] : 0.0f;
    float ra_res = 0.0f, rb_res = 0.0f;
    if constexpr (MODE == FUSED_RESIDUAL) {
        ra_res = f.residual[ra];
        rb_res = f.residual[rb];
    }
    float rope_c = 1.0f, rope_s = 0.0f;
    if constexpr (MODE == FUSED_QKV) {
        const int pair = rope ? p % (f.head_dim / 2) : 0;
        if constexpr (DEVPOS) {
            const int pos = min(max(*f.position_at, 0), f.rope_positions - 1);
            const float* cs = f.rope_dev + static_cast<int64_t>(pos) * f.head_dim + 2 * pair;
            rope_c = cs[0];
            rope_s = cs[1];
        } else {
            rope_c = f.rope.cs[2 * pair];
            rope_s = f.rope.cs[2 * pair + 1];
        }
    }
    float* const y = pick3(f.y, seg);
    __builtin_amdgcn_sched_barrier(0);  // keep the weight loads after x's
    PairPrefetch<BF16W, NU, true> pf(fused_row_ptr(f, ma, ra), fused_row_ptr(f, mb, rb), K, lane);
    if constexpr (NORM) {
        // rms_inverse's arithmetic on the registers: thread t sums x[t],
        // x[t + 256], ... (below K) in that order with fma, then the wave and
        // the 4 wavefronts.
        float ss = 0.0f;
#pragma unroll
        for (int u = 0; u < XU; ++u) ss = t + 256 * u < K ? fmaf(xv[u], xv[u], ss) : ss;
        ss = wave_sum(ss);
        if (lane == 0) red[t >> 6] = ss;
        __syncthreads();
        const float total = (red[0] + red[1]) + (red[2] + red[3]);
        const float inv = 1.0f / sqrtf(total / static_cast<float>(K) + f.eps);
#pragma unroll
        for (int u = 0; u < XU; ++u) x_s[t + 256 * u] = xv[u] * inv * gv[u];
    } else {
#pragma unroll
        for (int u = 0; u < XU; ++u) x_s[t + 256 * u] = xv[u];
    }
    __syncthreads();
    if (!live) return;
    float a, b;
    pf.finish(x_s, K, lane, a, b);

    if constexpr (MODE == FUSED_QKV) {
        if (lane == 0) {
            a += ba;
            b += bb;
            if (rope) rotate_pair(a, b, rope_c, rope_s);
            y[ra] = a;
            y[rb] = b;
        }
    } else if constexpr (MODE == FUSED_GATE_UP) {
        if (lane == 0) y[ra] = swiglu_of(a + ba, b + bb);
    } else if constexpr (MODE == FUSED_RESIDUAL) {
        if (lane == 0) {
            y[ra] = (a + ba) + ra_res;
            if (rb != ra) y[rb] = (b + bb) + rb_res;
        }
    } else {
        if (lane == 0) {
            y[ra] = a + ba;
            if (rb != ra) y[rb] = b + bb;
        }
    }
}

// Fused projections of `rows` tokens (prompt prefill), inputs already
// normalised (rmsnorm_kernel on the host side of the call).  Each wavefront
// keeps its two weight rows whole in registers (K = steps * STEP, steps <=
// NU; the host checks), so the weights are read from HBM once for all
// tokens.  Tokens go in tiles of 16: for each wave-wide step of k the
// workgroup stages that step of the 16 inputs in LDS (two buffers, the next
// step loaded while this one is computed, one barrier per step) and every
// wavefront accumulates 16 x 2 dot products.  The per-token accumulation
// order is PairPrefetch's and the final reduction wave_sum's, so each token's
// outputs have the bits fused_gemv_kernel gives for that token alone; RoPE
// rotates token m at position + m with rope_cos_sin (the host table's values).
typedef float f32x4_t __attribute__((ext_vector_type(4)));
constexpr int kRowsTile = 16;

template <bool BF16W, int MODE, int NU, int WPG>
__global__ __launch_bounds__(64 * WPG) void fused_gemv_rows_kernel(FusedGemv f) {
    using PF = PairPrefetch<BF16W, NU, true>;  // K is a nonzero multiple of STEP
    constexpr int STEP = PF::STEP, EPL = PF::EPL, T = kRowsTile;
    constexpr int Q4 = STEP / 4;                  // float4 per staged input row
    constexpr int LPT = T * Q4 / (64 * WPG);      // float4 staged per thread per step
    static_assert(LPT * 64 * WPG == T * Q4, "step staging");
    extern __shared__ f32x4_t xs4[];              // [2][T][Q4]
    const int t = threadIdx.x, lane = t & 63;
    const int K = f.K, steps = K / STEP, rows = f.rows;
    const int ntiles = cdiv(rows, T);
    auto bias_of = [&](int m, int r) {
        const float* bp = pick3(f.bias, m);
        return bp != nullptr ? bp[r] : 0.0f;
    };
    const FusedRowPair rp = fused_row_pair<MODE>(f, blockIdx.x * WPG + __builtin_amdgcn_readfirstlane(t >> 6));
    float* const y_seg = pick3(f.y, rp.seg);
    const int n_seg = pick3(f.n, rp.seg);
    f32x4_t st[LPT];
    auto load_step = [&](int tile, int c) __attribute__((always_inline)) {  // rows past the end repeat the last row
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int idx = t + i * 64 * WPG, m = idx / Q4;
            const int64_t row = min(tile * T + m, rows - 1);
            st[i] = reinterpret_cast<const f32x4_t*>(f.x + row * K + c * STEP)[idx - m * Q4];
        }
    };
    // Issue order: the first input step, then the weights; the empty asm
    // reads every weight register here, so the compiler keeps the whole rows
    // resident instead of sinking the loads to their uses (one wait for all).
    load_step(0, 0);
    const PF pf(fused_row_ptr(f, rp.ma, rp.ra), fused_row_ptr(f, rp.mb, rp.rb), K, lane);
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int u = 0; u < NU; ++u)
            asm volatile("" ::"v"(pf.q[j][u].x), "v"(pf.q[j][u].y), "v"(pf.q[j][u].z), "v"(pf.q[j][u].w));
    int g = 0;
    for (int tile = 0; tile < ntiles; ++tile) {
        float acc[T][2];
#pragma unroll
        for (int m = 0; m < T; ++m) acc[m][0] = acc[m][1] = 0.0f;
#pragma unroll
        for (int c = 0; c < NU; ++c) {
            if (c >= steps) continue;  // (not break: the loop must unroll, pf.q[.][c] stays in registers)
            f32x4_t* buf = xs4 + (g & 1) * T * Q4;
#pragma unroll
            for (int i = 0; i < LPT; ++i) buf[t + i * 64 * WPG] = st[i];
            __syncthreads();
            // Next step (the next tile's first after the last; past the end,
            // this tile's last again: every load is issued unconditionally).
            int nt = tile, nc = c + 1;
            if (nc == steps) nt = tile + 1, nc = 0;
            if (nt == ntiles) nt = ntiles - 1, nc = steps - 1;
            load_step(nt, nc);
            float w[2][EPL];
            widen16<BF16W>(pf.q[0][c], w[0]);
            widen16<BF16W>(pf.q[1][c], w[1]);
#pragma unroll
            for (int m = 0; m < T; ++m) {
                float xv[EPL];
#pragma unroll
                for (int q = 0; q < EPL / 4; ++q) {
                    const f32x4_t x4 = buf[m * Q4 + lane * (EPL / 4) + q];
                    xv[4 * q + 0] = x4[0];
                    xv[4 * q + 1] = x4[1];
                    xv[4 * q + 2] = x4[2];
                    xv[4 * q + 3] = x4[3];
                }
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[m][j] = fmaf(xv[e], w[j][e], acc[m][j]);
            }
            ++g;
        }
        // Lane (r, .) = (lane >> 3, .) ends with tokens 2r and 2r + 1.
        float v[2 * T];
#pragma unroll
        for (int m = 0; m < T; ++m) {
            v[2 * m] = acc[m][0];
            v[2 * m + 1] = acc[m][1];
        }
        wave_sum_scatter<2 * T>(v);
        if (!rp.live || (lane & 7) != 0) continue;
        auto emit = [&](int m, float a, float b) __attribute__((always_inline)) {
            if (m >= rows) return;
            if constexpr (MODE == FUSED_QKV) {
                a += bias_of(rp.seg, rp.ra);
                b += bias_of(rp.seg, rp.rb);
                if (rp.rope) {
                    float cs, sn;
                    rope_cos_sin(f.position + m, f.rope.cs[rp.p % (f.head_dim / 2)], cs, sn);
                    rotate_pair(a, b, cs, sn);
                }
                float* y = y_seg + static_cast<int64_t>(m) * n_seg;
                y[rp.ra] = a;
                y[rp.rb] = b;
            } else if constexpr (MODE == FUSED_GATE_UP) {
                f.y[0][static_cast<int64_t>(m) * f.n[0] + rp.ra] =
                    swiglu_of(a + bias_of(0, rp.ra), b + bias_of(1, rp.ra));
            } else {
                const int64_t row = static_cast<int64_t>(m) * f.n[0];
                f.y[0][row + rp.ra] = (a + bias_of(0, rp.ra)) + f.residual[row + rp.ra];
                if (rp.rb != rp.ra) f.y[0][row + rp.rb] = (b + bias_of(0, rp.rb)) + f.residual[row + rp.rb];
            }
        };
        emit(tile * T + 2 * (lane >> 3), v[0], v[1]);
        emit(tile * T + 2 * (lane >> 3) + 1, v[2], v[3]);
    }
}

// Common checks of the fused entry points: output-major rows, 16-byte aligned,
// input staged in LDS.
bool fused_rows_ok(const void* w, int64_t stride_k, int64_t stride_n, int K, int esz) {
    const int step = esz == 2 ? 512 : 256;  // one wave-wide load of a row
    return w != nullptr && stride_k == 1 && stride_n >= K && aligned16(w) &&
           (stride_n * esz) % 16 == 0 && K >= step && K <= kGemvMaxLdsK;
}

template <int MODE>
int launch_fused(const FusedGemv& f, bool bf16, int items, hipStream_t s) {
    const unsigned grid = static_cast<unsigned>(cdiv(items, 4));
    // The whole input is preloaded (XU elements per thread, staged into
    // 256 XU floats of LDS) and up to 12 wave-wide steps of each weight row are
    // requested at once.
    const bool norm = f.gamma != nullptr;
    auto go = [&](auto kern, int xu) { kern<<<grid, 256, sizeof(float) * 256 * static_cast<size_t>(xu), s>>>(f); };
    // A device-held position (QKV only) selects the DEVPOS instance.
    constexpr bool QKV = MODE == FUSED_QKV;
    const bool devpos = QKV && f.position_at != nullptr;
#define SKV_FUSED(NU_B, NU_F, XU_)                                                                       \
    {                                                                                                    \
        if (devpos) {                                                                                    \
            if (bf16 && norm) go(fused_gemv_kernel<true, MODE, NU_B, XU_, QKV, QKV>, XU_);               \
            else if (bf16) go(fused_gemv_kernel<true, MODE, NU_B, XU_, false, QKV>, XU_);                \
            else if (norm) go(fused_gemv_kernel<false, MODE, NU_F, XU_, QKV, QKV>, XU_);                 \
            else go(fused_gemv_kernel<false, MODE, NU_F, XU_, false, QKV>, XU_);                         \
        } else if (bf16 && norm) go(fused_gemv_kernel<true, MODE, NU_B, XU_, MODE <= FUSED_GATE_UP>, XU_);  \
        else if (bf16) go(fused_gemv_kernel<true, MODE, NU_B, XU_, false>, XU_);                         \
        else if (norm) go(fused_gemv_kernel<false, MODE, NU_F, XU_, MODE <= FUSED_GATE_UP>, XU_);        \
        else go(fused_gemv_kernel<false, MODE, NU_F, XU_, false>, XU_);                                  \
    }
    if (f.K <= 2048) SKV_FUSED(4, 8, 8)
    else if (f.K <= 4096) SKV_FUSED(8, 12, 16)
    else if (f.K <= 6144) SKV_FUSED(12, 12, 24)
    else SKV_FUSED(12, 12, 32)
#undef SKV_FUSED
    return check_launch("fused_gemv_kernel");
}

bool rows_supported(bool bf16, int K) {
    return bf16 ? K % 512 == 0 && K <= 6144 : K % 256 == 0 && K <= 2048;
}

// fused_gemv_rows_kernel needs every weight row whole in registers: K a
// multiple of the wave-wide step and at most 12 steps (bf16: K <= 6,144,
// fp32: K <= 2,048).  Otherwise SKV_ERR_UNSUPPORTED (nothing launched).
// The wide gate/up launch uses 8-wavefront workgroups (each staged input
// serves 16 rows), the narrower projections 4 (more workgroups).
template <int MODE>
int launch_fused_rows(const FusedGemv& f, bool bf16, int items, hipStream_t s) {
    constexpr int WPG = MODE == FUSED_GATE_UP ? 8 : 4;
    const unsigned grid = static_cast<unsigned>(cdiv(items, WPG));
    auto go = [&](auto kern, int step) {
        const size_t lds = 2 * sizeof(float) * static_cast<size_t>(kRowsTile) * step;
        const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                                    static_cast<int>(lds));
        if (attr != hipSuccess) return set_error(SKV_ERR_HIP, "fused_gemv_rows_kernel: %s", hipGetErrorString(attr));
        kern<<<grid, 64 * WPG, lds, s>>>(f);
        return check_launch("fused_gemv_rows_kernel");
    };
    if (bf16 && f.K % 512 == 0) {
        if (f.K <= 2048) return go(fused_gemv_rows_kernel<true, MODE, 4, WPG>, 512);
        if (f.K <= 4096) return go(fused_gemv_rows_kernel<true, MODE, 8, WPG>, 512);
        if (f.K <= 6144) return go(fused_gemv_rows_kernel<true, MODE, 12, WPG>, 512);
    }
    if (!bf16 && f.K % 256 == 0 && f.K <= 2048) return go(fused_gemv_rows_kernel<false, MODE, 8, WPG>, 256);
    return set_error(SKV_ERR_UNSUPPORTED,
                     "fused projections of several tokens need K a multiple of %d and at most %d", bf16 ? 512 : 256,
                     bf16 ? 6144 : 2048);
}

// ---------------------------------------------------------------------------
// Matrix-core projections of a block of tokens (long prompts).  Each input
// value v (the rmsnorm_kernel output when gamma is given) is split into bf16
// parts hi = bf16(v) and lo = bf16(v - hi), so that W v = W hi + W lo on
// v_mfma_f32_16x16x32_bf16 with fp32 accumulation: every product of a bf16
// weight with a part is exact and v keeps ~16 significant bits, close to the
// fp32 dot products of the one-token kernels (not bit-identical to them: the
// summation order differs).
// ---------------------------------------------------------------------------
typedef __bf16 mm_bf16x8_t __attribute__((ext_vector_type(8)));
typedef uint32_t mm_u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMmTokens = 64;                      // tokens per workgroup (4 column tiles of 16)
constexpr int kMmWaves = 4;                        // wavefronts per workgroup, one feature group each
constexpr int kMmStageK = 64;                      // k per LDS stage (two 32-wide MFMA steps)
constexpr int kMmRowBytes = kMmStageK * 2 + 16;    // one token's stage in LDS (bf16, padded)
constexpr int kMmRing = 2;                         // stages of operands in flight

struct MmArgs {
    FusedGemv f;
    int groups;                 // 32-feature groups
    int token_tiles;            // cdiv(rows, kMmTokens)
};

// Feature group `g` (32 outputs as two 16-row tiles) of a projection:
// matrix, first row of each tile, and whether the pair (tile 0 row r, tile 1
// row r) is rotated together.  QKV with RoPE pairs rows (r, r + hd/2) of one
// head (hd a multiple of 32); GATE_UP takes rows r of gate and of up; the
// others 32 consecutive rows.
struct MmGroup {
    int m, r0, r1;
    bool rope;
};

template <int MODE>
__device__ __forceinline__ MmGroup mm_group(const FusedGemv& f, int g) {
    MmGroup q{0, 0, 0, false};
    if constexpr (MODE == FUSED_QKV) {
        while (q.m < 2 && g >= f.n[q.m] / 32) g -= f.n[q.m] / 32, ++q.m;
        q.rope = q.m < 2 && f.position >= 0;
        if (q.rope) {
            const int half = f.head_dim / 2, per_head = half / 16;
            q.r0 = (g / per_head) * f.head_dim + (g % per_head) * 16;
            q.r1 = q.r0 + half;
        } else {
            q.r0 = 32 * g;
            q.r1 = q.r0 + 16;
        }
    } else if constexpr (MODE == FUSED_GATE_UP) {
        q.r0 = q.r1 = 16 * g;
    } else {
        q.r0 = 32 * g;
        q.r1 = q.r0 + 16;
    }
    return q;
}

// One workgroup = kMmWaves / KS feature groups x kMmTokens tokens, K split
// into KS parts (KS = 2 when the grid would be too small to fill the chip):
// wavefront w computes group w % (kMmWaves / KS) over part w / (kMmWaves / KS)
// and the parts are summed through LDS in a fixed order.  The inputs go
// through LDS in stages of kMmStageK per part: each thread loads 16
// consecutive fp32 of one token per part, splits them into hi and lo parts
// and stores them (two LDS buffers, one barrier per stage); a wavefront reads
// them in the MFMA B layout (lane (t, j): token t of a column tile, k chunk
// 8j..8j+7) and its weight rows straight from global memory in the A layout
// (row t of a tile, the same chunk).  Inputs and weights are requested
// kMmRing stages ahead, the inputs of a stage after its weights, so that each
// wait in issue order covers exactly the stage it needs.  Output lane layout:
// acc[a][c][i] = feature (tile a) 4j + i, token 16c + t.
constexpr int kMmPartBytes = 2 * kMmTokens * kMmRowBytes;   // hi + lo of one part's stage

template <int MODE, int KS>
__global__ __launch_bounds__(64 * kMmWaves) void proj_mm_kernel(MmArgs args) {
    constexpr int GPW = kMmWaves / KS;   // feature groups per workgroup
    const FusedGemv& f = args.f;
    extern __shared__ __align__(16) unsigned char xs[];   // [buffer][part][hi, lo][token]
    auto xs_at = [&](int buf, int part, int half) { return xs + ((buf * KS + part) * 2 + half) * (kMmPartBytes / 2); };
    const int tid = threadIdx.x, lane = tid & 63, t = lane & 15, j = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int part = w / GPW;
    // Workgroups are dealt to the 8 XCDs round-robin: the token tiles of one
    // feature tile go to the same XCD, one after another, so its weight rows
    // are read from HBM once and then from that XCD's L2.
    const int id = blockIdx.x, xcd = id & 7, local = id >> 3;
    const int ftile = (local / args.token_tiles) * 8 + xcd;
    const int tile = local % args.token_tiles;
    if (ftile * GPW >= args.groups) return;      // the whole workgroup, before any barrier
    const int g = ftile * GPW + w % GPW;
    const bool live = g < args.groups;           // a wave past the last group stores nothing
    const MmGroup grp = mm_group<MODE>(f, min(g, args.groups - 1));
    const int K = f.K, rows = f.rows, nst = K / kMmStageK / KS;   // stages per part
    const int tok0 = tile * kMmTokens;

    // Staging: thread -> token tid / 4, k (tid % 4) * 16 .. + 15 of a stage.
    const int st_tok = tid >> 2, st_k = (tid & 3) * 16;
    const float* xrow = f.x + static_cast<int64_t>(min(tok0 + st_tok, rows - 1)) * K + st_k;
    // Weight rows of this wavefront's two tiles.
    const int mb = MODE == FUSED_GATE_UP ? 1 : grp.m;
    const char* wa = static_cast<const char*>(f.w[grp.m]) + static_cast<int64_t>(grp.r0 + t) * f.row_bytes[grp.m];
    const char* wb = static_cast<const char*>(f.w[mb]) + static_cast<int64_t>(grp.r1 + t) * f.row_bytes[mb];

    struct Stage {
        mm_u32x4_t wop[2][2];   // [k-step][tile] weight operands of this wavefront's part
        f32x4_t x[KS][4];       // this thread's 16 staged inputs of every part
    };
    auto load = [&](int s, Stage& o) __attribute__((always_inline)) {
        s = min(s, nst - 1);    // past the end: the last stage again (in bounds, unused)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            const int k = (part * nst + s) * kMmStageK + ks * 32 + 8 * j;
            o.wop[ks][0] = *reinterpret_cast<const mm_u32x4_t*>(wa + 2 * k);
            o.wop[ks][1] = *reinterpret_cast<const mm_u32x4_t*>(wb + 2 * k);
        }
#pragma unroll
        for (int q = 0; q < KS; ++q)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                o.x[q][r] = reinterpret_cast<const f32x4_t*>(xrow + (q * nst + s) * kMmStageK)[r];
    };
    auto stage_inputs = [&](int buf, const Stage& o) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < KS; ++q) {
            // hi = bf16(v) for a pair in one conversion; its two values back as
            // floats with a byte permute (low half to the top) and a mask; lo =
            // bf16 of the exact remainder v - hi, one conversion per pair.
            typedef __bf16 mm_bf16x2_t __attribute__((ext_vector_type(2)));
            uint32_t hw[8], lw[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float v0 = o.x[q][e >> 1][2 * (e & 1)], v1 = o.x[q][e >> 1][2 * (e & 1) + 1];
                const mm_bf16x2_t h = {static_cast<__bf16>(v0), static_cast<__bf16>(v1)};
                hw[e] = __builtin_bit_cast(uint32_t, h);
                const float h0 = __uint_as_float(__builtin_amdgcn_perm(hw[e], hw[e], 0x01000c0cu));
                const float h1 = __uint_as_float(hw[e] & 0xFFFF0000u);
                const mm_bf16x2_t l = {static_cast<__bf16>(v0 - h0), static_cast<__bf16>(v1 - h1)};
                lw[e] = __builtin_bit_cast(uint32_t, l);
            }
            unsigned char* dh = xs_at(buf, q, 0) + st_tok * kMmRowBytes + st_k * 2;
            unsigned char* dl = xs_at(buf, q, 1) + st_tok * kMmRowBytes + st_k * 2;
            reinterpret_cast<mm_u32x4_t*>(dh)[0] = mm_u32x4_t{hw[0], hw[1], hw[2], hw[3]};
            reinterpret_cast<mm_u32x4_t*>(dh)[1] = mm_u32x4_t{hw[4], hw[5], hw[6], hw[7]};
            reinterpret_cast<mm_u32x4_t*>(dl)[0] = mm_u32x4_t{lw[0], lw[1], lw[2], lw[3]};
            reinterpret_cast<mm_u32x4_t*>(dl)[1] = mm_u32x4_t{lw[4], lw[5], lw[6], lw[7]};
        }
    };

    f32x4_t acc[2][4];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[a][c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int buf, const Stage& o) __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            mm_u32x4_t bh[4], bl[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int off = (16 * c + t) * kMmRowBytes + (ks * 32 + 8 * j) * 2;
                bh[c] = *reinterpret_cast<const mm_u32x4_t*>(xs_at(buf, part, 0) + off);
                bl[c] = *reinterpret_cast<const mm_u32x4_t*>(xs_at(buf, part, 1) + off);
            }
            // All hi products, then all lo products: no MFMA waits on the one
            // issued just before it.
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(mm_bf16x8_t, o.wop[ks][a]), __builtin_bit_cast(mm_bf16x8_t, bh[c]),
                        acc[a][c], 0, 0, 0);
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[a][c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        __builtin_bit_cast(mm_bf16x8_t, o.wop[ks][a]), __builtin_bit_cast(mm_bf16x8_t, bl[c]),
                        acc[a][c], 0, 0, 0);
        }
    };

    // Ring: slot u holds stage s0 + u (weights for the compute of that stage,
    // inputs for its staging one stage earlier).  Stage 0's inputs are staged
    // before the loop; the loop computes stage s, then stages s + 1.
    Stage ring[kMmRing];
#pragma unroll
    for (int u = 0; u < kMmRing; ++u) load(u, ring[u]);
    stage_inputs(0, ring[0]);
    __syncthreads();
    for (int s0 = 0; s0 < nst; s0 += kMmRing) {   // nst is a multiple of kMmRing
#pragma unroll
        for (int u = 0; u < kMmRing; ++u) {
            const int s = s0 + u;
            compute(s & 1, ring[u]);
            load(s + kMmRing, ring[u]);
            __builtin_amdgcn_sched_barrier(0);   // issue order kept: the loads stay kMmRing stages ahead
            stage_inputs((s + 1) & 1, ring[(u + 1) % kMmRing]);
            __syncthreads();
        }
    }
    if constexpr (KS == 2) {
        // Part 1's sums into LDS (the staging buffers are idle after the
        // last barrier), then part 0 adds them: part 0 + part 1.
        f32x4_t* red = reinterpret_cast<f32x4_t*>(xs) + (w % GPW) * 8 * 64;
        if (part == 1) {
#pragma unroll
            for (int a = 0; a < 2; ++a)
#pragma unroll
                for (int c = 0; c < 4; ++c) red[(4 * a + c) * 64 + lane] = acc[a][c];
        }
        __syncthreads();
        if (part == 1) return;
#pragma unroll
        for (int a = 0; a < 2; ++a)
#pragma unroll
            for (int c = 0; c < 4; ++c) acc[a][c] += red[(4 * a + c) * 64 + lane];
    }
    if (!live) return;

    auto bias4 = [&](int m, int r) {
        const float* b = f.bias[m];
        return b != nullptr ? f32x4_t{b[r], b[r + 1], b[r + 2], b[r + 3]} : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    };
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const int tok = tok0 + 16 * c + t;
        if (tok >= rows) continue;
        const int ra = grp.r0 + 4 * j, rb = grp.r1 + 4 * j;
        if constexpr (MODE == FUSED_QKV) {
            f32x4_t ya = acc[0][c] + bias4(grp.m, ra), yb = acc[1][c] + bias4(grp.m, rb);
            if (grp.rope) {
                const int half = f.head_dim / 2;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float cs, sn, va = ya[i], vb = yb[i];
                    rope_cos_sin(f.position + tok, f.rope.cs[(ra + i) % f.head_dim % half], cs, sn);
                    rotate_pair(va, vb, cs, sn);
                    ya[i] = va;
                    yb[i] = vb;
                }
            }
            float* y = f.y[grp.m] + static_cast<int64_t>(tok) * f.n[grp.m];
            *reinterpret_cast<f32x4_t*>(y + ra) = ya;
            *reinterpret_cast<f32x4_t*>(y + rb) = yb;
        } else if constexpr (MODE == FUSED_GATE_UP) {
            const f32x4_t gv = acc[0][c] + bias4(0, ra), uv = acc[1][c] + bias4(1, ra);
            const f32x4_t act = {swiglu_of(gv[0], uv[0]), swiglu_of(gv[1], uv[1]), swiglu_of(gv[2], uv[2]),
                                 swiglu_of(gv[3], uv[3])};
            *reinterpret_cast<f32x4_t*>(f.y[0] + static_cast<int64_t>(tok) * f.n[0] + ra) = act;
        } else {
            const int64_t row = static_cast<int64_t>(tok) * f.n[0];
            const f32x4_t res_a = *reinterpret_cast<const f32x4_t*>(f.residual + row + ra);
            const f32x4_t res_b = *reinterpret_cast<const f32x4_t*>(f.residual + row + rb);
            *reinterpret_cast<f32x4_t*>(f.y[0] + row + ra) = (acc[0][c] + bias4(0, ra)) + res_a;
            *reinterpret_cast<f32x4_t*>(f.y[0] + row + rb) = (acc[1][c] + bias4(0, rb)) + res_b;
        }
    }
}

// Shapes the matrix-core projections take: bf16 weights in 16-byte aligned
// output-major rows, K a multiple of 128 (stages of 64 in pairs), every
// matrix's output count a multiple of 32 (16 for gate/up), a 16-byte aligned
// input, and for RoPE head_dim a multiple of 32.
bool mm_supported(const FusedGemv& f, int nmat, int esz, int64_t stride_k) {
    if (esz != 2 || stride_k != 1 || f.K < 128 || f.K % 128 != 0 || !aligned16(f.x)) return false;
    for (int m = 0; m < nmat; ++m)
        if (f.w[m] == nullptr || !aligned16(f.w[m]) || f.row_bytes[m] % 16 != 0 || f.row_bytes[m] < 2 * f.K ||
            f.n[m] % 16 != 0 || (nmat != 2 && f.n[m] % 32 != 0))
            return false;
    return true;
}

// Launches proj_mm_kernel over `groups` feature groups (f.x already
// normalised when the projection normalises).
// K is split in two (twice the workgroups, half the stages each) when the
// whole-K grid would give fewer than 256 workgroups and K is a multiple of 256.
template <int MODE>
int launch_mm(const FusedGemv& f, int groups, hipStream_t s) {
    MmArgs a{f, groups, cdiv(f.rows, kMmTokens)};
    auto grid_of = [&](int gpw) { return static_cast<int64_t>(cdiv(cdiv(groups, gpw), 8)) * 8 * a.token_tiles; };
    auto go = [&](auto kern, int ks) {
        const int64_t wgs = grid_of(kMmWaves / ks);
        SKV_REQUIRE(wgs <= INT32_MAX, "proj_mm_kernel: grid of %lld workgroups is too large",
                    static_cast<long long>(wgs));
        const size_t lds = 2 * static_cast<size_t>(ks) * kMmPartBytes;
        const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                    hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds));
        if (attr != hipSuccess) return set_error(SKV_ERR_HIP, "proj_mm_kernel: %s", hipGetErrorString(attr));
        kern<<<static_cast<unsigned>(wgs), 64 * kMmWaves, lds, s>>>(a);
        return check_launch("proj_mm_kernel");
    };
    if (grid_of(kMmWaves) < 256 && f.K % 256 == 0) return go(proj_mm_kernel<MODE, 2>, 2);
    return go(proj_mm_kernel<MODE, 1>, 1);
}

// ---------------------------------------------------------------------------
// Kernels around the library GEMMs of the prompt-pass projections
// (skv_prompt_gemm.hip): the input split before them and the epilogues after.
// ---------------------------------------------------------------------------
typedef __bf16 pg_bf16x2_t __attribute__((ext_vector_type(2)));

// hi = bf16(v) (round to nearest even) of two values and lo = bf16 of the
// exact remainders v - hi, packed two to a word.
__device__ __forceinline__ void split_pair(float v0, float v1, uint32_t& hi, uint32_t& lo) {
    const pg_bf16x2_t h = {static_cast<__bf16>(v0), static_cast<__bf16>(v1)};
    hi = __builtin_bit_cast(uint32_t, h);
    const pg_bf16x2_t l = {static_cast<__bf16>(v0 - bf16_lo(hi)), static_cast<__bf16>(v1 - bf16_hi(hi))};
    lo = __builtin_bit_cast(uint32_t, l);
}

// One workgroup per row; each thread splits 4 consecutive values per pass.
// With a RoPE table (rope.cs != nullptr) the workgroup also writes its token's
// cos / sin per rotation pair (rope_cos_sin of position first + row), which
// the q/k/v epilogue then reads for every head.
struct SplitRope {
    float* cs;        // [rows][head_dim / 2][cos, sin], or nullptr
    int first, head_dim;
};

template <bool NORM>
__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ x, int rows, int K,
                                                         const float* __restrict__ gamma, float eps,
                                                         float* __restrict__ normalized,
                                                         uint16_t* __restrict__ parts, SplitRope rope,
                                                         RopeTable freq) {
    extern __shared__ float xg_s[];  // NORM: [2][K], the row and gamma
    __shared__ float red[4];
    const int row = blockIdx.x;
    if (rope.cs != nullptr && static_cast<int>(threadIdx.x) < rope.head_dim / 2) {
        float c, sn;
        rope_cos_sin(rope.first + row, freq.cs[threadIdx.x], c, sn);
        *reinterpret_cast<float2*>(rope.cs + (static_cast<int64_t>(row) * (rope.head_dim / 2) + threadIdx.x) * 2) =
            float2{c, sn};
    }
    const float* xr = x + static_cast<int64_t>(row) * K;
    float inv = 1.0f;
    if constexpr (NORM) {
        stage_to_lds(xr, xg_s, K);
        stage_to_lds(gamma, xg_s + K, K);
        __syncthreads();
        inv = rms_inverse([&](int i) { return xg_s[i]; }, K, eps, red);
    }
    uint16_t* hi_row = parts + static_cast<int64_t>(row) * K;
    uint16_t* lo_row = parts + (static_cast<int64_t>(rows) + row) * K;
    for (int i = 4 * threadIdx.x; i < K; i += 4 * 256) {
        f32x4_t v;
        if constexpr (NORM) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = xg_s[i + e] * inv * xg_s[K + i + e];   // rmsnorm_kernel's rounding
            *reinterpret_cast<f32x4_t*>(normalized + static_cast<int64_t>(row) * K + i) = v;
        } else {
            v = *reinterpret_cast<const f32x4_t*>(xr + i);
        }
        uint2 h, l;
        split_pair(v[0], v[1], h.x, l.x);
        split_pair(v[2], v[3], h.y, l.y);
        *reinterpret_cast<uint2*>(hi_row + i) = h;
        *reinterpret_cast<uint2*>(lo_row + i) = l;
    }
}

__device__ __forceinline__ f32x4_t ld4(const float* p) { return *reinterpret_cast<const f32x4_t*>(p); }
__device__ __forceinline__ f32x4_t bias4_at(const float* b, int j) {
    return b != nullptr ? ld4(b + j) : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
}
// Output j..j+3 of token r from the two halves of d (row stride ld), plus bias.
__device__ __forceinline__ f32x4_t gemm_out4(const float* d, const float* bias, int ld, int rows, int r, int j) {
    return (ld4(d + static_cast<int64_t>(r) * ld + j) + ld4(d + (static_cast<int64_t>(rows) + r) * ld + j)) +
           bias4_at(bias, j);
}

// qkv: each thread takes 8 outputs of one token: 4 rotation pairs
// (p .. p+3 with p + hd/2 .. p+3 + hd/2 of one head) of q or k, or 8
// consecutive outputs of v (or of q and k without RoPE).
__global__ __launch_bounds__(256) void qkv_epilogue_kernel(GemmEpilogue e) {
    const int units = (e.n[0] + e.n[1] + e.n[2]) / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(e.rows) * units) return;
    const int r = static_cast<int>(i / units);
    int u = static_cast<int>(i - static_cast<int64_t>(r) * units), m = 0;
    while (m < 2 && u >= e.n[m] / 8) u -= e.n[m] / 8, ++m;
    const bool rope = m < 2 && e.first >= 0;
    const int half = e.head_dim / 2;
    const int ja = rope ? (u / (half / 4)) * e.head_dim + (u % (half / 4)) * 4 : 8 * u;
    const int jb = rope ? ja + half : ja + 4;
    f32x4_t a = gemm_out4(e.d[m], e.bias[m], e.ld[m], e.rows, r, ja);
    f32x4_t b = gemm_out4(e.d[m], e.bias[m], e.ld[m], e.rows, r, jb);
    if (rope) {
        const float* cs = e.rope_cs + (static_cast<int64_t>(r) * half + ja % e.head_dim) * 2;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            float va = a[t], vb = b[t];
            rotate_pair(va, vb, cs[2 * t], cs[2 * t + 1]);
            a[t] = va;
            b[t] = vb;
        }
    }
    float* y = e.y[m] + static_cast<int64_t>(r) * e.n[m];
    *reinterpret_cast<f32x4_t*>(y + ja) = a;
    *reinterpret_cast<f32x4_t*>(y + jb) = b;
}

// PARTS: the activations go out already split (e.parts, [2 rows][n] bf16,
// split_rows_kernel's layout and rounding) as the next GEMM's input, instead
// of as fp32 rows.
template <bool PARTS>
__global__ __launch_bounds__(256) void gate_up_epilogue_kernel(GemmEpilogue e) {
    const int units = e.n[0] / 4;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(e.rows) * units) return;
    const int r = static_cast<int>(i / units), j = 4 * static_cast<int>(i - static_cast<int64_t>(r) * units);
    const f32x4_t g = gemm_out4(e.d[0], e.bias[0], e.ld[0], e.rows, r, j);
    const f32x4_t u = gemm_out4(e.d[1], e.bias[1], e.ld[1], e.rows, r, j);
    const f32x4_t act = {swiglu_of(g[0], u[0]), swiglu_of(g[1], u[1]), swiglu_of(g[2], u[2]), swiglu_of(g[3], u[3])};
    if constexpr (PARTS) {
        uint2 h, l;
        split_pair(act[0], act[1], h.x, l.x);
        split_pair(act[2], act[3], h.y, l.y);
        *reinterpret_cast<uint2*>(e.parts + static_cast<int64_t>(r) * e.n[0] + j) = h;
        *reinterpret_cast<uint2*>(e.parts + (static_cast<int64_t>(e.rows) + r) * e.n[0] + j) = l;
    } else {
        *reinterpret_cast<f32x4_t*>(e.y[0] + static_cast<int64_t>(r) * e.n[0] + j) = act;
    }
}

__global__ __launch_bounds__(256) void residual_epilogue_kernel(GemmEpilogue e) {
    const int units = e.n[0] / 4;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(e.rows) * units) return;
    const int r = static_cast<int>(i / units), j = 4 * static_cast<int>(i - static_cast<int64_t>(r) * units);
    const int64_t at = static_cast<int64_t>(r) * e.n[0] + j;
    *reinterpret_cast<f32x4_t*>(e.y[0] + at) = gemm_out4(e.d[0], e.bias[0], e.ld[0], e.rows, r, j) + ld4(e.residual + at);
}

int launch_split_rows(const float* x, int rows, int K, const float* gamma, float eps, float* normalized,
                      uint16_t* parts, hipStream_t s, float* rope_cs, int first, int head_dim) {
    const SplitRope rope{rope_cs, first, head_dim};
    const RopeTable& inv = rope_cs != nullptr ? rope_inv_freq(head_dim) : RopeTable{};
    if (gamma != nullptr)
        split_rows_kernel<true><<<rows, 256, 2 * sizeof(float) * K, s>>>(x, rows, K, gamma, eps, normalized, parts,
                                                                          rope, inv);
    else
        split_rows_kernel<false><<<rows, 256, 0, s>>>(x, rows, K, nullptr, eps, nullptr, parts, rope, inv);
    return check_launch("split_rows_kernel");
}

namespace {
unsigned epilogue_grid(int rows, int units) {
    return static_cast<unsigned>(cdiv<int64_t>(static_cast<int64_t>(rows) * units, 256));
}
}  // namespace

int launch_qkv_epilogue(const GemmEpilogue& e, hipStream_t s) {
    qkv_epilogue_kernel<<<epilogue_grid(e.rows, (e.n[0] + e.n[1] + e.n[2]) / 8), 256, 0, s>>>(e);
    return check_launch("qkv_epilogue_kernel");
}

int launch_gate_up_epilogue(const GemmEpilogue& e, hipStream_t s) {
    if (e.parts != nullptr) gate_up_epilogue_kernel<true><<<epilogue_grid(e.rows, e.n[0] / 4), 256, 0, s>>>(e);
    else gate_up_epilogue_kernel<false><<<epilogue_grid(e.rows, e.n[0] / 4), 256, 0, s>>>(e);
    return check_launch("gate_up_epilogue_kernel");
}

int launch_residual_epilogue(const GemmEpilogue& e, hipStream_t s) {
    residual_epilogue_kernel<<<epilogue_grid(e.rows, e.n[0] / 4), 256, 0, s>>>(e);
    return check_launch("residual_epilogue_kernel");
}

}  // namespace skv

using namespace skv;

extern "C" int skv_rmsnorm_f32(const float* input, float* output, const float* gamma, int rows,
                               int hidden, float epsilon, void* stream) {
    SKV_REQUIRE(input && output && gamma && rows > 0 && hidden > 0,
                "skv_rmsnorm_f32: invalid pointers or sizes");
    SKV_REQUIRE(hidden <= 8192, "skv_rmsnorm_f32: hidden size %d exceeds 8192", hidden);
    rmsnorm_kernel<<<rows, 256, 2 * sizeof(float) * hidden, static_cast<hipStream_t>(stream)>>>(
        input, output, gamma, hidden, epsilon);
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
    if (rows == 1 && fused_rows_ok(weight, stride_k, stride_n, in_dim, static_cast<int>(esz))) {
        FusedGemv f{};
        f.x = x;
        f.K = in_dim;
        f.w[0] = weight;
        f.row_bytes[0] = stride_n * esz;
        f.bias[0] = bias;
        f.n[0] = out_dim;
        f.y[0] = y;
        return launch_fused<FUSED_LINEAR>(f, bf16, cdiv(out_dim, 2), s);
    }
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
    SKV_REQUIRE(head_dim / 2 <= kMaxRopePairs, "skv_rope_f32: head_dim %d exceeds %d", head_dim,
                2 * kMaxRopePairs);
    const int n = heads * (head_dim / 2);
    rope_kernel<<<cdiv(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(x, heads, head_dim,
                                                                          rope_table(head_dim, position));
    return check_launch("rope_kernel");
}

extern "C" int skv_rope_rows_f32(float* x, int rows, int heads, int head_dim, int first_position,
                                 void* stream) {
    SKV_REQUIRE(x && rows > 0 && heads > 0 && head_dim > 0 && head_dim % 2 == 0 && first_position >= 0,
                "skv_rope_rows_f32: invalid pointers or sizes");
    SKV_REQUIRE(head_dim / 2 <= kMaxRopePairs, "skv_rope_rows_f32: head_dim %d exceeds %d", head_dim,
                2 * kMaxRopePairs);
    const int64_t n = static_cast<int64_t>(rows) * heads * (head_dim / 2);
    rope_rows_kernel<<<static_cast<unsigned>(cdiv<int64_t>(n, 256)), 256, 0, static_cast<hipStream_t>(stream)>>>(
        x, rows, heads, head_dim, first_position, rope_inv_freq(head_dim));
    return check_launch("rope_rows_kernel");
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

namespace {

// Shared by the one-token entry points and their *_rows variants (rows
// tokens, row-major x / y / residual); `fn` names the entry point in errors.
// Several tokens with gamma: rmsnorm_kernel writes the normalised rows into
// `normalized` (the bits the one-token kernels normalise to), which the
// projections then read.
int normalize_rows(const char* fn, const float*& x, int rows, const float* gamma, float epsilon, int K,
                   float* normalized, hipStream_t s) {
    if (gamma == nullptr) return SKV_OK;
    SKV_REQUIRE(normalized != nullptr, "%s: normalized scratch required with gamma", fn);
    rmsnorm_kernel<<<rows, 256, 2 * sizeof(float) * K, s>>>(x, normalized, gamma, K, epsilon);
    if (int rc = check_launch("rmsnorm_kernel")) return rc;
    x = normalized;
    return SKV_OK;
}

int fused_qkv(const char* fn, const float* hidden, int rows, const float* gamma, float epsilon,
              const void* wq, const void* wk, const void* wv, int weight_dtype, int64_t stride_k,
              const int64_t stride_n[3], const float* bias_q, const float* bias_k, const float* bias_v,
              int hidden_dim, int num_heads, int num_kv_heads, int head_dim, int position, float* q,
              float* k, float* v, float* normalized, void* stream, bool mm = false,
              const int32_t* position_at = nullptr, const float* rope_dev = nullptr, int rope_positions = 0) {
    SKV_REQUIRE(hidden && stride_n && q && k && v && rows > 0 && hidden_dim > 0 && num_heads > 0 &&
                    num_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0,
                "%s: invalid pointers or sizes", fn);
    SKV_REQUIRE(weight_dtype == SKV_DTYPE_BF16 || weight_dtype == SKV_DTYPE_FP32,
                "%s: unknown weight dtype %d", fn, weight_dtype);
    const int esz = weight_dtype == SKV_DTYPE_BF16 ? 2 : 4;
    const void* ws[3] = {wq, wk, wv};
    for (int m = 0; m < 3; ++m)
        if (!fused_rows_ok(ws[m], stride_k, stride_n[m], hidden_dim, esz))
            return set_error(SKV_ERR_UNSUPPORTED,
                             "%s: weights must be 16-byte aligned output-major rows and hidden_dim <= %d", fn,
                             kGemvMaxLdsK);
    FusedGemv f{};
    f.x = hidden;
    f.gamma = gamma;
    f.eps = epsilon;
    f.K = hidden_dim;
    f.rows = rows;
    const int ns[3] = {num_heads * head_dim, num_kv_heads * head_dim, num_kv_heads * head_dim};
    const float* bs[3] = {bias_q, bias_k, bias_v};
    float* ys[3] = {q, k, v};
    for (int m = 0; m < 3; ++m) {
        f.w[m] = ws[m];
        f.row_bytes[m] = stride_n[m] * esz;
        f.bias[m] = bs[m];
        f.n[m] = ns[m];
        f.y[m] = ys[m];
    }
    f.head_dim = head_dim;
    f.position = position;
    if (position >= 0 && head_dim / 2 > kMaxRopePairs)
        return set_error(SKV_ERR_UNSUPPORTED, "%s: head_dim %d exceeds %d", fn, head_dim, 2 * kMaxRopePairs);
    const int items = (ns[0] + ns[1] + ns[2]) / 2;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (mm) {
        if (gamma != nullptr) SKV_REQUIRE(normalized != nullptr, "%s: normalized scratch required with gamma", fn);
        FusedGemv fx = f;
        fx.x = gamma != nullptr ? normalized : hidden;
        if (!mm_supported(fx, 3, esz, stride_k) || (position >= 0 && head_dim % 32 != 0) || !aligned16(q) ||
            !aligned16(k) || !aligned16(v))
            return set_error(SKV_ERR_UNSUPPORTED,
                             "%s: needs bf16 weights, hidden_dim a multiple of 128, outputs and head_dim multiples "
                             "of 32 and 16-byte aligned input and outputs", fn);
        if (position >= 0) f.rope = rope_inv_freq(head_dim);
        if (int rc = normalize_rows(fn, f.x, rows, gamma, epsilon, hidden_dim, normalized, s)) return rc;
        f.gamma = nullptr;
        return launch_mm<FUSED_QKV>(f, (ns[0] + ns[1] + ns[2]) / 32, s);
    }
    if (rows == 1) {
        if (position_at != nullptr) {
            f.position = 0;   // RoPE on; the position itself is read on the device
            f.position_at = position_at;
            f.rope_dev = rope_dev;
            f.rope_positions = rope_positions;
        } else if (position >= 0) {
            f.rope = rope_table(head_dim, position);
        }
        return launch_fused<FUSED_QKV>(f, esz == 2, items, s);
    }
    if (position >= 0) f.rope = rope_inv_freq(head_dim);
    if (!rows_supported(esz == 2, hidden_dim))
        return set_error(SKV_ERR_UNSUPPORTED, "%s: hidden_dim %d is not a supported multi-token size", fn,
                         hidden_dim);
    if (int rc = normalize_rows(fn, f.x, rows, gamma, epsilon, hidden_dim, normalized, s)) return rc;
    f.gamma = nullptr;
    return launch_fused_rows<FUSED_QKV>(f, esz == 2, items, s);
}

int fused_gate_up(const char* fn, const float* x, int rows, const float* gamma, float epsilon,
                  const void* w_gate, const void* w_up, int weight_dtype, int64_t stride_k,
                  int64_t stride_n_gate, int64_t stride_n_up, const float* bias_gate, const float* bias_up,
                  int in_dim, int out_dim, float* act, float* normalized, void* stream, bool mm = false) {
    SKV_REQUIRE(x && act && rows > 0 && in_dim > 0 && out_dim > 0, "%s: invalid pointers or sizes", fn);
    SKV_REQUIRE(weight_dtype == SKV_DTYPE_BF16 || weight_dtype == SKV_DTYPE_FP32,
                "%s: unknown weight dtype %d", fn, weight_dtype);
    const int esz = weight_dtype == SKV_DTYPE_BF16 ? 2 : 4;
    if (!fused_rows_ok(w_gate, stride_k, stride_n_gate, in_dim, esz) ||
        !fused_rows_ok(w_up, stride_k, stride_n_up, in_dim, esz))
        return set_error(SKV_ERR_UNSUPPORTED,
                         "%s: weights must be 16-byte aligned output-major rows and in_dim <= %d", fn,
                         kGemvMaxLdsK);
    FusedGemv f{};
    f.x = x;
    f.gamma = gamma;
    f.eps = epsilon;
    f.K = in_dim;
    f.rows = rows;
    f.w[0] = w_gate;
    f.w[1] = w_up;
    f.row_bytes[0] = stride_n_gate * esz;
    f.row_bytes[1] = stride_n_up * esz;
    f.bias[0] = bias_gate;
    f.bias[1] = bias_up;
    f.n[0] = f.n[1] = out_dim;
    f.y[0] = act;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (mm) {
        if (gamma != nullptr) SKV_REQUIRE(normalized != nullptr, "%s: normalized scratch required with gamma", fn);
        FusedGemv fx = f;
        fx.x = gamma != nullptr ? normalized : x;
        if (!mm_supported(fx, 2, esz, stride_k) || !aligned16(act))
            return set_error(SKV_ERR_UNSUPPORTED,
                             "%s: needs bf16 weights, in_dim a multiple of 128, out_dim a multiple of 16 and "
                             "16-byte aligned input and output", fn);
        if (int rc = normalize_rows(fn, f.x, rows, gamma, epsilon, in_dim, normalized, s)) return rc;
        f.gamma = nullptr;
        return launch_mm<FUSED_GATE_UP>(f, out_dim / 16, s);
    }
    if (rows == 1) return launch_fused<FUSED_GATE_UP>(f, esz == 2, out_dim, s);
    if (!rows_supported(esz == 2, in_dim))
        return set_error(SKV_ERR_UNSUPPORTED, "%s: in_dim %d is not a supported multi-token size", fn, in_dim);
    if (int rc = normalize_rows(fn, f.x, rows, gamma, epsilon, in_dim, normalized, s)) return rc;
    f.gamma = nullptr;
    return launch_fused_rows<FUSED_GATE_UP>(f, esz == 2, out_dim, s);
}

int linear_residual(const char* fn, const float* x, int rows, const void* weight, int weight_dtype,
                    int64_t stride_k, int64_t stride_n, int in_dim, int out_dim, const float* bias,
                    const float* residual, float* y, void* stream, bool mm = false) {
    SKV_REQUIRE(x && residual && y && rows > 0 && in_dim > 0 && out_dim > 0, "%s: invalid pointers or sizes",
                fn);
    SKV_REQUIRE(weight_dtype == SKV_DTYPE_BF16 || weight_dtype == SKV_DTYPE_FP32,
                "%s: unknown weight dtype %d", fn, weight_dtype);
    const int esz = weight_dtype == SKV_DTYPE_BF16 ? 2 : 4;
    if (!fused_rows_ok(weight, stride_k, stride_n, in_dim, esz))
        return set_error(SKV_ERR_UNSUPPORTED,
                         "%s: weights must be 16-byte aligned output-major rows and in_dim <= %d", fn,
                         kGemvMaxLdsK);
    FusedGemv f{};
    f.x = x;
    f.gamma = nullptr;
    f.K = in_dim;
    f.rows = rows;
    f.w[0] = weight;
    f.row_bytes[0] = stride_n * esz;
    f.bias[0] = bias;
    f.n[0] = out_dim;
    f.y[0] = y;
    f.residual = residual;
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (mm) {
        if (!mm_supported(f, 1, esz, stride_k) || !aligned16(y) || !aligned16(residual))
            return set_error(SKV_ERR_UNSUPPORTED,
                             "%s: needs bf16 weights, in_dim a multiple of 128, out_dim a multiple of 32 and "
                             "16-byte aligned input, residual and output", fn);
        return launch_mm<FUSED_RESIDUAL>(f, out_dim / 32, s);
    }
    if (rows == 1) return launch_fused<FUSED_RESIDUAL>(f, esz == 2, cdiv(out_dim, 2), s);
    return launch_fused_rows<FUSED_RESIDUAL>(f, esz == 2, cdiv(out_dim, 2), s);
}

}  // namespace

extern "C" int skv_fused_qkv_f32(const float* hidden, const float* gamma, float epsilon,
                                 const void* wq, const void* wk, const void* wv, int weight_dtype,
                                 int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                                 const float* bias_k, const float* bias_v, int hidden_dim,
                                 int num_heads, int num_kv_heads, int head_dim, int position,
                                 float* q, float* k, float* v, void* stream) {
    return fused_qkv("skv_fused_qkv_f32", hidden, 1, gamma, epsilon, wq, wk, wv, weight_dtype, stride_k,
                     stride_n, bias_q, bias_k, bias_v, hidden_dim, num_heads, num_kv_heads, head_dim, position,
                     q, k, v, nullptr, stream);
}

extern "C" int skv_fused_qkv_at_f32(const float* hidden, const float* gamma, float epsilon,
                                    const void* wq, const void* wk, const void* wv, int weight_dtype,
                                    int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                                    const float* bias_k, const float* bias_v, int hidden_dim,
                                    int num_heads, int num_kv_heads, int head_dim, const int32_t* position_at,
                                    const float* rope_cos_sin, int rope_positions, float* q, float* k, float* v,
                                    void* stream) {
    SKV_REQUIRE(position_at && rope_cos_sin && rope_positions > 0,
                "skv_fused_qkv_at_f32: NULL position or RoPE table, or no positions");
    SKV_REQUIRE(head_dim / 2 <= kMaxRopePairs, "skv_fused_qkv_at_f32: head_dim %d exceeds %d", head_dim,
                2 * kMaxRopePairs);
    return fused_qkv("skv_fused_qkv_at_f32", hidden, 1, gamma, epsilon, wq, wk, wv, weight_dtype, stride_k, stride_n,
                     bias_q, bias_k, bias_v, hidden_dim, num_heads, num_kv_heads, head_dim, 0, q, k, v, nullptr,
                     stream, false, position_at, rope_cos_sin, rope_positions);
}

extern "C" int skv_rope_cos_sin(int head_dim, int first_position, int positions, float* cos_sin) {
    SKV_REQUIRE(cos_sin && head_dim > 0 && head_dim % 2 == 0 && first_position >= 0 && positions > 0 &&
                    first_position <= INT32_MAX - positions,
                "skv_rope_cos_sin: invalid arguments");
    SKV_REQUIRE(head_dim / 2 <= kMaxRopePairs, "skv_rope_cos_sin: head_dim %d exceeds %d", head_dim,
                2 * kMaxRopePairs);
    for (int i = 0; i < positions; ++i) {
        const RopeTable& t = rope_table(head_dim, first_position + i);
        std::copy(t.cs, t.cs + head_dim, cos_sin + static_cast<size_t>(i) * head_dim);
    }
    return SKV_OK;
}

extern "C" int skv_fused_qkv_rows_f32(const float* hidden, int rows, const float* gamma, float epsilon,
                                      const void* wq, const void* wk, const void* wv, int weight_dtype,
                                      int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                                      const float* bias_k, const float* bias_v, int hidden_dim,
                                      int num_heads, int num_kv_heads, int head_dim, int first_position,
                                      float* q, float* k, float* v, float* normalized, void* stream) {
    return fused_qkv("skv_fused_qkv_rows_f32", hidden, rows, gamma, epsilon, wq, wk, wv, weight_dtype,
                     stride_k, stride_n, bias_q, bias_k, bias_v, hidden_dim, num_heads, num_kv_heads, head_dim,
                     first_position, q, k, v, normalized, stream);
}

extern "C" int skv_fused_gate_up_swiglu_f32(const float* x, const float* gamma, float epsilon,
                                            const void* w_gate, const void* w_up, int weight_dtype,
                                            int64_t stride_k, int64_t stride_n_gate,
                                            int64_t stride_n_up, const float* bias_gate,
                                            const float* bias_up, int in_dim, int out_dim,
                                            float* act, void* stream) {
    return fused_gate_up("skv_fused_gate_up_swiglu_f32", x, 1, gamma, epsilon, w_gate, w_up, weight_dtype,
                         stride_k, stride_n_gate, stride_n_up, bias_gate, bias_up, in_dim, out_dim, act, nullptr,
                         stream);
}

extern "C" int skv_fused_gate_up_swiglu_rows_f32(const float* x, int rows, const float* gamma, float epsilon,
                                                 const void* w_gate, const void* w_up, int weight_dtype,
                                                 int64_t stride_k, int64_t stride_n_gate,
                                                 int64_t stride_n_up, const float* bias_gate,
                                                 const float* bias_up, int in_dim, int out_dim,
                                                 float* act, float* normalized, void* stream) {
    return fused_gate_up("skv_fused_gate_up_swiglu_rows_f32", x, rows, gamma, epsilon, w_gate, w_up,
                         weight_dtype, stride_k, stride_n_gate, stride_n_up, bias_gate, bias_up, in_dim,
                         out_dim, act, normalized, stream);
}

extern "C" int skv_linear_residual_f32(const float* x, const void* weight, int weight_dtype,
                                       int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                                       const float* bias, const float* residual, float* y,
                                       void* stream) {
    return linear_residual("skv_linear_residual_f32", x, 1, weight, weight_dtype, stride_k, stride_n, in_dim,
                           out_dim, bias, residual, y, stream);
}

extern "C" int skv_linear_residual_rows_f32(const float* x, int rows, const void* weight, int weight_dtype,
                                            int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                                            const float* bias, const float* residual, float* y,
                                            void* stream) {
    return linear_residual("skv_linear_residual_rows_f32", x, rows, weight, weight_dtype, stride_k, stride_n,
                           in_dim, out_dim, bias, residual, y, stream);
}

extern "C" int skv_fused_qkv_mm_f32(const float* hidden, int rows, const float* gamma, float epsilon,
                                    const void* wq, const void* wk, const void* wv, int weight_dtype,
                                    int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                                    const float* bias_k, const float* bias_v, int hidden_dim, int num_heads,
                                    int num_kv_heads, int head_dim, int first_position, float* q, float* k,
                                    float* v, float* normalized, void* stream) {
    return fused_qkv("skv_fused_qkv_mm_f32", hidden, rows, gamma, epsilon, wq, wk, wv, weight_dtype, stride_k,
                     stride_n, bias_q, bias_k, bias_v, hidden_dim, num_heads, num_kv_heads, head_dim,
                     first_position, q, k, v, normalized, stream, true);
}

extern "C" int skv_fused_gate_up_swiglu_mm_f32(const float* x, int rows, const float* gamma, float epsilon,
                                               const void* w_gate, const void* w_up, int weight_dtype,
                                               int64_t stride_k, int64_t stride_n_gate, int64_t stride_n_up,
                                               const float* bias_gate, const float* bias_up, int in_dim,
                                               int out_dim, float* act, float* normalized, void* stream) {
    return fused_gate_up("skv_fused_gate_up_swiglu_mm_f32", x, rows, gamma, epsilon, w_gate, w_up, weight_dtype,
                         stride_k, stride_n_gate, stride_n_up, bias_gate, bias_up, in_dim, out_dim, act, normalized,
                         stream, true);
}

extern "C" int skv_linear_residual_mm_f32(const float* x, int rows, const void* weight, int weight_dtype,
                                          int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                                          const float* bias, const float* residual, float* y, void* stream) {
    return linear_residual("skv_linear_residual_mm_f32", x, rows, weight, weight_dtype, stride_k, stride_n,
                           in_dim, out_dim, bias, residual, y, stream, true);
}

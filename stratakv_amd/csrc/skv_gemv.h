// skv_gemv.h -- the GEMV row primitives shared by the decode-step projections
// (skv_layer_ops.hip) and the attention kernel that folds the output
// projection into its epilogue (skv_decode.hip): every caller computes a
// weight row's dot product with exactly the same loads and arithmetic, so a
// fused and a separate projection give the same bits.  Internal header: not
// part of the C ABI.
#pragma once

#include "skv_common.h"

namespace skv {

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

    PairPrefetch() = default;                    // nothing requested (assigned before use)
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

}  // namespace skv

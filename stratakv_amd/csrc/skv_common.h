// skv_common.h -- shared device helpers and host error plumbing for the gfx950
// paged KV-cache kernels.  Internal header: not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <string>

#include "stratakv_amd.h"

namespace skv {

// ---------------------------------------------------------------------------
// Host-side error reporting.  The ABI never throws; it records a message per
// thread and returns a status code.
// ---------------------------------------------------------------------------
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Mirrors STRATAKV_SYNC_KERNELS=1 of the reference (include/stratakv/cuda_utils.cuh:42-51):
// when set, every launch is followed by a device synchronisation so a kernel
// fault is reported by the call that caused it.
bool sync_kernels_enabled();
int check_launch(const char* what);

#define SKV_HIP_TRY(expr)                                                        \
    do {                                                                         \
        hipError_t skv_e_ = (expr);                                              \
        if (skv_e_ != hipSuccess)                                                \
            return ::skv::set_error(SKV_ERR_HIP, "%s failed: %s", #expr,         \
                                    hipGetErrorString(skv_e_));                  \
    } while (0)

#define SKV_REQUIRE(cond, ...)                                                   \
    do {                                                                         \
        if (!(cond)) return ::skv::set_error(SKV_ERR_INVALID_ARGUMENT, __VA_ARGS__); \
    } while (0)

inline bool aligned16(const void* p) {
    return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0;
}

template <typename T>
__host__ __device__ inline T cdiv(T a, T b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// bf16 bit rules.  Widening is exact (the bits become the high half of an
// fp32, src/cpu/tensor.cpp:200-206).  Narrowing rounds to nearest, ties to
// even, on the raw bit pattern exactly as Tensor::set_value does
// (src/cpu/tensor.cpp:218-225): no special case for NaN, so the result is
// bit-identical to the reference for every input.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float bf16_lo(uint32_t pair) {
    return __uint_as_float(pair << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t pair) {
    return __uint_as_float(pair & 0xffff0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
    return __uint_as_float(static_cast<uint32_t>(h) << 16);
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    const uint32_t bits = __float_as_uint(f);
    uint32_t upper = bits >> 16;
    const uint32_t lower = bits & 0xffffu;
    if (lower > 0x8000u || (lower == 0x8000u && (upper & 1u) != 0u)) ++upper;
    return upper & 0xffffu;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// Unpack 8 bf16 held in a 16-byte vector into fp32.
__device__ __forceinline__ void unpack8(const uint4& w, float (&f)[8]) {
    f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
    f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
    f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
    f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

// ---------------------------------------------------------------------------
// Wavefront data movement.  DPP moves stay inside a 16-lane row and cost no
// LDS traffic; the encodings are the GFX9 DPP control words.
// ---------------------------------------------------------------------------
enum : int {
    DPP_QUAD_1032 = 0xB1,   // quad_perm [1,0,3,2]
    DPP_QUAD_2301 = 0x4E,   // quad_perm [2,3,0,1]
    DPP_ROW_MIRROR = 0x140, // lane i <- lane 15-i within a row of 16
    DPP_ROW_HALF_MIRROR = 0x141, // lane i <- lane 7-i within each half-row of 8
};

template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(
        0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Butterfly sum over aligned groups of N lanes (N = 2, 4, 8 or 16).  Every lane
// of a group ends with the same bits: each step adds the same two operands.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
    static_assert(N == 2 || N == 4 || N == 8 || N == 16, "group size");
    x += dpp_mov<DPP_QUAD_1032>(x);
    if constexpr (N >= 4) x += dpp_mov<DPP_QUAD_2301>(x);
    if constexpr (N >= 8) x += dpp_mov<DPP_ROW_HALF_MIRROR>(x);
    if constexpr (N >= 16) x += dpp_mov<DPP_ROW_MIRROR>(x);
    return x;
}

__device__ __forceinline__ float shfl_xor_f(float x, int mask) {
    return __shfl_xor(x, mask, 64);
}

__device__ __forceinline__ float wave_max(float x) {
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}
__device__ __forceinline__ float wave_sum(float x) {
    for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

__device__ __forceinline__ float fast_exp2(float x) {
    return __builtin_amdgcn_exp2f(x);
}

// LDS hand-off between the lanes of ONE wavefront (not between wavefronts).
// The LDS instructions of a wavefront execute in issue order, so a ds_read
// issued after a ds_write of the same wavefront sees it without s_barrier; the
// fences only stop the compiler from moving LDS accesses across this point.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Value of lane `src` (a compile-time or wave-uniform index), as a scalar.
__device__ __forceinline__ float lane_value(float x, int src) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), src));
}

}  // namespace skv

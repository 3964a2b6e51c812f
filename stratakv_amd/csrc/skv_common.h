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
    DPP_ROW_ROR8 = 0x128,   // lane i <- lane i ^ 8 within a row of 16 (rotation by 8)
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

// Pairwise exchange-and-add between lane l and lane l ^ 32 (swap32_sum),
// l ^ 16 (swap16_sum) or l ^ 8 (swap8_sum) of two values a, b: the lower lane
// of each pair returns a(lower) + a(upper), the upper lane b(lower) + b(upper).
// v_permlane32_swap exchanges the upper half of its first operand with the
// lower half of its second, v_permlane16_swap the odd 16-lane rows of the
// first with the even rows of the second; the 8-lane exchange is a row
// rotation by 8 (DPP) written to one half of each row's banks at a time.
__device__ __forceinline__ float swap32_sum(float a, float b) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float swap16_sum(float a, float b) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float swap8_sum(float a, float b) {
    constexpr int kRowRor8 = 0x128;
    const float lo = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(b), __float_as_int(a), kRowRor8, 0xF, 0x3, false));
    const float hi = __int_as_float(
        __builtin_amdgcn_update_dpp(__float_as_int(a), __float_as_int(b), kRowRor8, 0xF, 0xC, false));
    return lo + hi;
}

// Reduce-scatter of N per-lane values over the lanes that share lane bits
// 0 .. LO-1 (the groups l, l + 2^LO, ...; LO = 3 or 4): every exchange keeps
// complementary halves, so afterwards lane l holds, in v[0 .. N/2^(6-LO)), the
// group sums of values (l >> LO) * N/2^(6-LO) + i.  Each sum is the same
// pairwise tree for every value: bit 5 pairs first, then bit 4, then bit 3.
template <int N, int LO>
__device__ __forceinline__ void reduce_scatter_high_bits(float (&v)[N]) {
    static_assert((LO == 3 || LO == 4) && N % (1 << (6 - LO)) == 0, "reduce-scatter shape");
#pragma unroll
    for (int i = 0; i < N / 2; ++i) v[i] = swap32_sum(v[i], v[i + N / 2]);
#pragma unroll
    for (int i = 0; i < N / 4; ++i) v[i] = swap16_sum(v[i], v[i + N / 4]);
    if constexpr (LO == 3) {
#pragma unroll
        for (int i = 0; i < N / 8; ++i) v[i] = swap8_sum(v[i], v[i + N / 8]);
    }
}

__device__ __forceinline__ float shfl_xor_f(float x, int mask) {
    return __shfl_xor(x, mask, 64);
}

// wave_sum of N values at once, scattered: afterwards lane l holds, in
// v[0 .. N/8), the wave sums of values (l >> 3) * N/8 + i (all 8 lanes of the
// group the same).  Each sum pairs and orders its additions exactly as
// wave_sum does (lane bit 5 first, then 4, 3, 2, 1, 0, adding the two lanes'
// partial sums at each step), so it has wave_sum's bits.
template <int N>
__device__ __forceinline__ void wave_sum_scatter(float (&v)[N]) {
    reduce_scatter_high_bits<N, 3>(v);
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
        float x = v[i];
        x += __shfl_xor(x, 4, 64);
        x += dpp_mov<DPP_QUAD_2301>(x);
        x += dpp_mov<DPP_QUAD_1032>(x);
        v[i] = x;
    }
}

// Lane l combined with lane l ^ 32 (xor32_*) or l ^ 16 (xor16_*) without the
// LDS crossbar: the permlane swap of x with itself hands each lane its
// partner's value in one of the two results and its own in the other, and the
// operation is commutative (fmaxf and + give the same bits either way round),
// so every lane gets exactly op(x, __shfl_xor(x, 32 or 16)).
__device__ __forceinline__ float xor32_sum(float x) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float xor16_sum(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}
__device__ __forceinline__ float xor32_max(float x) {
    const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}
__device__ __forceinline__ float xor16_max(float x) {
    const auto s = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

// Butterflies over the 64 lanes, partner lane ^ 32, ^ 16, ^ 8, ^ 4, ^ 2, ^ 1
// in that order, each step combining the lane's and its partner's partial
// result: the bits of `for (o = 32; o > 0; o >>= 1) x op= __shfl_xor(x, o)`.
// Only the ^ 4 step goes through the LDS crossbar (GFX9 DPP has no such
// pattern); the others are permlane swaps and DPP moves.
__device__ __forceinline__ float wave_max(float x) {
    x = xor32_max(x);
    x = xor16_max(x);
    x = fmaxf(x, dpp_mov<DPP_ROW_ROR8>(x));
    x = fmaxf(x, __shfl_xor(x, 4, 64));
    x = fmaxf(x, dpp_mov<DPP_QUAD_2301>(x));
    return fmaxf(x, dpp_mov<DPP_QUAD_1032>(x));
}
__device__ __forceinline__ float wave_sum(float x) {
    x = xor32_sum(x);
    x = xor16_sum(x);
    x += dpp_mov<DPP_ROW_ROR8>(x);
    x += __shfl_xor(x, 4, 64);
    x += dpp_mov<DPP_QUAD_2301>(x);
    return x + dpp_mov<DPP_QUAD_1032>(x);
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

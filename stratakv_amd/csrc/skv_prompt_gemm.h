// skv_prompt_gemm.h -- the kernels around the library GEMMs of the prompt-pass
// projections (defined in skv_layer_ops.hip beside the RMSNorm, RoPE and
// SwiGLU arithmetic they share).  Internal header: not part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace skv {

// Prologue: row r of x (K floats; with gamma rmsnorm'd into normalized[r], the
// bits of rmsnorm_kernel) split into bf16 parts, hi = bf16(v) into row r and
// lo = bf16(v - hi) into row rows + r of `parts` ([2 * rows][K] bf16).  With
// rope_cs, also the cos / sin of every rotation pair at position first + r
// ([rows][head_dim / 2][cos, sin]) for the q/k/v epilogue.
int launch_split_rows(const float* x, int rows, int K, const float* gamma, float eps, float* normalized,
                      uint16_t* parts, hipStream_t s, float* rope_cs = nullptr, int first = 0, int head_dim = 0);

// Epilogues over GEMM outputs d[m] = [2 * rows][ld[m]] fp32 (row r: the hi
// products of token r, row rows + r its lo products): out = d[r] + d[rows + r]
// + bias, then
//   qkv:      RoPE of q and k at position first + r (first < 0: none; the
//             cos / sin from rope_cs, written by launch_split_rows) into y[m];
//   gate/up:  act = swiglu(gate, up) (into y[0], or split into parts);
//   residual: y = out + residual (y may alias residual).
struct GemmEpilogue {
    const float* d[3];
    const float* bias[3];
    float* y[3];
    int n[3];
    int ld[3];                // row stride of d[m] (n[m], or the packed GEMM's width)
    const float* residual;
    const float* rope_cs;
    uint16_t* parts;          // gate/up: write the activations split for the next GEMM here (else y[0])
    int rows, head_dim, first;
};
int launch_qkv_epilogue(const GemmEpilogue& e, hipStream_t s);
int launch_gate_up_epilogue(const GemmEpilogue& e, hipStream_t s);
int launch_residual_epilogue(const GemmEpilogue& e, hipStream_t s);

}  // namespace skv

/*
 * stratakv_amd_gemm.h -- C ABI of libstratakv_amd_gemm.so: the projections of
 * long prompt chunks with their products on hipBLASLt.
 *
 * Kept apart from stratakv_amd.h because it is the only part of this build
 * that links hipBLASLt: libstratakv_amd.so (append, decode, the layer kernels
 * and the C++ host layer) loads without it.  libstratakv_amd_gemm.so depends
 * on libstratakv_amd.so (the split and epilogue kernels, skv_last_error) and
 * is opened on demand by TransformerBlock::prefill_into; when it cannot be
 * opened, prompts run on the matrix-core projections (skv_*_mm_f32) instead.
 * Same conventions as stratakv_amd.h: plain C types, an int status, the
 * message of the last failure from skv_last_error().
 */
#ifndef STRATAKV_AMD_GEMM_H
#define STRATAKV_AMD_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The same three projections as the *_mm variants with the products on
 * hipBLASLt (bf16 x bf16 GEMMs, fp32 accumulation), for long prompts.  A
 * prologue kernel normalises the rows (with gamma, into `normalized`, the bits
 * of skv_rmsnorm_f32) and splits every input value v into hi = bf16(v) and
 * lo = bf16(v - hi), stacked as 2 * rows GEMM columns; one GEMM per weight
 * matrix computes W hi and W lo; an epilogue kernel adds the two halves and
 * applies bias, RoPE, SwiGLU or the residual as the *_mm variants do (y may
 * alias residual).  hi + lo keeps ~16 significant bits of v (relative error up
 * to ~2^-16, rounding of the lo part), every product is exact and the sums are
 * fp32: results agree with the *_mm variants' within that bound, not bit for
 * bit (different summation orders).
 * `workspace` (256-byte aligned) holds the split inputs, the GEMM outputs and
 * the library's own scratch: at least skv_prompt_gemm_workspace_bytes(rows,
 * in_dim, outputs per token: q + k + v, gate + up, or out_dim) bytes, else
 * SKV_ERR_INVALID_ARGUMENT.  SKV_ERR_UNSUPPORTED (nothing launched) unless the
 * weights are bf16 aligned output-major rows with a 16-byte row stride, in_dim
 * is a multiple of 8 up to 8,192, every output count is a multiple of 8,
 * head_dim is a multiple of 8 when rotating, the input, outputs, biases and
 * residual are 16-byte aligned and hipBLASLt offers an algorithm for each
 * GEMM.  Every GEMM runs hipBLASLt's first-ranked algorithm for its shape
 * (chosen by the library's heuristic, never by timing), so the results depend
 * only on the shape, the device and the hipBLASLt version: two processes give
 * the same bits.  The first call of a shape (the token count is part of it)
 * asks the heuristic once and keeps the plan; calls on one workspace must not
 * overlap.
 * Replaces: the same reference code as the rows variants
 * (src/models/transformer_block.cpp:300-332); no counterpart of its own. */
size_t skv_prompt_gemm_workspace_bytes(int rows, int in_dim, int outputs);
int skv_fused_qkv_gemm_f32(const float* hidden, int rows, const float* gamma, float epsilon,
                           const void* wq, const void* wk, const void* wv, int weight_dtype,
                           int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                           const float* bias_k, const float* bias_v, int hidden_dim,
                           int num_heads, int num_kv_heads, int head_dim, int first_position,
                           float* q, float* k, float* v, float* normalized, void* workspace,
                           size_t workspace_bytes, void* stream);
int skv_fused_gate_up_swiglu_gemm_f32(const float* x, int rows, const float* gamma, float epsilon,
                                      const void* w_gate, const void* w_up, int weight_dtype,
                                      int64_t stride_k, int64_t stride_n_gate,
                                      int64_t stride_n_up, const float* bias_gate,
                                      const float* bias_up, int in_dim, int out_dim,
                                      float* act, float* normalized, void* workspace,
                                      size_t workspace_bytes, void* stream);
int skv_linear_residual_gemm_f32(const float* x, int rows, const void* weight, int weight_dtype,
                                 int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                                 const float* bias, const float* residual, float* y,
                                 void* workspace, size_t workspace_bytes, void* stream);
/* The whole feed-forward half of the layer on the library GEMMs:
 * y = x + down(swiglu(gate(n), up(n))) with n = rmsnorm(x, gamma) (written to
 * `normalized`) and the projections' biases; y may alias x.  The SwiGLU
 * epilogue writes the activations straight as the bf16 hi / lo operand of
 * down_proj (no fp32 activation rows): the arithmetic of
 * skv_fused_gate_up_swiglu_gemm_f32 followed by skv_linear_residual_gemm_f32
 * (residual x), equal to it to fp32 rounding (hipBLASLt's kernels for skinny
 * shapes may split K and add the parts in any order).  Workspace: skv_prompt_gemm_workspace_bytes(rows,
 * max(hidden_dim, inter_dim), max(2 * inter_dim, hidden_dim)).  The same
 * SKV_ERR_UNSUPPORTED rules as the separate calls.
 * Replaces: src/models/transformer_block.cpp:310-332 (post-attention norm,
 * gate/up, SwiGLU, down_proj and the residual); no counterpart of its own. */
int skv_ffn_swiglu_gemm_f32(const float* x, int rows, const float* gamma, float epsilon,
                            const void* w_gate, const void* w_up, const void* w_down, int weight_dtype,
                            int64_t stride_k, int64_t stride_n_gate, int64_t stride_n_up,
                            int64_t stride_n_down, const float* bias_gate, const float* bias_up,
                            const float* bias_down, int hidden_dim, int inter_dim, float* y,
                            float* normalized, void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* STRATAKV_AMD_GEMM_H */

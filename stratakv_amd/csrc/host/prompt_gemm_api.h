// prompt_gemm_api.h -- the entry points of libstratakv_amd_gemm.so (the
// hipBLASLt projections of long prompt chunks, stratakv_amd_gemm.h), reached
// through dlopen so that libstratakv_amd.so itself does not link hipBLASLt.
#pragma once

#include "stratakv_amd_gemm.h"

namespace stratakv {
namespace detail {

struct PromptGemmApi {
    decltype(&skv_prompt_gemm_workspace_bytes) workspace_bytes;
    decltype(&skv_fused_qkv_gemm_f32) fused_qkv;
    decltype(&skv_fused_gate_up_swiglu_gemm_f32) fused_gate_up_swiglu;
    decltype(&skv_linear_residual_gemm_f32) linear_residual;
    decltype(&skv_ffn_swiglu_gemm_f32) ffn_swiglu;
};

// The library beside the one holding this code, opened on the first call
// (thread-safe); nullptr when it cannot be opened (not built, or hipBLASLt
// missing), for the rest of the process.
const PromptGemmApi* prompt_gemm_api() noexcept;

}  // namespace detail
}  // namespace stratakv

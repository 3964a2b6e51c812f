// prompt_gemm_api.cpp -- opens libstratakv_amd_gemm.so from the directory of
// the library (or program) this code is part of, and resolves its entry
// points.  No reference counterpart: the reference has no library GEMM path
// (its prompt runs on the CPU, src/models/transformer_block.cpp:300-332).
#include "prompt_gemm_api.h"

#include <dlfcn.h>

#include <mutex>
#include <string>
#include <type_traits>

namespace stratakv {
namespace detail {
namespace {

constexpr const char* kGemmLibrary = "libstratakv_amd_gemm.so";

PromptGemmApi g_api{};
bool g_loaded = false;

void open_library() {
    Dl_info info{};
    if (dladdr(reinterpret_cast<void*>(&prompt_gemm_api), &info) == 0 || info.dli_fname == nullptr) return;
    std::string path(info.dli_fname);
    const std::size_t slash = path.rfind('/');
    path = (slash == std::string::npos ? std::string() : path.substr(0, slash + 1)) + kGemmLibrary;
    void* handle = dlopen(path.c_str(), RTLD_NOW | RTLD_LOCAL);
    if (handle == nullptr) return;
    PromptGemmApi api{};
    bool ok = true;
    auto resolve = [&](auto& fn, const char* name) {
        fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(handle, name));
        ok = ok && fn != nullptr;
    };
    resolve(api.workspace_bytes, "skv_prompt_gemm_workspace_bytes");
    resolve(api.fused_qkv, "skv_fused_qkv_gemm_f32");
    resolve(api.fused_gate_up_swiglu, "skv_fused_gate_up_swiglu_gemm_f32");
    resolve(api.linear_residual, "skv_linear_residual_gemm_f32");
    resolve(api.ffn_swiglu, "skv_ffn_swiglu_gemm_f32");
    if (!ok) {
        dlclose(handle);
        return;
    }
    g_api = api;   // the handle stays open for the process
    g_loaded = true;
}

}  // namespace

const PromptGemmApi* prompt_gemm_api() noexcept {
    static std::once_flag once;
    std::call_once(once, open_library);
    return g_loaded ? &g_api : nullptr;
}

}  // namespace detail
}  // namespace stratakv

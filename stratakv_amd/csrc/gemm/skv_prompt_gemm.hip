// skv_prompt_gemm.hip -- the projections of long prompt chunks with their
// products on hipBLASLt: bf16 weights x bf16 parts of the fp32 inputs, fp32
// accumulation.  The library GEMMs run the multiply-adds; the kernels around
// them (skv_layer_ops.hip, in libstratakv_amd.so) split the inputs and apply
// the layer's epilogue.  Built as its own shared object,
// libstratakv_amd_gemm.so, the only part of the build that links hipBLASLt:
// the append / decode library loads without it, and its host layer opens this
// one on demand (host/prompt_gemm_api.cpp).
//
// Why hi and lo parts: the activations are fp32 and the weights bf16 (the
// reference multiplies fp32 activations by bf16 weights in fp32,
// src/cuda/gemm_cuda.cu:445-560).  Each input v becomes hi = bf16(v) and
// lo = bf16(v - hi); both parts are rounded to bf16, so hi + lo keeps ~16
// significant bits of v (relative error up to ~2^-16, against fp32's 2^-24),
// and every product of a part with a bf16 weight is exact in fp32.  The two
// parts are stacked as 2 * rows GEMM columns, so each weight matrix is one
// GEMM of twice the tokens instead of two.
//
// Layout, column-major as hipBLASLt sees it: a weight matrix of N
// output-major rows with row stride ld is the K x N matrix W^T (op T, lda =
// ld); the parts are K x 2 rows (op N, ldb = K); the output is N x 2 rows
// (ldc = N), i.e. [2 * rows][N] row-major with token r's hi products in row r
// and its lo products in row rows + r.
//
// Algorithm choice: hipBLASLt's heuristic ranks the algorithms of a shape;
// every call takes its first choice.  The choice depends only on the shape,
// the device and the library version, never on timing, so two processes on
// the same device and library compute the same bits.
#include "skv_common.h"
#include "skv_prompt_gemm.h"
#include "stratakv_amd_gemm.h"

#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <tuple>

namespace skv {
namespace {

constexpr size_t kLibWorkspace = size_t{32} << 20;   // hipBLASLt's own scratch, the algorithm search's limit

size_t align256(size_t b) { return (b + 255) & ~size_t{255}; }

// One GEMM shape's descriptors and hipBLASLt's first-ranked algorithm for it.
struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    bool ok = false;
    ~Plan() {
        if (a != nullptr) hipblasLtMatrixLayoutDestroy(a);
        if (b != nullptr) hipblasLtMatrixLayoutDestroy(b);
        if (c != nullptr) hipblasLtMatrixLayoutDestroy(c);
        if (desc != nullptr) hipblasLtMatmulDescDestroy(desc);
    }
};
using PlanPtr = std::shared_ptr<const Plan>;

// Per device: the library handle (created on first use, kept for the process)
// and the plans of the shapes seen.  The plan of a shape holds the token count
// (each new prompt-tail length is a new shape), so the cache is bounded: past
// kMaxPlans shapes it starts afresh.  Callers hold shared pointers, so a plan
// in use outlives its removal from the cache.
constexpr size_t kMaxPlans = 256;
struct DeviceState {
    hipblasLtHandle_t handle = nullptr;
    bool failed = false;
    std::map<std::tuple<int, int, int, int64_t>, PlanPtr> plans;
};

std::mutex g_mutex;
std::map<int, DeviceState> g_devices;

// The plan of an m x n x k GEMM with lda, or nullptr when hipBLASLt has none
// (or cannot start on this device).
PlanPtr plan_for(int m, int n, int k, int64_t lda) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return nullptr;
    std::lock_guard<std::mutex> lock(g_mutex);
    DeviceState& ds = g_devices[dev];
    if (ds.handle == nullptr && !ds.failed && hipblasLtCreate(&ds.handle) != HIPBLAS_STATUS_SUCCESS) {
        ds.handle = nullptr;
        ds.failed = true;
    }
    if (ds.failed) return nullptr;
    const auto key = std::make_tuple(m, n, k, lda);
    auto it = ds.plans.find(key);
    if (it != ds.plans.end()) return it->second->ok ? it->second : nullptr;
    if (ds.plans.size() >= kMaxPlans) ds.plans.clear();
    auto p = std::make_shared<Plan>();
    const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    hipblasLtMatmulPreference_t pref = nullptr;
    bool ok = hipblasLtMatmulDescCreate(&p->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta)) ==
                  HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb)) ==
                  HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p->a, HIP_R_16BF, k, m, lda) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p->b, HIP_R_16BF, k, n, k) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatrixLayoutCreate(&p->c, HIP_R_32F, m, n, m) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS &&
              hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                    &kLibWorkspace, sizeof(kLibWorkspace)) == HIPBLAS_STATUS_SUCCESS;
    if (ok) {
        // The first algorithm of the heuristic's ranking that fits the workspace.
        constexpr int kRanked = 4;
        hipblasLtMatmulHeuristicResult_t found[kRanked];
        int nfound = 0;
        ok = hipblasLtMatmulAlgoGetHeuristic(ds.handle, p->desc, p->a, p->b, p->c, p->c, pref, kRanked, found,
                                             &nfound) == HIPBLAS_STATUS_SUCCESS;
        bool have = false;
        for (int i = 0; ok && !have && i < nfound; ++i)
            if (found[i].state == HIPBLAS_STATUS_SUCCESS && found[i].workspaceSize <= kLibWorkspace) {
                p->algo = found[i].algo;
                have = true;
            }
        ok = ok && have;
    }
    if (pref != nullptr) hipblasLtMatmulPreferenceDestroy(pref);
    p->ok = ok;
    ds.plans.emplace(key, p);
    return ok ? p : nullptr;
}

// The plans of every weight matrix of one call, looked up before anything is
// launched: a shape hipBLASLt does not take leaves the call unlaunched.
struct Gemm {
    const void* w;
    int64_t ld;
    int n;
    float* d;
    PlanPtr plan;
};

// Workspace: [2 rows][K] bf16 parts, then [2 rows][outputs] fp32 GEMM
// outputs, the RoPE table of q/k/v, then the library's scratch.
struct Workspace {
    uint16_t* parts;
    float* out;
    float* rope_cs;
    void* lib;
};

Workspace carve(void* ws, int rows, int K, int outputs) {
    char* p = static_cast<char*>(ws);
    const size_t parts = align256(size_t{4} * rows * K), out = align256(size_t{8} * rows * outputs);
    const size_t rope = align256(size_t{4} * rows * (outputs / 3));
    return Workspace{reinterpret_cast<uint16_t*>(p), reinterpret_cast<float*>(p + parts),
                     reinterpret_cast<float*>(p + parts + out), p + parts + out + rope};
}

int check_workspace(const char* fn, void* ws, size_t bytes, int rows, int K, int outputs) {
    SKV_REQUIRE(ws != nullptr && (reinterpret_cast<std::uintptr_t>(ws) & 255u) == 0,
                "%s: workspace must be 256-byte aligned", fn);
    const size_t need = skv_prompt_gemm_workspace_bytes(rows, K, outputs);
    SKV_REQUIRE(bytes >= need, "%s: workspace of %zu bytes, %zu needed", fn, bytes, need);
    return SKV_OK;
}

// Biases are read 4 at a time by the epilogues.
bool bias_ok(const float* b) { return b == nullptr || aligned16(b); }

// The common layout rules; SKV_ERR_UNSUPPORTED when a shape is not taken.
bool layout_ok(const void* w, int weight_dtype, int64_t stride_k, int64_t stride_n, int K, int n) {
    return w != nullptr && weight_dtype == SKV_DTYPE_BF16 && stride_k == 1 && stride_n >= K &&
           (stride_n * 2) % 16 == 0 && aligned16(w) && n % 8 == 0;
}

// Whether matrix m + 1's rows follow matrix m's in memory with the same
// stride (a packed allocation): then both are one GEMM of their summed width.
bool follows(const void* a, int n_a, int64_t stride_a, const void* b, int64_t stride_b) {
    return stride_a == stride_b &&
           static_cast<const char*>(b) == static_cast<const char*>(a) + 2 * static_cast<int64_t>(n_a) * stride_a;
}

// Plans every GEMM of the call (nothing launched yet).
bool plan_all(Gemm* g, int count, int rows, int K) {
    for (int i = 0; i < count; ++i)
        if ((g[i].plan = plan_for(g[i].n, 2 * rows, K, g[i].ld)) == nullptr) return false;
    return true;
}

int run_gemms(const char* fn, const Gemm* g, int count, const uint16_t* parts, void* lib, hipStream_t s) {
    const float alpha = 1.0f, beta = 0.0f;
    int dev = 0;
    SKV_HIP_TRY(hipGetDevice(&dev));
    hipblasLtHandle_t handle;
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        handle = g_devices[dev].handle;
    }
    for (int i = 0; i < count; ++i) {
        const Plan& p = *g[i].plan;
        const hipblasStatus_t st = hipblasLtMatmul(handle, p.desc, &alpha, g[i].w, p.a, parts, p.b, &beta, g[i].d,
                                                   p.c, g[i].d, p.c, &p.algo, lib, kLibWorkspace, s);
        if (st != HIPBLAS_STATUS_SUCCESS) return set_error(SKV_ERR_HIP, "%s: hipblasLtMatmul failed (%d)", fn, st);
    }
    return check_launch("hipblasLtMatmul");
}

}  // namespace
}  // namespace skv

using namespace skv;

extern "C" size_t skv_prompt_gemm_workspace_bytes(int rows, int in_dim, int outputs) {
    if (rows <= 0 || in_dim <= 0 || outputs <= 0) return 0;
    // + the RoPE table of q/k/v, [rows][head_dim / 2][cos, sin] with head_dim <= outputs / 3.
    return align256(size_t{4} * rows * in_dim) + align256(size_t{8} * rows * outputs) +
           align256(size_t{4} * rows * (outputs / 3)) + kLibWorkspace;
}

extern "C" int skv_fused_qkv_gemm_f32(const float* hidden, int rows, const float* gamma, float epsilon,
                                      const void* wq, const void* wk, const void* wv, int weight_dtype,
                                      int64_t stride_k, const int64_t stride_n[3], const float* bias_q,
                                      const float* bias_k, const float* bias_v, int hidden_dim, int num_heads,
                                      int num_kv_heads, int head_dim, int first_position, float* q, float* k,
                                      float* v, float* normalized, void* workspace, size_t workspace_bytes,
                                      void* stream) {
    const char* fn = "skv_fused_qkv_gemm_f32";
    SKV_REQUIRE(hidden && stride_n && q && k && v && rows > 0 && hidden_dim > 0 && num_heads > 0 &&
                    num_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0,
                "%s: invalid pointers or sizes", fn);
    SKV_REQUIRE(gamma == nullptr || normalized != nullptr, "%s: normalized scratch required with gamma", fn);
    SKV_REQUIRE(head_dim <= 512, "%s: head_dim %d exceeds 512", fn, head_dim);
    const int n[3] = {num_heads * head_dim, num_kv_heads * head_dim, num_kv_heads * head_dim};
    const int K = hidden_dim;
    if (int rc = check_workspace(fn, workspace, workspace_bytes, rows, K, n[0] + n[1] + n[2])) return rc;
    const bool rope = first_position >= 0;
    const void* w[3] = {wq, wk, wv};
    bool ok = K % 8 == 0 && K <= 8192 && (!rope || head_dim % 8 == 0) && aligned16(hidden) && aligned16(q) &&
              aligned16(k) && aligned16(v) && (gamma == nullptr || aligned16(normalized)) && bias_ok(bias_q) &&
              bias_ok(bias_k) && bias_ok(bias_v);
    for (int m = 0; m < 3 && ok; ++m) ok = layout_ok(w[m], weight_dtype, stride_k, stride_n[m], K, n[m]);
    if (!ok) return set_error(SKV_ERR_UNSUPPORTED, "%s: layout not taken by the library GEMMs", fn);
    Workspace ws = carve(workspace, rows, K, n[0] + n[1] + n[2]);
    float* y[3] = {q, k, v};
    // q, k and v rows packed one after another: one GEMM over all three, each
    // matrix's outputs a column range of its [2 rows][q + k + v] result.
    const bool packed = follows(wq, n[0], stride_n[0], wk, stride_n[1]) && follows(wk, n[1], stride_n[1], wv, stride_n[2]);
    Gemm g[3];
    int ngemm = 3;
    const float* dm[3];
    int ldm[3];
    if (packed) {
        ngemm = 1;
        g[0] = Gemm{wq, stride_n[0], n[0] + n[1] + n[2], ws.out, nullptr};
        for (int m = 0, off = 0; m < 3; off += n[m], ++m) {
            dm[m] = ws.out + off;
            ldm[m] = n[0] + n[1] + n[2];
        }
    } else {
        float* d = ws.out;
        for (int m = 0; m < 3; ++m) {
            g[m] = Gemm{w[m], stride_n[m], n[m], d, nullptr};
            dm[m] = d;
            ldm[m] = n[m];
            d += size_t{2} * rows * n[m];
        }
    }
    if (!plan_all(g, ngemm, rows, K)) return set_error(SKV_ERR_UNSUPPORTED, "%s: no hipBLASLt algorithm", fn);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int rc = launch_split_rows(hidden, rows, K, gamma, epsilon, normalized, ws.parts, s,
                                   rope ? ws.rope_cs : nullptr, first_position, head_dim))
        return rc;
    if (int rc = run_gemms(fn, g, ngemm, ws.parts, ws.lib, s)) return rc;
    GemmEpilogue e{};
    const float* bias[3] = {bias_q, bias_k, bias_v};
    for (int m = 0; m < 3; ++m) {
        e.d[m] = dm[m];
        e.ld[m] = ldm[m];
        e.bias[m] = bias[m];
        e.y[m] = y[m];
        e.n[m] = n[m];
    }
    e.rope_cs = ws.rope_cs;
    e.rows = rows;
    e.head_dim = head_dim;
    e.first = first_position;
    return launch_qkv_epilogue(e, s);
}

extern "C" int skv_fused_gate_up_swiglu_gemm_f32(const float* x, int rows, const float* gamma, float epsilon,
                                                 const void* w_gate, const void* w_up, int weight_dtype,
                                                 int64_t stride_k, int64_t stride_n_gate, int64_t stride_n_up,
                                                 const float* bias_gate, const float* bias_up, int in_dim,
                                                 int out_dim, float* act, float* normalized, void* workspace,
                                                 size_t workspace_bytes, void* stream) {
    const char* fn = "skv_fused_gate_up_swiglu_gemm_f32";
    SKV_REQUIRE(x && act && rows > 0 && in_dim > 0 && out_dim > 0, "%s: invalid pointers or sizes", fn);
    SKV_REQUIRE(gamma == nullptr || normalized != nullptr, "%s: normalized scratch required with gamma", fn);
    const int K = in_dim;
    if (int rc = check_workspace(fn, workspace, workspace_bytes, rows, K, 2 * out_dim)) return rc;
    const bool ok = K % 8 == 0 && K <= 8192 && aligned16(x) && aligned16(act) &&
                    (gamma == nullptr || aligned16(normalized)) && bias_ok(bias_gate) && bias_ok(bias_up) &&
                    layout_ok(w_gate, weight_dtype, stride_k, stride_n_gate, K, out_dim) &&
                    layout_ok(w_up, weight_dtype, stride_k, stride_n_up, K, out_dim);
    if (!ok) return set_error(SKV_ERR_UNSUPPORTED, "%s: layout not taken by the library GEMMs", fn);
    Workspace ws = carve(workspace, rows, K, 2 * out_dim);
    // gate and up rows packed one after another: one GEMM of 2 out_dim outputs.
    const bool packed = follows(w_gate, out_dim, stride_n_gate, w_up, stride_n_up);
    Gemm g[2] = {{w_gate, stride_n_gate, out_dim, ws.out, nullptr},
                 {w_up, stride_n_up, out_dim, ws.out + size_t{2} * rows * out_dim, nullptr}};
    if (packed) g[0].n = 2 * out_dim;
    const int ngemm = packed ? 1 : 2;
    if (!plan_all(g, ngemm, rows, K)) return set_error(SKV_ERR_UNSUPPORTED, "%s: no hipBLASLt algorithm", fn);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int rc = launch_split_rows(x, rows, K, gamma, epsilon, normalized, ws.parts, s)) return rc;
    if (int rc = run_gemms(fn, g, ngemm, ws.parts, ws.lib, s)) return rc;
    GemmEpilogue e{};
    e.d[0] = ws.out;
    e.d[1] = packed ? ws.out + out_dim : g[1].d;
    e.ld[0] = e.ld[1] = packed ? 2 * out_dim : out_dim;
    e.bias[0] = bias_gate;
    e.bias[1] = bias_up;
    e.y[0] = act;
    e.n[0] = e.n[1] = out_dim;
    e.rows = rows;
    return launch_gate_up_epilogue(e, s);
}

extern "C" int skv_linear_residual_gemm_f32(const float* x, int rows, const void* weight, int weight_dtype,
                                            int64_t stride_k, int64_t stride_n, int in_dim, int out_dim,
                                            const float* bias, const float* residual, float* y, void* workspace,
                                            size_t workspace_bytes, void* stream) {
    const char* fn = "skv_linear_residual_gemm_f32";
    SKV_REQUIRE(x && residual && y && rows > 0 && in_dim > 0 && out_dim > 0, "%s: invalid pointers or sizes", fn);
    const int K = in_dim;
    if (int rc = check_workspace(fn, workspace, workspace_bytes, rows, K, out_dim)) return rc;
    const bool ok = K % 8 == 0 && K <= 8192 && aligned16(x) && aligned16(residual) && aligned16(y) && bias_ok(bias) &&
                    layout_ok(weight, weight_dtype, stride_k, stride_n, K, out_dim);
    if (!ok) return set_error(SKV_ERR_UNSUPPORTED, "%s: layout not taken by the library GEMMs", fn);
    Workspace ws = carve(workspace, rows, K, out_dim);
    Gemm g[1] = {{weight, stride_n, out_dim, ws.out, nullptr}};
    if (!plan_all(g, 1, rows, K)) return set_error(SKV_ERR_UNSUPPORTED, "%s: no hipBLASLt algorithm", fn);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (int rc = launch_split_rows(x, rows, K, nullptr, 0.0f, nullptr, ws.parts, s)) return rc;
    if (int rc = run_gemms(fn, g, 1, ws.parts, ws.lib, s)) return rc;
    GemmEpilogue e{};
    e.d[0] = g[0].d;
    e.ld[0] = out_dim;
    e.bias[0] = bias;
    e.y[0] = y;
    e.n[0] = out_dim;
    e.residual = residual;
    e.rows = rows;
    return launch_residual_epilogue(e, s);
}

extern "C" int skv_ffn_swiglu_gemm_f32(const float* x, int rows, const float* gamma, float epsilon,
                                       const void* w_gate, const void* w_up, const void* w_down, int weight_dtype,
                                       int64_t stride_k, int64_t stride_n_gate, int64_t stride_n_up,
                                       int64_t stride_n_down, const float* bias_gate, const float* bias_up,
                                       const float* bias_down, int hidden_dim, int inter_dim, float* y,
                                       float* normalized, void* workspace, size_t workspace_bytes, void* stream) {
    const char* fn = "skv_ffn_swiglu_gemm_f32";
    SKV_REQUIRE(x && y && rows > 0 && hidden_dim > 0 && inter_dim > 0, "%s: invalid pointers or sizes", fn);
    SKV_REQUIRE(gamma == nullptr || normalized != nullptr, "%s: normalized scratch required with gamma", fn);
    const int H = hidden_dim, I = inter_dim;
    const int kmax = std::max(H, I), outs = std::max(2 * I, H);
    if (int rc = check_workspace(fn, workspace, workspace_bytes, rows, kmax, outs)) return rc;
    const bool ok = H % 8 == 0 && H <= 8192 && I % 8 == 0 && I <= 8192 && aligned16(x) && aligned16(y) &&
                    (gamma == nullptr || aligned16(normalized)) && bias_ok(bias_gate) && bias_ok(bias_up) &&
                    bias_ok(bias_down) &&
                    layout_ok(w_gate, weight_dtype, stride_k, stride_n_gate, H, I) &&
                    layout_ok(w_up, weight_dtype, stride_k, stride_n_up, H, I) &&
                    layout_ok(w_down, weight_dtype, stride_k, stride_n_down, I, H);
    if (!ok) return set_error(SKV_ERR_UNSUPPORTED, "%s: layout not taken by the library GEMMs", fn);
    Workspace ws = carve(workspace, rows, kmax, outs);
    const bool packed = follows(w_gate, I, stride_n_gate, w_up, stride_n_up);
    Gemm g[3] = {{w_gate, stride_n_gate, packed ? 2 * I : I, ws.out, nullptr},
                 {w_up, stride_n_up, I, ws.out + size_t{2} * rows * I, nullptr},
                 {w_down, stride_n_down, H, ws.out, nullptr}};
    const int ngate = packed ? 1 : 2;
    if (!plan_all(g, ngate, rows, H) || !plan_all(g + 2, 1, rows, I))
        return set_error(SKV_ERR_UNSUPPORTED, "%s: no hipBLASLt algorithm", fn);
    hipStream_t s = static_cast<hipStream_t>(stream);
    // rmsnorm + split of x; gate/up; SwiGLU straight into the split operand
    // of down_proj (the activations never go to memory in fp32); down_proj;
    // + bias + x.  The GEMM outputs reuse one region: each is consumed before
    // the next GEMM writes it.
    if (int rc = launch_split_rows(x, rows, H, gamma, epsilon, normalized, ws.parts, s)) return rc;
    if (int rc = run_gemms(fn, g, ngate, ws.parts, ws.lib, s)) return rc;
    GemmEpilogue a{};
    a.d[0] = ws.out;
    a.d[1] = packed ? ws.out + I : g[1].d;
    a.ld[0] = a.ld[1] = packed ? 2 * I : I;
    a.bias[0] = bias_gate;
    a.bias[1] = bias_up;
    a.n[0] = a.n[1] = I;
    a.parts = ws.parts;
    a.rows = rows;
    if (int rc = launch_gate_up_epilogue(a, s)) return rc;
    if (int rc = run_gemms(fn, g + 2, 1, ws.parts, ws.lib, s)) return rc;
    GemmEpilogue e{};
    e.d[0] = ws.out;
    e.ld[0] = H;
    e.bias[0] = bias_down;
    e.y[0] = y;
    e.n[0] = H;
    e.residual = x;
    e.rows = rows;
    return launch_residual_epilogue(e, s);
}

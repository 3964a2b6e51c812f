// abi_host_stand_in.cpp -- test infrastructure, never part of the product
// library: the C ABI entry points the C++ host layer calls, over host memory,
// so BlockPool / PageTable / DeviceBatch host logic, the safetensors parser and
// Tensor can be built and run under AddressSanitizer and
// UndefinedBehaviorSanitizer in a container without a GPU (build target
// `asan` of stratakv_amd/_build.py).  "Device" memory is malloc'ed, copies are
// memcpy, events and streams complete at once, and the table scatter runs on
// the host.  Every compute entry point returns SKV_ERR_UNSUPPORTED: the
// kernels themselves are covered by the GPU tests.
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>

#include "stratakv_amd.h"

namespace {
thread_local std::string g_error;
constexpr int kWriteI32Max = 16;  // the device entry point carries at most 16 values

int fail(const char* msg, int code = SKV_ERR_INVALID_ARGUMENT) {
    g_error = msg;
    return code;
}

int copy(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return SKV_OK;
    if (!dst || !src) return fail("skv_memcpy: NULL pointer");
    std::memmove(dst, src, bytes);
    return SKV_OK;
}
}  // namespace

extern "C" {

int skv_argmax_at_f32(const float*, int, int32_t*, const int32_t*, int32_t*, const int32_t*, void*) { return fail("skv_argmax_at_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_add_f32(float*, const float*, int, void*) { return fail("skv_add_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }
int skv_fill_normal_bf16(uint16_t*, size_t, uint64_t, uint64_t, void*) { return fail("skv_fill_normal_bf16: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_check_finite(const void*, int, size_t, int32_t*, void*) { return fail("skv_check_finite: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_convert_to_bf16(const void*, int, size_t, uint16_t*, int32_t*, void*) { return fail("skv_convert_to_bf16: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_convert_to_f32(const void*, int, size_t, float*, int32_t*, void*) { return fail("skv_convert_to_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_device_synchronize(void) { return SKV_OK; }

int skv_embedding_at_f32(const void*, int, int, int, const int32_t*, const int32_t*, float*, int32_t*, const int32_t*, void*) { return fail("skv_embedding_at_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_embedding_f32(const void*, int, int, int, const int32_t*, int, float*, int32_t*, void*) { return fail("skv_embedding_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_embedding_rows_f32(const void*, int, int, int, const int32_t*, int, int, float*, int32_t*, void*) { return fail("skv_embedding_rows_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_event_create(void** event) {
    if (!event) return fail("skv_event_create: NULL out pointer");
    *event = new int(0);
    return SKV_OK;
}

int skv_event_destroy(void* event) {
    delete static_cast<int*>(event);
    return SKV_OK;
}

int skv_event_query(void* event, int* done) {
    if (!event || !done) return fail("skv_event_query: NULL argument");
    *done = 1;
    return SKV_OK;
}

int skv_event_record(void* event, void*) { return event ? SKV_OK : fail("skv_event_record: NULL event"); }

int skv_event_synchronize(void* event) { return event ? SKV_OK : fail("skv_event_synchronize: NULL event"); }

int skv_free(void* ptr) {
    std::free(ptr);
    return SKV_OK;
}

int skv_fused_gate_up_swiglu_f32(const float*, const float*, float, const void*, const void*, int, int64_t, int64_t, int64_t, const float*, const float*, int, int, float*, void*) { return fail("skv_fused_gate_up_swiglu_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_fused_gate_up_swiglu_mm_f32(const float*, int, const float*, float, const void*, const void*, int, int64_t, int64_t, int64_t, const float*, const float*, int, int, float*, float*, void*) { return fail("skv_fused_gate_up_swiglu_mm_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_fused_gate_up_swiglu_rows_f32(const float*, int, const float*, float, const void*, const void*, int, int64_t, int64_t, int64_t, const float*, const float*, int, int, float*, float*, void*) { return fail("skv_fused_gate_up_swiglu_rows_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_fused_qkv_at_f32(const float*, const float*, float, const void*, const void*, const void*, int, int64_t, const int64_t*, const float*, const float*, const float*, int, int, int, int, const int32_t*, const float*, int, float*, float*, float*, void*) { return fail("skv_fused_qkv_at_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_graph_abort_capture(void*) { return fail("skv_graph_abort_capture: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_graph_begin_capture(void*) { return fail("skv_graph_begin_capture: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_graph_destroy(void* exec) { return exec ? fail("skv_graph_destroy: no GPU in the host-only build", SKV_ERR_UNSUPPORTED) : SKV_OK; }

int skv_graph_end_capture(void*, void**) { return fail("skv_graph_end_capture: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_graph_launch(void*, void*) { return fail("skv_graph_launch: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_fused_qkv_f32(const float*, const float*, float, const void*, const void*, const void*, int, int64_t, const int64_t*, const float*, const float*, const float*, int, int, int, int, int, float*, float*, float*, void*) { return fail("skv_fused_qkv_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_fused_qkv_mm_f32(const float*, int, const float*, float, const void*, const void*, const void*, int, int64_t, const int64_t*, const float*, const float*, const float*, int, int, int, int, int, float*, float*, float*, float*, void*) { return fail("skv_fused_qkv_mm_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_fused_qkv_rows_f32(const float*, int, const float*, float, const void*, const void*, const void*, int, int64_t, const int64_t*, const float*, const float*, const float*, int, int, int, int, int, float*, float*, float*, float*, void*) { return fail("skv_fused_qkv_rows_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_host_alloc(void** ptr, size_t bytes) {
    if (!ptr) return fail("skv_host_alloc: ptr is NULL");
    *ptr = nullptr;
    if (bytes == 0) return SKV_OK;
    *ptr = std::malloc(bytes);
    return *ptr ? SKV_OK : fail("skv_host_alloc: out of host memory");
}

int skv_host_free(void* ptr) { return skv_free(ptr); }

int skv_kv_append(const void*, const void*, int, uint16_t*, uint16_t*, int64_t, const int32_t*, int, const int32_t*, const int32_t*, int, int, int, int, int, void*) { return fail("skv_kv_append: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

const char* skv_last_error(void) { return g_error.c_str(); }

int skv_linear_f32(const float*, int, const void*, int, int64_t, int64_t, int, int, const float*, float*, void*) { return fail("skv_linear_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_linear_residual_f32(const float*, const void*, int, int64_t, int64_t, int, int, const float*, const float*, float*, void*) { return fail("skv_linear_residual_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_linear_residual_mm_f32(const float*, int, const void*, int, int64_t, int64_t, int, int, const float*, const float*, float*, void*) { return fail("skv_linear_residual_mm_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_linear_residual_rows_f32(const float*, int, const void*, int, int64_t, int64_t, int, int, const float*, const float*, float*, void*) { return fail("skv_linear_residual_rows_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_malloc(void** ptr, size_t bytes) {
    if (!ptr) return fail("skv_malloc: ptr is NULL");
    *ptr = bytes ? std::malloc(bytes) : nullptr;
    return bytes && !*ptr ? fail("skv_malloc: out of host memory") : SKV_OK;
}

int skv_memcpy_d2d(void* dst, const void* src, size_t bytes, void*) { return copy(dst, src, bytes); }

int skv_copy_chunks(const void* const* src, void* const* dst, int count, size_t chunk_bytes, void*) {
    if (count == 0) return SKV_OK;
    if (!src || !dst || count < 0 || chunk_bytes % 16 != 0) return fail("skv_copy_chunks: invalid arguments");
    for (int i = 0; i < count; ++i)
        if (int rc = copy(dst[i], src[i], chunk_bytes)) return rc;
    return SKV_OK;
}

int skv_memcpy_d2h(void* dst, const void* src, size_t bytes, void*) { return copy(dst, src, bytes); }

int skv_memcpy_d2h_async(void* dst, const void* src, size_t bytes, void*) { return copy(dst, src, bytes); }

int skv_memcpy_h2d(void* dst, const void* src, size_t bytes, void*) { return copy(dst, src, bytes); }

int skv_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void*) { return copy(dst, src, bytes); }

int skv_memset_d8(void* dst, int value, size_t bytes, void*) {
    if (bytes == 0) return SKV_OK;
    if (!dst) return fail("skv_memset_d8: NULL pointer");
    std::memset(dst, value, bytes);
    return SKV_OK;
}

int skv_paged_attention_decode_append(const float*, const void*, const void*, int, uint16_t*, uint16_t*, int64_t, const int32_t*, float*, int, int, int, int, int, float, void*, size_t, void*) { return fail("skv_paged_attention_decode_append: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

size_t skv_paged_attention_decode_workspace_bytes(int, int, int) { return 0; }

int skv_paged_decode_append(const void*, int, const void*, const void*, int, uint16_t*, uint16_t*, int64_t, const int32_t*, int, const int32_t*, int, int, int, int, int, float, float*, void*, size_t, void*) { return fail("skv_paged_decode_append: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_paged_prefill(const void*, int, const uint16_t*, const uint16_t*, int64_t, const int32_t*, int, const int32_t*, const int32_t*, int, int, int, int, int, int, float, float*, void*) { return fail("skv_paged_prefill: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_rmsnorm_f32(const float*, float*, const float*, int, int, float, void*) { return fail("skv_rmsnorm_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_rope_cos_sin(int, int, int, float*) { return fail("skv_rope_cos_sin: not in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_rope_f32(float*, int, int, int, void*) { return fail("skv_rope_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_rope_rows_f32(float*, int, int, int, int, void*) { return fail("skv_rope_rows_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_sample_f32(const float*, int, float, int, float, double, int32_t*, int, int32_t*, void*) { return fail("skv_sample_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_scatter_i32(int32_t* dst, const int32_t* pairs, int n, void*) {
    if (n == 0) return SKV_OK;
    if (!dst || !pairs || n < 0) return fail("skv_scatter_i32: invalid arguments");
    for (int i = 0; i < n; ++i) dst[pairs[2 * i]] = pairs[2 * i + 1];
    return SKV_OK;
}

int skv_stream_create(void**) { return fail("skv_stream_create: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_stream_destroy(void* stream) { return stream ? fail("skv_stream_destroy: no GPU in the host-only build", SKV_ERR_UNSUPPORTED) : SKV_OK; }

int skv_stream_synchronize(void*) { return SKV_OK; }

int skv_swiglu_f32(float*, const float*, int, void*) { return fail("skv_swiglu_f32: no GPU in the host-only build", SKV_ERR_UNSUPPORTED); }

int skv_write_i32(int32_t* dst, const int32_t* values, int n, void*) {
    if (n == 0) return SKV_OK;
    if (!dst || !values || n < 0 || n > kWriteI32Max) return fail("skv_write_i32: invalid arguments");
    std::memcpy(dst, values, sizeof(int32_t) * static_cast<size_t>(n));
    return SKV_OK;
}

}  // extern "C"

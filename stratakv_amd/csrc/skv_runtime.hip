// skv_runtime.hip -- error state, device plumbing, synthetic data and test
// support entry points of the C ABI (include/stratakv_amd.h).
#include "skv_common.h"

#include <cmath>
#include <cstdarg>
#include <cstdlib>
#include <cstring>

namespace skv {

namespace {
thread_local std::string g_last_error;
}

int set_error(int code, const char* fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

void clear_error() { g_last_error.clear(); }

bool sync_kernels_enabled() {
    static const bool enabled = [] {
        const char* v = std::getenv("STRATAKV_SYNC_KERNELS");
        return v != nullptr && v[0] == '1';
    }();
    return enabled;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(SKV_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(e));
    if (sync_kernels_enabled()) {
        e = hipDeviceSynchronize();
        if (e != hipSuccess)
            return set_error(SKV_ERR_HIP, "%s failed: %s", what, hipGetErrorString(e));
    }
    return SKV_OK;
}

// ---------------------------------------------------------------------------
// Counter-hash normal generator.  Each element's value depends only on
// (seed, index), so any slice of a pool can be regenerated independently.
// splitmix64 finaliser for mixing, Box-Muller for the normal deviate.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void fill_normal_bf16_kernel(uint16_t* __restrict__ dst, size_t count,
                                        uint64_t seed, uint64_t first, float stddev) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < count; i += stride) {
        const uint64_t h = mix64(seed ^ mix64(first + i));
        const float u1 = (static_cast<float>(static_cast<uint32_t>(h >> 40)) + 1.0f) *
                         (1.0f / 16777216.0f);                      // (0, 1]
        const float u2 = static_cast<float>(static_cast<uint32_t>(h & 0xFFFFFFu)) *
                         (1.0f / 16777216.0f);                      // [0, 1)
        const float r = sqrtf(-2.0f * logf(u1));
        const float z = r * cospif(2.0f * u2);
        dst[i] = static_cast<uint16_t>(f32_to_bf16_bits(z * stddev));
    }
}

__global__ void fill_u16_kernel(uint16_t* __restrict__ dst, size_t count, uint16_t value) {
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < count; i += stride)
        dst[i] = value;
}

// Gather whole blocks listed in a table into a contiguous buffer.
__global__ void gather_blocks_kernel(const uint16_t* __restrict__ pool, int64_t total_blocks,
                                     const int32_t* __restrict__ table, int num_blocks,
                                     int64_t block_elems, uint16_t* __restrict__ dst) {
    const int i = blockIdx.y;
    const int64_t pb = table[i];
    const bool ok = pb >= 0 && pb < total_blocks;
    uint16_t* out = dst + static_cast<int64_t>(i) * block_elems;
    const uint16_t* in = pool + pb * block_elems;
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         e < block_elems; e += static_cast<int64_t>(gridDim.x) * blockDim.x)
        out[e] = ok ? in[e] : uint16_t(0);
}

// Chunk i: bytes [0, chunk_bytes) of src[i] to dst[i] (16-byte aligned, a
// multiple of 16 bytes); one workgroup per chunk (the y dimension) and slice.
__global__ __launch_bounds__(256) void copy_chunks_kernel(const void* const* __restrict__ src,
                                                          void* const* __restrict__ dst, int64_t chunk16) {
    const uint4* in = static_cast<const uint4*>(src[blockIdx.y]);
    uint4* out = static_cast<uint4*>(dst[blockIdx.y]);
    for (int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; e < chunk16;
         e += static_cast<int64_t>(gridDim.x) * blockDim.x)
        out[e] = in[e];
}

// Up to kWriteI32Max int32 values carried in the kernel arguments (copied at
// launch, so the caller's host array is free as soon as the call returns).
constexpr int kWriteI32Max = 16;
struct SmallI32 {
    int32_t x[kWriteI32Max];
};

__global__ void write_i32_kernel(int32_t* __restrict__ dst, SmallI32 v, int n) {
    if (static_cast<int>(threadIdx.x) < n) dst[threadIdx.x] = v.x[threadIdx.x];
}

__global__ void scatter_i32_kernel(int32_t* __restrict__ dst, const int32_t* __restrict__ pairs,
                                   int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[pairs[2 * i]] = pairs[2 * i + 1];
}

// Streaming read of one contiguous buffer, a measurement of the rate plain
// reads reach: a persistent grid whose wavefronts take consecutive 4 MiB
// chunks in turn, with kReadUnroll non-temporal 16-byte loads per lane in
// flight.  *sum (zeroed by the caller) receives the wrapping sum of the
// buffer's 32-bit words, so no load can be dropped; one atomic per wavefront.
constexpr int kReadUnroll = 8;
constexpr int64_t kReadChunk16 = (int64_t{4} << 20) / 16;   // 16-byte units per chunk
constexpr int kReadMaxGroups = 1024;

__global__ __launch_bounds__(256) void stream_read_kernel(const uint4* __restrict__ p, int64_t n16,
                                                          uint32_t* __restrict__ sum) {
    typedef uint32_t u32x4s_t __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63;
    const int64_t wave = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) >> 6;
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * 4;
    uint32_t acc = 0;
    for (int64_t c = wave * kReadChunk16; c < n16; c += nwaves * kReadChunk16) {
        const int64_t end = c + kReadChunk16 < n16 ? c + kReadChunk16 : n16;
        for (int64_t i = c + lane; i < end; i += 64 * kReadUnroll) {
            u32x4s_t v[kReadUnroll];
#pragma unroll
            for (int u = 0; u < kReadUnroll; ++u) {
                const int64_t k = i + 64 * u < end ? i + 64 * u : end - 1;   // in bounds; not summed
                v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4s_t*>(p + k));
            }
#pragma unroll
            for (int u = 0; u < kReadUnroll; ++u)
                acc += i + 64 * u < end ? (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]) : 0u;
        }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, 64);
    if (lane == 0) atomicAdd(sum, acc);
}

}  // namespace skv

using namespace skv;

extern "C" {

const char* skv_last_error(void) { return g_last_error.c_str(); }

int skv_abi_version(void) { return 1; }

int skv_device_count(int* count) {
    SKV_REQUIRE(count != nullptr, "skv_device_count: count is NULL");
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess) n = 0;
    *count = n;
    return SKV_OK;
}

int skv_set_device(int device) {
    SKV_HIP_TRY(hipSetDevice(device));
    return SKV_OK;
}

int skv_malloc(void** ptr, size_t bytes) {
    SKV_REQUIRE(ptr != nullptr, "skv_malloc: ptr is NULL");
    *ptr = nullptr;
    if (bytes == 0) return SKV_OK;
    SKV_HIP_TRY(hipMalloc(ptr, bytes));
    return SKV_OK;
}

int skv_free(void* ptr) {
    if (ptr != nullptr) SKV_HIP_TRY(hipFree(ptr));
    return SKV_OK;
}

int skv_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return SKV_OK;
    SKV_REQUIRE(dst && src, "skv_memcpy_h2d: NULL pointer");
    SKV_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice,
                               static_cast<hipStream_t>(stream)));
    SKV_HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return SKV_OK;
    SKV_REQUIRE(dst && src, "skv_memcpy_d2h: NULL pointer");
    SKV_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost,
                               static_cast<hipStream_t>(stream)));
    SKV_HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return SKV_OK;
    SKV_REQUIRE(dst && src, "skv_memcpy_d2d: NULL pointer");
    SKV_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice,
                               static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_memset_d8(void* dst, int value, size_t bytes, void* stream) {
    if (bytes == 0) return SKV_OK;
    SKV_REQUIRE(dst != nullptr, "skv_memset_d8: NULL pointer");
    SKV_HIP_TRY(hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_stream_create(void** stream) {
    SKV_REQUIRE(stream != nullptr, "skv_stream_create: NULL out pointer");
    hipStream_t s = nullptr;
    SKV_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return SKV_OK;
}

int skv_stream_destroy(void* stream) {
    if (stream != nullptr) SKV_HIP_TRY(hipStreamDestroy(static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_stream_synchronize(void* stream) {
    SKV_HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_device_synchronize(void) {
    SKV_HIP_TRY(hipDeviceSynchronize());
    return SKV_OK;
}

int skv_event_create(void** event) {
    SKV_REQUIRE(event != nullptr, "skv_event_create: NULL out pointer");
    hipEvent_t e = nullptr;
    SKV_HIP_TRY(hipEventCreate(&e));
    *event = e;
    return SKV_OK;
}

int skv_event_destroy(void* event) {
    if (event != nullptr) SKV_HIP_TRY(hipEventDestroy(static_cast<hipEvent_t>(event)));
    return SKV_OK;
}

int skv_event_record(void* event, void* stream) {
    SKV_REQUIRE(event != nullptr, "skv_event_record: NULL event");
    SKV_HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_event_synchronize(void* event) {
    SKV_REQUIRE(event != nullptr, "skv_event_synchronize: NULL event");
    SKV_HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(event)));
    return SKV_OK;
}

int skv_event_query(void* event, int* done) {
    SKV_REQUIRE(event != nullptr && done != nullptr, "skv_event_query: NULL argument");
    const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
    if (e == hipErrorNotReady) {
        *done = 0;
        return SKV_OK;
    }
    SKV_HIP_TRY(e);
    *done = 1;
    return SKV_OK;
}

int skv_host_alloc(void** ptr, size_t bytes) {
    SKV_REQUIRE(ptr != nullptr, "skv_host_alloc: ptr is NULL");
    *ptr = nullptr;
    if (bytes == 0) return SKV_OK;
    SKV_HIP_TRY(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
    return SKV_OK;
}

int skv_host_free(void* ptr) {
    if (ptr != nullptr) SKV_HIP_TRY(hipHostFree(ptr));
    return SKV_OK;
}

int skv_memcpy_h2d_async(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return SKV_OK;
    SKV_REQUIRE(dst && src, "skv_memcpy_h2d_async: NULL pointer");
    SKV_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice,
                               static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_memcpy_d2h_async(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return SKV_OK;
    SKV_REQUIRE(dst && src, "skv_memcpy_d2h_async: NULL pointer");
    SKV_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost,
                               static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_scatter_i32(int32_t* dst, const int32_t* pairs, int n, void* stream) {
    if (n == 0) return SKV_OK;
    SKV_REQUIRE(dst && pairs && n > 0, "skv_scatter_i32: invalid arguments");
    scatter_i32_kernel<<<cdiv(n, 256), 256, 0, static_cast<hipStream_t>(stream)>>>(dst, pairs, n);
    return check_launch("scatter_i32_kernel");
}

int skv_write_i32(int32_t* dst, const int32_t* values, int n, void* stream) {
    if (n == 0) return SKV_OK;
    SKV_REQUIRE(dst && values && n > 0 && n <= kWriteI32Max, "skv_write_i32: invalid arguments (n <= %d)",
                kWriteI32Max);
    SmallI32 v{};
    for (int i = 0; i < n; ++i) v.x[i] = values[i];
    write_i32_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(dst, v, n);
    return check_launch("write_i32_kernel");
}

int skv_event_elapsed_ms(float* ms, void* start, void* stop) {
    SKV_REQUIRE(ms && start && stop, "skv_event_elapsed_ms: NULL argument");
    SKV_HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(stop)));
    SKV_HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                    static_cast<hipEvent_t>(stop)));
    return SKV_OK;
}

int skv_fill_normal_bf16(uint16_t* dst, size_t count, uint64_t seed, uint64_t first_index,
                         void* stream) {
    if (count == 0) return SKV_OK;
    SKV_REQUIRE(dst != nullptr, "skv_fill_normal_bf16: NULL destination");
    const unsigned grid = static_cast<unsigned>(std::min<size_t>(cdiv<size_t>(count, 256), 16384));
    fill_normal_bf16_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
        dst, count, seed, first_index, 1.0f);
    return check_launch("fill_normal_bf16_kernel");
}

int skv_fill_normal_scaled_bf16(uint16_t* dst, size_t count, uint64_t seed, uint64_t first_index,
                                float stddev, void* stream) {
    if (count == 0) return SKV_OK;
    SKV_REQUIRE(dst != nullptr, "skv_fill_normal_scaled_bf16: NULL destination");
    SKV_REQUIRE(std::isfinite(stddev), "skv_fill_normal_scaled_bf16: stddev must be finite");
    const unsigned grid = static_cast<unsigned>(std::min<size_t>(cdiv<size_t>(count, 256), 16384));
    fill_normal_bf16_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(
        dst, count, seed, first_index, stddev);
    return check_launch("fill_normal_bf16_kernel");
}

int skv_fill_u16(uint16_t* dst, size_t count, uint16_t value, void* stream) {
    if (count == 0) return SKV_OK;
    SKV_REQUIRE(dst != nullptr, "skv_fill_u16: NULL destination");
    const unsigned grid = static_cast<unsigned>(std::min<size_t>(cdiv<size_t>(count, 256), 16384));
    fill_u16_kernel<<<grid, 256, 0, static_cast<hipStream_t>(stream)>>>(dst, count, value);
    return check_launch("fill_u16_kernel");
}

int skv_gather_blocks(const uint16_t* pool, int64_t total_blocks, const int32_t* table,
                      int num_blocks, int64_t block_elems, uint16_t* dst, void* stream) {
    if (num_blocks == 0) return SKV_OK;
    SKV_REQUIRE(pool && table && dst, "skv_gather_blocks: NULL pointer");
    SKV_REQUIRE(num_blocks > 0 && num_blocks <= 65535 && block_elems > 0 && total_blocks > 0,
                "skv_gather_blocks: invalid sizes (num_blocks=%d, block_elems=%lld)",
                num_blocks, static_cast<long long>(block_elems));
    const unsigned gx = static_cast<unsigned>(std::min<int64_t>(cdiv<int64_t>(block_elems, 256), 64));
    gather_blocks_kernel<<<dim3(gx, num_blocks), 256, 0, static_cast<hipStream_t>(stream)>>>(
        pool, total_blocks, table, num_blocks, block_elems, dst);
    return check_launch("gather_blocks_kernel");
}

int skv_copy_chunks(const void* const* src, void* const* dst, int count, size_t chunk_bytes, void* stream) {
    if (count == 0) return SKV_OK;
    SKV_REQUIRE(src && dst, "skv_copy_chunks: NULL pointer array");
    SKV_REQUIRE(count > 0 && count <= 65535 && chunk_bytes > 0 && chunk_bytes % 16 == 0,
                "skv_copy_chunks: invalid sizes (count=%d, chunk_bytes=%zu)", count, chunk_bytes);
    const int64_t chunk16 = static_cast<int64_t>(chunk_bytes / 16);
    const unsigned gx = static_cast<unsigned>(std::min<int64_t>(cdiv<int64_t>(chunk16, 256), 64));
    copy_chunks_kernel<<<dim3(gx, static_cast<unsigned>(count)), 256, 0, static_cast<hipStream_t>(stream)>>>(
        src, dst, chunk16);
    return check_launch("copy_chunks_kernel");
}

int skv_graph_begin_capture(void* stream) {
    SKV_REQUIRE(stream != nullptr, "skv_graph_begin_capture: capture needs a created stream, not the null stream");
    SKV_HIP_TRY(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal));
    return SKV_OK;
}

int skv_graph_end_capture(void* stream, void** graph_exec) {
    SKV_REQUIRE(stream && graph_exec, "skv_graph_end_capture: NULL argument");
    *graph_exec = nullptr;
    hipGraph_t g = nullptr;
    SKV_HIP_TRY(hipStreamEndCapture(static_cast<hipStream_t>(stream), &g));
    hipGraphExec_t e = nullptr;
    const hipError_t rc = hipGraphInstantiate(&e, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (rc != hipSuccess)
        return set_error(SKV_ERR_HIP, "skv_graph_end_capture: hipGraphInstantiate: %s", hipGetErrorString(rc));
    *graph_exec = e;
    return SKV_OK;
}

int skv_graph_abort_capture(void* stream) {
    SKV_REQUIRE(stream != nullptr, "skv_graph_abort_capture: NULL stream");
    hipGraph_t g = nullptr;
    const hipError_t rc = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g);
    if (g != nullptr) (void)hipGraphDestroy(g);
    (void)hipGetLastError();   // an invalidated capture reports its error here; it is discarded with the graph
    return rc == hipSuccess || rc == hipErrorStreamCaptureInvalidated ? SKV_OK
                                                                       : set_error(SKV_ERR_HIP,
                                                                                   "skv_graph_abort_capture: %s",
                                                                                   hipGetErrorString(rc));
}

int skv_graph_launch(void* graph_exec, void* stream) {
    SKV_REQUIRE(graph_exec != nullptr, "skv_graph_launch: NULL graph");
    SKV_HIP_TRY(hipGraphLaunch(static_cast<hipGraphExec_t>(graph_exec), static_cast<hipStream_t>(stream)));
    return SKV_OK;
}

int skv_graph_destroy(void* graph_exec) {
    if (graph_exec == nullptr) return SKV_OK;
    SKV_HIP_TRY(hipGraphExecDestroy(static_cast<hipGraphExec_t>(graph_exec)));
    return SKV_OK;
}

int skv_stream_read_checksum(const void* data, int64_t bytes, uint32_t* checksum, void* stream) {
    SKV_REQUIRE(data && checksum, "skv_stream_read_checksum: NULL pointer");
    SKV_REQUIRE(bytes > 0 && bytes % 16 == 0 && aligned16(data),
                "skv_stream_read_checksum: the buffer must be 16-byte aligned, of a positive multiple of 16 "
                "bytes (got %lld)", static_cast<long long>(bytes));
    hipStream_t s = static_cast<hipStream_t>(stream);
    SKV_HIP_TRY(hipMemsetAsync(checksum, 0, sizeof(uint32_t), s));
    const int64_t n16 = bytes / 16;
    const int64_t chunks = cdiv<int64_t>(n16, kReadChunk16);
    const unsigned grid = static_cast<unsigned>(std::min<int64_t>(cdiv<int64_t>(chunks, 4), kReadMaxGroups));
    stream_read_kernel<<<grid, 256, 0, s>>>(static_cast<const uint4*>(data), n16, checksum);
    return check_launch("stream_read_kernel");
}

}  // extern "C"

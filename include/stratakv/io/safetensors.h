// safetensors.h -- checkpoint loading.
//
// Interface of the reference's stratakv::io loader
// (include/stratakv/io/safetensors.h:7-29, src/io/safetensors.cpp:237-681):
// the same header validation (UTF-8, the strict JSON schema, dtypes F32 / F16 /
// BF16 / "bfloat16", contiguous byte ranges covering the payload) with the same
// `std::runtime_error("safetensors: ...")` messages.
//
// Two loaders share that parser:
// * load_safetensors(path): the reference's host API.  Every tensor is
//   materialised as host FP32 (BF16 and F16 widened exactly); 64-byte-aligned
//   F32 norm tensors alias the mapping.
// * load_safetensors_device(path): the MI355X path.  File bytes are read into
//   page-locked staging buffers by several threads and copied to HBM while the
//   next chunk is read; BF16 tensors land as BF16 device tensors (their exact
//   values), F32 as FP32, and F16 is widened to FP32 on the device.  Nothing is
//   converted on the host.
#pragma once

#include <cstddef>
#include <filesystem>
#include <string>
#include <unordered_map>

#include "stratakv/tensor.h"

namespace stratakv {
namespace io {

using WeightMap = std::unordered_map<std::string, Tensor>;

struct LoadBreakdown {
    double mmap_open_ms = 0.0;
    double header_parse_ms = 0.0;
    double tensor_decode_ms = 0.0;  // device loader: file read + transfer + widening
    std::size_t payload_bytes = 0;  // bytes of tensor data read from the file
};

// Host FP32 tensors (reference behaviour).  require_mapped_f32 rejects F32
// tensors that cannot alias the mapping.
WeightMap load_safetensors(const std::filesystem::path& path, bool require_mapped_f32 = false);

// Device tensors in their exact values: BF16 -> BF16, F32 -> FP32, F16 -> FP32.
// All device work is queued on `stream` (a hipStream_t; nullptr = default
// stream) and complete when the call returns.
WeightMap load_safetensors_device(const std::filesystem::path& path, void* stream = nullptr);

// Timings of the last load_safetensors / load_safetensors_device call on any thread.
LoadBreakdown last_load_breakdown() noexcept;

// Host [out_features, in_features] BF16 or FP32 tensor -> [in_features,
// out_features] BF16 (FP32 truncated to its upper 16 bits), the reference's
// GEMM-ready linear layout.
Tensor load_linear_bf16_transposed(const Tensor& source, std::size_t out_features,
                                   std::size_t in_features);

}  // namespace io
}  // namespace stratakv

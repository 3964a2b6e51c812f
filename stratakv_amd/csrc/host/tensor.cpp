// tensor.cpp -- Tensor storage over the C ABI (device) or aligned host memory.
#include "stratakv/tensor.h"

#include <cstdlib>
#include <cstring>
#include <new>
#include <stdexcept>
#include <string>
#include <utility>

#include "abi_check.h"

namespace stratakv {
namespace {

void release_host(void* p) noexcept { std::free(p); }
void release_device(void* p) noexcept { (void)skv_free(p); }

// bf16 -> fp32 is exact: the two stored bytes become the high half.
float widen_bf16(std::uint16_t h) {
    const std::uint32_t bits = static_cast<std::uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &bits, sizeof f);
    return f;
}

// Round to nearest, ties to even on the raw bits (no NaN special case), the
// reference's Tensor::set_value rule.
std::uint16_t narrow_bf16(float value) {
    std::uint32_t bits;
    std::memcpy(&bits, &value, sizeof bits);
    std::uint32_t upper = bits >> 16u;
    const std::uint32_t lower = bits & 0xffffu;
    if (lower > 0x8000u || (lower == 0x8000u && (upper & 1u) != 0u)) ++upper;
    return static_cast<std::uint16_t>(upper & 0xffffu);
}

}  // namespace

Tensor::Tensor(const std::vector<std::size_t>& shape, DataType dtype, Device device)
    : device_(device), dtype_(dtype), shape_(shape) {
    compute_strides();
    const std::size_t bytes = (total_elements_ > 0 ? total_elements_ : 1) * element_size();
    if (device_ == Device::GPU) {
        void* p = nullptr;
        detail::check(skv_malloc(&p, bytes), "Tensor: device allocation");
        owner_ = std::shared_ptr<void>(p, release_device);
        data_ptr_ = p;
        detail::check(skv_memset_d8(p, 0, bytes, nullptr), "Tensor: device zero fill");
        detail::check(skv_stream_synchronize(nullptr), "Tensor: device zero fill");
        return;
    }
    // calloc hands large blocks out as fresh zero pages (nothing is touched
    // until used); the data pointer is rounded up to 64 bytes.
    void* raw = std::calloc(bytes + 64, 1);
    if (raw == nullptr) throw std::bad_alloc();
    owner_ = std::shared_ptr<void>(raw, release_host);
    data_ptr_ = reinterpret_cast<void*>((reinterpret_cast<std::uintptr_t>(raw) + 63) & ~std::uintptr_t{63});
}

Tensor::Tensor(Tensor&& other) noexcept
    : data_ptr_(std::exchange(other.data_ptr_, nullptr)),
      device_(other.device_),
      dtype_(other.dtype_),
      total_elements_(std::exchange(other.total_elements_, 0)),
      shape_(std::move(other.shape_)),
      strides_(std::move(other.strides_)),
      owner_(std::move(other.owner_)) {}

Tensor& Tensor::operator=(Tensor&& other) noexcept {
    if (this != &other) {
        owner_ = std::move(other.owner_);
        data_ptr_ = std::exchange(other.data_ptr_, nullptr);
        device_ = other.device_;
        dtype_ = other.dtype_;
        total_elements_ = std::exchange(other.total_elements_, 0);
        shape_ = std::move(other.shape_);
        strides_ = std::move(other.strides_);
    }
    return *this;
}

Tensor::Tensor(const Tensor& source, AliasTag)
    : data_ptr_(source.data_ptr_),
      device_(source.device_),
      dtype_(source.dtype_),
      total_elements_(source.total_elements_),
      shape_(source.shape_),
      strides_(source.strides_),
      owner_(source.owner_) {}

Tensor Tensor::from_external(const std::vector<std::size_t>& shape, float* data,
                             std::shared_ptr<void> owner) {
    if (!owner || data == nullptr || reinterpret_cast<std::uintptr_t>(data) % 64 != 0)
        throw std::invalid_argument("Tensor: invalid owner or unaligned alias");
    return from_external_bytes(shape, data, std::move(owner), DataType::FP32);
}

Tensor Tensor::from_external_bytes(const std::vector<std::size_t>& shape, void* data,
                                   std::shared_ptr<void> owner, DataType dtype) {
    if (!owner || data == nullptr) throw std::invalid_argument("Tensor: invalid owner or null alias");
    if (dtype == DataType::FP32 && reinterpret_cast<std::uintptr_t>(data) % 64 != 0)
        throw std::invalid_argument("Tensor: unaligned FP32 alias");
    Tensor t({0}, dtype, Device::CPU);
    t.shape_ = shape;
    t.compute_strides();
    t.data_ptr_ = data;
    t.owner_ = std::move(owner);
    return t;
}

void Tensor::compute_strides() {
    strides_.assign(shape_.size(), 1);
    std::size_t n = 1;
    for (std::size_t i = shape_.size(); i-- > 0;) {
        strides_[i] = n;
        n *= shape_[i];
    }
    total_elements_ = shape_.empty() ? 0 : n;
}

Tensor Tensor::to(Device target) const {
    Tensor result(shape_, dtype_, target);
    result.strides_ = strides_;  // physical buffer and its layout
    const std::size_t bytes = total_elements_ * element_size();
    if (bytes == 0) return result;
    if (device_ == Device::CPU && target == Device::CPU) {
        std::memcpy(result.raw_data(), data_ptr_, bytes);
    } else if (device_ == Device::CPU) {
        detail::check(skv_memcpy_h2d(result.raw_data(), data_ptr_, bytes, nullptr), "Tensor::to(GPU)");
    } else if (target == Device::CPU) {
        detail::check(skv_memcpy_d2h(result.raw_data(), data_ptr_, bytes, nullptr), "Tensor::to(CPU)");
    } else {
        detail::check(skv_memcpy_d2d(result.raw_data(), data_ptr_, bytes, nullptr), "Tensor::to(GPU)");
        detail::check(skv_stream_synchronize(nullptr), "Tensor::to(GPU)");
    }
    return result;
}

Tensor Tensor::transpose_2d() const {
    if (ndim() != 2 || dtype_ != DataType::BF16 || !owner_)
        throw std::invalid_argument("Tensor::transpose_2d: expected a BF16 matrix");
    Tensor view(*this, AliasTag{});
    std::swap(view.shape_[0], view.shape_[1]);
    std::swap(view.strides_[0], view.strides_[1]);
    return view;
}

Tensor Tensor::rows_view(std::size_t first, std::size_t count) const {
    if (ndim() != 2 || !is_contiguous() || !owner_ || count == 0 || first > shape_[0] || count > shape_[0] - first)
        throw std::invalid_argument("Tensor::rows_view: expected rows of a contiguous matrix");
    Tensor view(*this, AliasTag{});
    view.data_ptr_ = static_cast<char*>(data_ptr_) + first * shape_[1] * element_size();
    view.shape_[0] = count;
    view.total_elements_ = count * shape_[1];
    return view;
}

std::size_t Tensor::storage_index(std::size_t i) const noexcept {
    if (is_contiguous()) return i;
    return (i / shape_[1]) * strides_[0] + (i % shape_[1]) * strides_[1];
}

std::size_t Tensor::get_flat_index(const std::vector<std::size_t>& idx) const {
    if (idx.size() != shape_.size()) throw std::invalid_argument("Tensor: index rank mismatch");
    std::size_t flat = 0;
    for (std::size_t i = 0; i < idx.size(); ++i) {
        if (idx[i] >= shape_[i])
            throw std::out_of_range("Tensor: index at dimension " + std::to_string(i));
        flat = flat * shape_[i] + idx[i];
    }
    return flat;
}

float Tensor::value_at(std::size_t i) const {
    if (device_ != Device::CPU) throw std::runtime_error("Tensor: GPU tensor requires to(Device::CPU)");
    i = storage_index(i);
    if (dtype_ == DataType::FP32) return static_cast<const float*>(data_ptr_)[i];
    return widen_bf16(static_cast<const std::uint16_t*>(data_ptr_)[i]);
}

void Tensor::set_value(std::size_t i, float value) {
    if (device_ != Device::CPU) throw std::runtime_error("Tensor: GPU tensor requires to(Device::CPU)");
    i = storage_index(i);
    if (dtype_ == DataType::FP32) {
        static_cast<float*>(data_ptr_)[i] = value;
        return;
    }
    static_cast<std::uint16_t*>(data_ptr_)[i] = narrow_bf16(value);
}

}  // namespace stratakv

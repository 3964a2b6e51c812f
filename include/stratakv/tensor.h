// tensor.h -- minimal device/host tensor for the C++ host layer.
//
// Same names, constructors and accessors as the reference's Tensor
// (include/stratakv/tensor.h of StrataKV) so TransformerBlock::forward_into
// callers compile unchanged.  Device storage is allocated through the C ABI
// (skv_malloc) and zero-filled like the reference's device tensors
// (src/cpu/tensor.cpp:60-69); host storage is 64-byte aligned and zeroed.
// BF16 element access uses the reference's exact widen / round-to-nearest-even
// narrow (src/cpu/tensor.cpp:193-229).
#pragma once

#include <cstddef>
#include <cstdint>
#include <memory>
#include <vector>

namespace stratakv {

enum class Device {
    CPU,
    GPU,
};

enum class DataType {
    FP32,
    BF16,
};

class Tensor {
public:
    explicit Tensor(const std::vector<std::size_t>& shape, DataType dtype = DataType::FP32,
                    Device device = Device::CPU);
    explicit Tensor(const std::vector<std::size_t>& shape, Device device)
        : Tensor(shape, DataType::FP32, device) {}
    ~Tensor() = default;
    Tensor(const Tensor&) = delete;
    Tensor& operator=(const Tensor&) = delete;
    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(Tensor&& other) noexcept;

    // Alias external host memory kept alive by `owner` (64-byte aligned for FP32).
    static Tensor from_external(const std::vector<std::size_t>& shape, float* data,
                                std::shared_ptr<void> owner);
    static Tensor from_external_bytes(const std::vector<std::size_t>& shape, void* data,
                                      std::shared_ptr<void> owner, DataType dtype);

    Device device() const noexcept { return device_; }
    // Owning deep copy on `target`, preserving strides (the physical layout).
    Tensor to(Device target) const;
    // Shared-storage BF16 matrix transpose view (logical [K, N] over [N, K] rows).
    Tensor transpose_2d() const;
    // Shared-storage view of rows [first, first + count) of a contiguous 2-D
    // tensor (the projections of one layer packed in one allocation).  No
    // counterpart in the reference.
    Tensor rows_view(std::size_t first, std::size_t count) const;
    bool is_contiguous() const noexcept {
        return ndim() != 2 || (strides_[0] == shape_[1] && strides_[1] == 1);
    }
    DataType dtype() const noexcept { return dtype_; }
    std::size_t element_size() const noexcept {
        return dtype_ == DataType::BF16 ? sizeof(std::uint16_t) : sizeof(float);
    }
    // Only for contiguous CPU FP32 tensors; nullptr otherwise.
    float* data() noexcept {
        return device_ == Device::CPU && dtype_ == DataType::FP32 && is_contiguous()
                   ? static_cast<float*>(data_ptr_) : nullptr;
    }
    const float* data() const noexcept {
        return device_ == Device::CPU && dtype_ == DataType::FP32 && is_contiguous()
                   ? static_cast<const float*>(data_ptr_) : nullptr;
    }
    void* raw_data() noexcept { return data_ptr_; }
    const void* raw_data() const noexcept { return data_ptr_; }
    std::size_t num_elements() const noexcept { return total_elements_; }
    const std::vector<std::size_t>& shape() const noexcept { return shape_; }
    const std::vector<std::size_t>& strides() const noexcept { return strides_; }
    std::size_t ndim() const noexcept { return shape_.size(); }
    std::size_t get_flat_index(const std::vector<std::size_t>& idx) const;

    class ElementProxy {
    public:
        ElementProxy(Tensor& tensor, std::size_t index) noexcept : tensor_(&tensor), index_(index) {}
        operator float() const { return tensor_->value_at(index_); }
        ElementProxy& operator=(float value) {
            tensor_->set_value(index_, value);
            return *this;
        }
        ElementProxy& operator=(const ElementProxy& other) { return *this = static_cast<float>(other); }

    private:
        Tensor* tensor_;
        std::size_t index_;
    };

    ElementProxy operator[](std::size_t i) noexcept { return ElementProxy(*this, i); }
    float operator[](std::size_t i) const { return value_at(i); }
    float value_at(std::size_t i) const;

private:
    struct AliasTag {};
    Tensor(const Tensor& source, AliasTag);
    void compute_strides();
    std::size_t storage_index(std::size_t logical_index) const noexcept;
    void set_value(std::size_t i, float value);

    void* data_ptr_ = nullptr;
    Device device_ = Device::CPU;
    DataType dtype_ = DataType::FP32;
    std::size_t total_elements_ = 0;
    std::vector<std::size_t> shape_;
    std::vector<std::size_t> strides_;
    std::shared_ptr<void> owner_;
};

}  // namespace stratakv

#pragma once

// sci::Tensor: a contiguous, typed buffer on one device.
// Same API shape as SciComputeInfra's tensor/tensor.hpp (reference stub/include/tensor/tensor.hpp:16-94):
// owning (allocates on construction, frees on destruction) or non-owning (wraps external memory);
// move-only. copy_from moves bytes across devices (host <-> GPU, GPU <-> GPU).

#include <cstddef>
#include <string>

#include "core/status.hpp"
#include "core/types.hpp"
#include "device/device.hpp"

namespace sci {

class SCI_INFRA_API Tensor {
public:
    Tensor() = default;
    Tensor(const TensorShape& shape, DType dtype, Device& device);
    Tensor(const TensorShape& shape, DType dtype, Device& device, void* external_data,
           bool owns_data = false);
    ~Tensor();

    Tensor(Tensor&& other) noexcept;
    Tensor& operator=(Tensor&& other) noexcept;
    Tensor(const Tensor&) = delete;
    Tensor& operator=(const Tensor&) = delete;

    const TensorShape& shape() const { return shape_; }
    index_t ndims() const { return shape_.ndims(); }
    index_t dim(size_t i) const { return shape_.dim(i); }
    index_t num_elements() const { return shape_.num_elements(); }
    DType dtype() const { return dtype_; }
    Device& device() const { return *device_; }
    DeviceType device_type() const { return device_ != nullptr ? device_->type() : DeviceType::kCPU; }
    void* data() { return data_; }
    const void* data() const { return data_; }
    size_t num_bytes() const { return bytes_; }
    bool is_contiguous() const { return true; }

    // Copies `bytes` from host memory into this tensor (H2D for GPU tensors).
    void copy_from(const void* host_source, size_t bytes);
    // Copies min(bytes) from another tensor, whichever devices the two live on.
    void copy_from(const Tensor& other);
    // Copies this tensor's bytes into host memory.
    void copy_to_host(void* host_dest, size_t bytes) const;

private:
    void Release();

    TensorShape shape_{};
    DType dtype_{DType::kFloat32};
    Device* device_{nullptr};
    void* data_{nullptr};
    bool owns_{false};
    size_t bytes_{0};
};

}  // namespace sci

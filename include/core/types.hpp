#pragma once

// Element types, device kinds and tensor shapes of the attention stack's public API.
// Same API shape as SciComputeInfra's core/types.hpp (reference stub/include/core/types.hpp:14-99):
// the enumerator values are part of the interface.

#include <cstddef>
#include <cstdint>
#include <initializer_list>
#include <vector>

// Visibility of the sci:: infrastructure symbols exported by libsca_host.so.
#if defined(__GNUC__) || defined(__clang__)
#define SCI_INFRA_API __attribute__((visibility("default")))
#else
#define SCI_INFRA_API
#endif

namespace sci {

using index_t = int64_t;

enum class DType : uint8_t {
    kFloat32 = 0,
    kFloat16 = 1,
    kBFloat16 = 2,
    kInt8 = 3,
    kInt32 = 4,
    kInt64 = 5,
    kBool = 6,
    kFloat64 = 7,
    kUInt8 = 8,
};

constexpr size_t kDTypeSize(DType dtype) {
    switch (dtype) {
        case DType::kFloat32: return 4;
        case DType::kFloat16: return 2;
        case DType::kBFloat16: return 2;
        case DType::kInt8: return 1;
        case DType::kInt32: return 4;
        case DType::kInt64: return 8;
        case DType::kBool: return 1;
        case DType::kFloat64: return 8;
        case DType::kUInt8: return 1;
    }
    return 0;
}

constexpr const char* kDTypeName(DType dtype) {
    switch (dtype) {
        case DType::kFloat32: return "float32";
        case DType::kFloat16: return "float16";
        case DType::kBFloat16: return "bfloat16";
        case DType::kInt8: return "int8";
        case DType::kInt32: return "int32";
        case DType::kInt64: return "int64";
        case DType::kBool: return "bool";
        case DType::kFloat64: return "float64";
        case DType::kUInt8: return "uint8";
    }
    return "unknown";
}

// kGPU is the HIP device. kCUDA keeps the enumerator name (and value) that callers of the
// reference's API spell, so their code compiles unchanged against this build.
enum class DeviceType : uint8_t { kCPU = 0, kGPU = 1, kCPUPinned = 2, kCUDA = kGPU };

constexpr const char* kDeviceTypeName(DeviceType type) {
    switch (type) {
        case DeviceType::kCPU: return "cpu";
        case DeviceType::kGPU: return "gpu";
        case DeviceType::kCPUPinned: return "cpu_pinned";
    }
    return "unknown";
}

enum class Layout : uint8_t { kContiguous = 0, kStrided = 1 };

// Up to 8 dimensions, stored inline.
class TensorShape {
public:
    static constexpr int kMaxDims = 8;

    TensorShape() = default;
    TensorShape(std::initializer_list<index_t> dims) {
        for (index_t d : dims) Push(d);
    }
    explicit TensorShape(const std::vector<index_t>& dims) {
        for (index_t d : dims) Push(d);
    }

    index_t ndims() const { return ndims_; }
    index_t dim(size_t i) const { return dims_[i]; }
    index_t& dim(size_t i) { return dims_[i]; }
    index_t num_elements() const {
        if (ndims_ == 0) return 0;
        index_t n = 1;
        for (index_t i = 0; i < ndims_; ++i) n *= dims_[i];
        return n;
    }

private:
    void Push(index_t d) {
        if (ndims_ < kMaxDims) dims_[ndims_++] = d;
    }

    index_t dims_[kMaxDims]{};
    index_t ndims_{0};
};

}  // namespace sci

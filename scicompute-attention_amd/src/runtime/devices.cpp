// sci:: infrastructure over the kernel library's C ABI: the host and GPU devices, streams and
// tensors. No HIP header is included here; every device operation is a sca_hip_* call.
//
// GPU allocations go through a caching pool: requests are rounded to a size class, freed blocks
// are kept per class and handed out again, so a steady stream of attention calls (each returning
// a freshly allocated output, as the API contract requires) does not call hipMalloc.

#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "device/device.hpp"
#include "device/stream.hpp"
#include "sca_hip.h"
#include "tensor/tensor.hpp"

namespace sci {
namespace {

class HostDeviceImpl final : public Device {
public:
    DeviceType type() const override { return DeviceType::kCPU; }
    std::string name() const override { return "host"; }
    void* allocate(size_t bytes) override {
        void* p = nullptr;
        // 64-byte alignment keeps 16-byte vector loads of host staging buffers legal.
        if (posix_memalign(&p, 64, bytes == 0 ? 64 : bytes) != 0) return nullptr;
        std::memset(p, 0, bytes == 0 ? 64 : bytes);
        return p;
    }
    void deallocate(void* ptr) override { std::free(ptr); }
    void copy_to_device(void* dst, const void* src, size_t bytes) override {
        std::memcpy(dst, src, bytes);
    }
    void copy_to_host(void* dst, const void* src, size_t bytes) override {
        std::memcpy(dst, src, bytes);
    }
    void copy_within(void* dst, const void* src, size_t bytes) override {
        std::memmove(dst, src, bytes);
    }
    void memset(void* ptr, int value, size_t bytes) override { std::memset(ptr, value, bytes); }
    void synchronize() override {}
    void copy_async(void* dst, const void* src, size_t bytes, Stream&) override {
        std::memcpy(dst, src, bytes);
    }
};

// Size classes: 512 B granularity below 1 MiB, 2 MiB granularity above.
size_t SizeClass(size_t bytes) {
    if (bytes == 0) bytes = 1;
    if (bytes < (1u << 20)) return (bytes + 511) / 512 * 512;
    const size_t two_mib = size_t{2} << 20;
    return (bytes + two_mib - 1) / two_mib * two_mib;
}

class GpuDeviceImpl final : public Device {
public:
    explicit GpuDeviceImpl(int id) : id_(id) {}
    DeviceType type() const override { return DeviceType::kGPU; }
    int id() const override { return id_; }
    std::string name() const override { return "gpu:" + std::to_string(id_); }

    void* allocate(size_t bytes) override {
        const size_t cls = SizeClass(bytes);
        {
            std::lock_guard<std::mutex> lock(mu_);
            auto it = free_.find(cls);
            if (it != free_.end() && !it->second.empty()) {
                void* p = it->second.back();
                it->second.pop_back();
                cached_ -= cls;
                live_[p] = cls;
                allocated_ += cls;
                return p;
            }
        }
        void* p = nullptr;
        if (sca_hip_malloc(&p, cls) != 0 || p == nullptr) {
            // Out of memory: drop the cache and retry once.
            ReleaseCached();
            if (sca_hip_malloc(&p, cls) != 0) return nullptr;
        }
        std::lock_guard<std::mutex> lock(mu_);
        live_[p] = cls;
        allocated_ += cls;
        return p;
    }

    void deallocate(void* ptr) override {
        if (ptr == nullptr) return;
        std::lock_guard<std::mutex> lock(mu_);
        auto it = live_.find(ptr);
        if (it == live_.end()) return;  // not ours
        const size_t cls = it->second;
        live_.erase(it);
        allocated_ -= cls;
        free_[cls].push_back(ptr);
        cached_ += cls;
    }

    void copy_to_device(void* dst, const void* src, size_t bytes) override {
        sca_hip_memcpy(dst, src, bytes, SCA_COPY_H2D);
    }
    void copy_to_host(void* dst, const void* src, size_t bytes) override {
        sca_hip_memcpy(dst, src, bytes, SCA_COPY_D2H);
    }
    void copy_within(void* dst, const void* src, size_t bytes) override {
        sca_hip_memcpy(dst, src, bytes, SCA_COPY_D2D);
    }
    void memset(void* ptr, int value, size_t bytes) override {
        if (value == 0) {
            sca_hip_zero_async(ptr, bytes, nullptr);
            sca_hip_stream_synchronize(nullptr);
            return;
        }
        std::vector<unsigned char> host(bytes, static_cast<unsigned char>(value));
        sca_hip_memcpy(ptr, host.data(), bytes, SCA_COPY_H2D);
    }
    void synchronize() override { sca_hip_device_synchronize(); }
    void copy_async(void* dst, const void* src, size_t bytes, Stream& stream) override {
        sca_hip_memcpy_async(dst, src, bytes, 0 /*runtime infers the direction*/, stream.handle());
    }
    size_t total_memory() const override {
        unsigned long long f = 0, t = 0;
        return sca_hip_mem_get_info(&f, &t) == 0 ? static_cast<size_t>(t) : 0;
    }
    size_t free_memory() const override {
        unsigned long long f = 0, t = 0;
        return sca_hip_mem_get_info(&f, &t) == 0 ? static_cast<size_t>(f) : 0;
    }

    size_t ReleaseCached() {
        std::map<size_t, std::vector<void*>> drop;
        {
            std::lock_guard<std::mutex> lock(mu_);
            drop.swap(free_);
            cached_ = 0;
        }
        size_t released = 0;
        if (!drop.empty()) sca_hip_device_synchronize();
        for (auto& kv : drop) {
            for (void* p : kv.second) {
                sca_hip_free(p);
                released += kv.first;
            }
        }
        return released;
    }
    size_t Cached() const {
        std::lock_guard<std::mutex> lock(mu_);
        return cached_;
    }
    size_t Allocated() const {
        std::lock_guard<std::mutex> lock(mu_);
        return allocated_;
    }

private:
    int id_;
    mutable std::mutex mu_;
    std::map<size_t, std::vector<void*>> free_;
    std::unordered_map<void*, size_t> live_;
    size_t cached_{0};
    size_t allocated_{0};
};

GpuDeviceImpl& GpuImpl(int id) {
    // Leaked on purpose: device frees from static destructors would run after the HIP runtime has
    // started tearing down.
    static std::mutex mu;
    static auto* devices = new std::unordered_map<int, GpuDeviceImpl*>();
    std::lock_guard<std::mutex> lock(mu);
    auto it = devices->find(id);
    if (it != devices->end()) return *it->second;
    auto* dev = new GpuDeviceImpl(id);
    (*devices)[id] = dev;
    return *dev;
}

}  // namespace

Device& HostDevice() {
    static HostDeviceImpl device;
    return device;
}

Device& GpuDevice(int id) { return GpuImpl(id); }

bool GpuAvailable() {
    int n = 0;
    return sca_hip_get_device_count(&n) == 0 && n > 0;
}

size_t GpuEmptyCache(int id) { return GpuImpl(id).ReleaseCached(); }
size_t GpuCachedBytes(int id) { return GpuImpl(id).Cached(); }
size_t GpuAllocatedBytes(int id) { return GpuImpl(id).Allocated(); }

// ---- Stream ----------------------------------------------------------------------------------
Result<Stream> Stream::Create() {
    void* handle = nullptr;
    const int rc = sca_hip_stream_create(&handle);
    if (rc != 0) {
        return MakeUnexpected<Stream>(Status(StatusCode::kCudaError,
                                             std::string("stream creation failed: ") +
                                                 sca_hip_last_error_string()));
    }
    Stream s(handle);
    s.owns_ = true;
    return Result<Stream>(std::move(s));
}

void Stream::synchronize() { sca_hip_stream_synchronize(handle_); }

void Stream::Release() {
    if (owns_ && handle_ != nullptr) sca_hip_stream_destroy(handle_);
    owns_ = false;
    handle_ = nullptr;
}

Stream& Stream::GetCurrent() {
    thread_local Stream current;
    return current;
}

void Stream::SetCurrent(const Stream& stream) { GetCurrent() = stream; }

// ---- Tensor ------------------------------------------------------------------------------------
Tensor::Tensor(const TensorShape& shape, DType dtype, Device& device)
    : shape_(shape), dtype_(dtype), device_(&device) {
    bytes_ = static_cast<size_t>(shape.num_elements()) * kDTypeSize(dtype);
    data_ = device.allocate(bytes_);
    owns_ = data_ != nullptr;
}

Tensor::Tensor(const TensorShape& shape, DType dtype, Device& device, void* external_data,
               bool owns_data)
    : shape_(shape), dtype_(dtype), device_(&device), data_(external_data), owns_(owns_data) {
    bytes_ = static_cast<size_t>(shape.num_elements()) * kDTypeSize(dtype);
}

Tensor::~Tensor() { Release(); }

Tensor::Tensor(Tensor&& other) noexcept
    : shape_(other.shape_),
      dtype_(other.dtype_),
      device_(other.device_),
      data_(other.data_),
      owns_(other.owns_),
      bytes_(other.bytes_) {
    other.data_ = nullptr;
    other.owns_ = false;
}

Tensor& Tensor::operator=(Tensor&& other) noexcept {
    if (this != &other) {
        Release();
        shape_ = other.shape_;
        dtype_ = other.dtype_;
        device_ = other.device_;
        data_ = other.data_;
        owns_ = other.owns_;
        bytes_ = other.bytes_;
        other.data_ = nullptr;
        other.owns_ = false;
    }
    return *this;
}

void Tensor::Release() {
    if (owns_ && data_ != nullptr && device_ != nullptr) device_->deallocate(data_);
    data_ = nullptr;
    owns_ = false;
}

void Tensor::copy_from(const void* host_source, size_t bytes) {
    if (data_ == nullptr || host_source == nullptr || device_ == nullptr) return;
    if (bytes > bytes_) bytes = bytes_;
    device_->copy_to_device(data_, host_source, bytes);
}

void Tensor::copy_from(const Tensor& other) {
    if (data_ == nullptr || other.data_ == nullptr || device_ == nullptr) return;
    const size_t bytes = bytes_ < other.bytes_ ? bytes_ : other.bytes_;
    const bool src_gpu = other.device_type() == DeviceType::kGPU;
    const bool dst_gpu = device_type() == DeviceType::kGPU;
    if (src_gpu && dst_gpu) {
        sca_hip_memcpy(data_, other.data_, bytes, SCA_COPY_D2D);
    } else if (src_gpu) {
        sca_hip_memcpy(data_, other.data_, bytes, SCA_COPY_D2H);
    } else if (dst_gpu) {
        sca_hip_memcpy(data_, other.data_, bytes, SCA_COPY_H2D);
    } else {
        std::memcpy(data_, other.data_, bytes);
    }
}

void Tensor::copy_to_host(void* host_dest, size_t bytes) const {
    if (data_ == nullptr || host_dest == nullptr) return;
    if (bytes > bytes_) bytes = bytes_;
    if (device_type() == DeviceType::kGPU) {
        sca_hip_memcpy(host_dest, data_, bytes, SCA_COPY_D2H);
    } else {
        std::memcpy(host_dest, data_, bytes);
    }
}

}  // namespace sci

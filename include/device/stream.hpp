#pragma once

// sci::Stream: an ordered queue of GPU work (a hipStream_t underneath).
// Same API shape as SciComputeInfra's device/stream.hpp (reference stub/include/device/stream.hpp:9-20).
// A default-constructed Stream is the device's default (null) stream; Create() makes an owning
// non-blocking stream at the default priority.

#include "core/status.hpp"
#include "core/types.hpp"

namespace sci {

class SCI_INFRA_API Stream {
public:
    Stream() = default;
    explicit Stream(void* handle) : handle_(handle) {}
    Stream(const Stream& other) : handle_(other.handle_) {}  // non-owning copy
    Stream& operator=(const Stream& other) {
        if (this != &other) {
            Release();
            handle_ = other.handle_;
        }
        return *this;
    }
    Stream(Stream&& other) noexcept : handle_(other.handle_), owns_(other.owns_) {
        other.owns_ = false;
    }
    ~Stream() { Release(); }

    // Creates an owning stream on the current device.
    static Result<Stream> Create();

    void* handle() const { return handle_; }
    DeviceType device_type() const { return DeviceType::kGPU; }
    void synchronize();

    // The calling thread's current stream (the default stream unless SetCurrent was called).
    static Stream& GetCurrent();
    static void SetCurrent(const Stream& stream);

private:
    void Release();

    void* handle_{nullptr};
    bool owns_{false};
};

}  // namespace sci

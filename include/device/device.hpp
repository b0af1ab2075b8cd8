#pragma once

// sci::Device: where a tensor's bytes live.
// Same API shape as SciComputeInfra's device/device.hpp (reference stub/include/device/device.hpp:16-62).
// This build provides two devices:
//   * HostDevice()   - the CPU heap;
//   * GpuDevice(id)  - a HIP GPU. Its allocate() serves requests from a per-device caching pool
//     (freed blocks are kept for reuse and handed out again to the next request of the same size
//     class), so steady-state attention calls do not call hipMalloc. The pool is stream-ordered
//     for single-stream use, like the allocators of the usual ML frameworks.

#include <cstddef>
#include <string>

#include "core/status.hpp"
#include "core/types.hpp"

namespace sci {

class Stream;

class SCI_INFRA_API Device {
public:
    virtual ~Device() = default;
    virtual DeviceType type() const = 0;
    virtual int id() const { return 0; }
    virtual std::string name() const = 0;
    virtual void* allocate(size_t bytes) = 0;
    virtual void deallocate(void* ptr) = 0;
    virtual void copy_to_device(void* dst, const void* src, size_t bytes) = 0;
    virtual void copy_to_host(void* dst, const void* src, size_t bytes) = 0;
    virtual void copy_within(void* dst, const void* src, size_t bytes) = 0;
    virtual void memset(void* ptr, int value, size_t bytes) = 0;
    virtual void synchronize() = 0;
    virtual void copy_async(void* dst, const void* src, size_t bytes, Stream& stream) = 0;
    virtual size_t total_memory() const { return 0; }
    virtual size_t free_memory() const { return 0; }
};

// Process-wide CPU device.
SCI_INFRA_API Device& HostDevice();

// Process-wide HIP device `id`. Callers should check GpuAvailable() first: on a machine without a
// GPU the returned device fails every allocation (allocate returns nullptr).
SCI_INFRA_API Device& GpuDevice(int id = 0);
SCI_INFRA_API bool GpuAvailable();

// Releases every block cached by GpuDevice(id)'s pool; returns the number of bytes released.
SCI_INFRA_API size_t GpuEmptyCache(int id = 0);
// Bytes currently cached (not handed out) and bytes handed out by GpuDevice(id)'s pool.
SCI_INFRA_API size_t GpuCachedBytes(int id = 0);
SCI_INFRA_API size_t GpuAllocatedBytes(int id = 0);

}  // namespace sci

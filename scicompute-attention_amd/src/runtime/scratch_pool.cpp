// Split-K partial scratch: one FP32 buffer per (device, kind), reused across calls.
// Growth rule as in the reference's src/runtime/scratch_pool.cpp:38-60 (x1.25 + 1024 elements).

#include <algorithm>
#include <cstring>
#include <map>
#include <mutex>
#include <utility>

#include "device/device.hpp"
#include "runtime/internal.hpp"
#include "sca_hip.h"

namespace sca {
namespace runtime {
namespace {

struct Entry {
    void* ptr{nullptr};
    size_t elements{0};
    int device_id{0};
};

std::mutex& PoolMutex() {
    static std::mutex mu;
    return mu;
}

// Leaked on purpose: freeing device memory from a static destructor would race the HIP runtime's
// own teardown at process exit.
std::map<std::pair<int, int>, Entry>& Pool() {
    static auto* pool = new std::map<std::pair<int, int>, Entry>();
    return *pool;
}

size_t g_high_water_bytes = 0;

}  // namespace

sci::Result<float*> AcquireScratchFp32(ScratchKind kind, size_t elements, int device_id) {
    if (elements == 0) {
        return sci::MakeUnexpected<float*>(
            MakeStatus(AttnStatusCode::kWorkspaceExceeded, "scratch request with 0 elements"));
    }
    std::lock_guard<std::mutex> lock(PoolMutex());
    Entry& entry = Pool()[{device_id, static_cast<int>(kind)}];
    if (entry.ptr == nullptr || entry.elements < elements) {
        sci::Device& device = sci::GpuDevice(device_id);
        if (entry.ptr != nullptr) {
            // The previous buffer may still be read by queued kernels.
            device.synchronize();
            device.deallocate(entry.ptr);
            entry.ptr = nullptr;
            entry.elements = 0;
        }
        const size_t grown = static_cast<size_t>(static_cast<double>(elements) * 1.25) + 1024;
        entry.ptr = device.allocate(grown * sizeof(float));
        if (entry.ptr == nullptr) {
            return sci::MakeUnexpected<float*>(MakeStatus(
                AttnStatusCode::kWorkspaceExceeded,
                "scratch allocation of " + std::to_string(grown * sizeof(float)) + " B failed"));
        }
        entry.elements = grown;
        entry.device_id = device_id;
        g_high_water_bytes = std::max(g_high_water_bytes, grown * sizeof(float));
    }
    return sci::Ok(static_cast<float*>(entry.ptr));
}

sci::Status ReleaseScratch() {
    std::lock_guard<std::mutex> lock(PoolMutex());
    for (auto& kv : Pool()) {
        if (kv.second.ptr != nullptr) {
            sci::Device& device = sci::GpuDevice(kv.second.device_id);
            device.synchronize();
            device.deallocate(kv.second.ptr);
        }
    }
    Pool().clear();
    return sci::Status::Ok();
}

size_t ScratchHighWaterMarkBytes() {
    std::lock_guard<std::mutex> lock(PoolMutex());
    return g_high_water_bytes;
}

}  // namespace runtime
}  // namespace sca

namespace sca {
namespace runtime {
namespace {

struct Staging {
    void* host{nullptr};
    size_t bytes{0};
    void* event{nullptr};  // recorded after the last copy out of `host`
};

std::mutex& StagingMutex() {
    static std::mutex mu;
    return mu;
}

std::map<int, Staging>& StagingPool() {  // leaked on purpose, like the scratch pool
    static auto* pool = new std::map<int, Staging>();
    return *pool;
}

}  // namespace

sci::Result<void*> UploadToScratch(ScratchKind kind, const void* host, size_t bytes,
                                   int device_id, void* stream) {
    sci::Result<float*> dst = AcquireScratchFp32(kind, (bytes + 3) / 4, device_id);
    if (!dst.ok()) return sci::MakeUnexpected<void*>(dst.error());
    std::lock_guard<std::mutex> lock(StagingMutex());
    Staging& st = StagingPool()[device_id];
    if (st.event != nullptr) {
        const sci::Status done =
            StatusFromHip(sca_hip_event_synchronize(st.event), "scratch staging reuse");
        if (!done.ok()) return sci::MakeUnexpected<void*>(done);
    } else {
        const sci::Status made =
            StatusFromHip(sca_hip_event_create(&st.event), "scratch staging event");
        if (!made.ok()) return sci::MakeUnexpected<void*>(made);
    }
    if (st.bytes < bytes) {
        if (st.host != nullptr) sca_hip_host_free(st.host);
        st.host = nullptr;
        st.bytes = 0;
        const size_t grown = std::max<size_t>(bytes, 4096);
        const sci::Status got =
            StatusFromHip(sca_hip_host_malloc(&st.host, grown), "scratch staging allocation");
        if (!got.ok()) return sci::MakeUnexpected<void*>(got);
        st.bytes = grown;
    }
    std::memcpy(st.host, host, bytes);
    sci::Status status = StatusFromHip(
        sca_hip_memcpy_async(*dst, st.host, bytes, SCA_COPY_H2D, stream), "scratch upload");
    if (status.ok()) {
        status = StatusFromHip(sca_hip_event_record(st.event, stream), "scratch staging event");
    }
    if (!status.ok()) return sci::MakeUnexpected<void*>(status);
    return sci::Ok(static_cast<void*>(*dst));
}

}  // namespace runtime
}  // namespace sca

// Device capability, probed once per device through sca_hip_probe_device and cached under a mutex
// (the reference's src/runtime/capability.cpp:12-90 keeps the same cache and env override).

#include <cstdlib>
#include <mutex>
#include <string>
#include <unordered_map>

#include "runtime/internal.hpp"
#include "scicompute_attention/capability.hpp"

namespace sca {
namespace {

std::mutex& CacheMutex() {
    static std::mutex mu;
    return mu;
}

std::unordered_map<int, DeviceCapability>& Cache() {
    static auto* cache = new std::unordered_map<int, DeviceCapability>();
    return *cache;
}

DeviceCapability Probe(int device_id) {
    DeviceCapability cap;
    ScaHipDeviceProbe raw{};
    if (sca_hip_probe_device(device_id, &raw) != 0 || raw.gpu_available == 0) {
        cap.device_name = "gpu-unavailable";
        return cap;
    }
    cap.arch_name = raw.arch_name;
    // The marketing name can be empty when the driver's name table is not installed.
    cap.device_name = raw.name[0] != '\0' ? std::string(raw.name) : "AMD " + cap.arch_name;
    cap.major = raw.major;
    cap.minor = raw.minor;
    cap.sm_count = raw.cu_count;
    cap.wave_size = raw.wave_size;
    cap.clock_khz = raw.clock_khz;
    cap.smem_per_sm = static_cast<size_t>(raw.lds_per_cu);
    cap.smem_per_block_default = static_cast<size_t>(raw.lds_per_block);
    cap.smem_per_block_optin = static_cast<size_t>(raw.lds_per_block);
    cap.regs_per_sm = static_cast<size_t>(raw.regs_per_cu);
    cap.max_threads_per_sm = static_cast<size_t>(raw.max_threads_per_cu);
    cap.l2_bytes = static_cast<size_t>(raw.l2_bytes);
    cap.total_mem_bytes = static_cast<size_t>(raw.total_mem_bytes);
    cap.free_mem_bytes = static_cast<size_t>(raw.free_mem_bytes);
    cap.has_mfma_f16_k16 = raw.binary_has_gfx950 != 0 && cap.arch_name.rfind("gfx950", 0) == 0;
    return cap;
}

size_t EnvLimit(const char* name) {
    const char* text = std::getenv(name);
    if (text == nullptr) return 0;
    const long long v = std::strtoll(text, nullptr, 10);
    return v > 0 ? static_cast<size_t>(v) : 0;
}

}  // namespace

const DeviceCapability& DeviceCapability::ForDevice(int device_id) {
    std::lock_guard<std::mutex> lock(CacheMutex());
    auto& cache = Cache();
    auto it = cache.find(device_id);
    if (it == cache.end()) it = cache.emplace(device_id, Probe(device_id)).first;
    return it->second;
}

sci::Status DeviceCapability::Refresh(int device_id) {
    DeviceCapability fresh = Probe(device_id);
    std::lock_guard<std::mutex> lock(CacheMutex());
    Cache()[device_id] = std::move(fresh);
    return sci::Status::Ok();
}

size_t DeviceCapability::SmemLimitPerBlock(const DeviceCapability& cap) noexcept {
    size_t limit = cap.smem_per_block_optin != 0 ? cap.smem_per_block_optin
                                                 : cap.smem_per_block_default;
    for (const char* name : {"SCI_ATTENTION_MAX_LDS_BYTES", "SCI_ATTENTION_MAX_SMEM_BYTES"}) {
        const size_t env = EnvLimit(name);
        if (env != 0 && env < limit) limit = env;
    }
    if (cap.smem_per_sm != 0 && limit > cap.smem_per_sm) limit = cap.smem_per_sm;
    return limit;
}

bool DeviceCapability::GpuAvailable() noexcept {
    int count = 0;
    return sca_hip_get_device_count(&count) == 0 && count > 0;
}

}  // namespace sca

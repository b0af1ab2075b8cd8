// Runtime plumbing of the C ABI: device probe, memory, streams, events, zero-fill and the
// thread-local error text. All HIP runtime calls of the stack are in this directory.
//
// Replaces the reference's device probe and launch helper
// (src/runtime/device_probe.cu:35-84, src/runtime/launcher.cu:26-111): errors are reported as
// codes plus a message, and SCI_ATTENTION_DEBUG_SYNC=1 adds a synchronise + error check after
// every launch.

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "sca_device.hpp"

namespace sca_hip {
namespace {

thread_local std::string g_last_error;

bool DebugSync() {
    static const bool enabled = [] {
        const char* env = std::getenv("SCI_ATTENTION_DEBUG_SYNC");
        return env != nullptr && env[0] == '1';
    }();
    return enabled;
}

// Zero-fill with 16 B stores plus a byte tail. Used instead of hipMemsetAsync so that callers
// that capture the stream into a graph record a kernel node, not a memset node.
__global__ void zero_fill_kernel(uint8_t* dst, size_t bytes) {
    const size_t n16 = bytes / 16;
    const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
    uint4* dst16 = reinterpret_cast<uint4*>(dst);
    for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16;
         i += stride) {
        dst16[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    const size_t tail_begin = n16 * 16;
    for (size_t i = tail_begin + static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
         i < bytes; i += stride) {
        dst[i] = 0;
    }
}

}  // namespace

int SetError(int code, const std::string& message) {
    g_last_error = message;
    return code;
}

int FromHip(hipError_t err, const char* what) {
    if (err == hipSuccess) return 0;
    return SetError(static_cast<int>(err),
                    std::string(what) + ": " + hipGetErrorName(err) + " (" +
                        hipGetErrorString(err) + ")");
}

int CheckLaunch(const char* what, hipStream_t stream) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return FromHip(err, what);
    if (DebugSync()) {
        err = hipStreamSynchronize(stream);
        if (err != hipSuccess) return FromHip(err, what);
        err = hipGetLastError();
        if (err != hipSuccess) return FromHip(err, what);
    }
    return 0;
}

}  // namespace sca_hip

using sca_hip::FromHip;
using sca_hip::SetError;

extern "C" {

const char* sca_hip_last_error_string(void) { return sca_hip::g_last_error.c_str(); }

int sca_hip_get_device_count(int* count) {
    if (count == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_get_device_count: null");
    int n = 0;
    const hipError_t err = hipGetDeviceCount(&n);
    if (err != hipSuccess) {
        (void)hipGetLastError();  // clear the sticky "no device" error
        *count = 0;
        return 0;
    }
    *count = n;
    return 0;
}

int sca_hip_probe_device(int device_id, ScaHipDeviceProbe* out) {
    if (out == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_probe_device: null out");
    std::memset(out, 0, sizeof(*out));
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        out->gpu_available = 0;
        std::strncpy(out->name, "hip-unavailable", sizeof(out->name) - 1);
        return 0;
    }
    if (device_id < 0 || device_id >= n) {
        return SetError(SCA_E_DEVICE_CAPABILITY,
                        "sca_hip_probe_device: device_id=" + std::to_string(device_id) +
                            " out of range [0," + std::to_string(n) + ")");
    }
    hipDeviceProp_t prop;
    int rc = FromHip(hipGetDeviceProperties(&prop, device_id), "hipGetDeviceProperties");
    if (rc != 0) return rc;
    std::strncpy(out->name, prop.name, sizeof(out->name) - 1);
    std::strncpy(out->arch_name, prop.gcnArchName, sizeof(out->arch_name) - 1);
    out->major = prop.major;
    out->minor = prop.minor;
    out->cu_count = prop.multiProcessorCount;
    out->wave_size = prop.warpSize;
    out->clock_khz = prop.clockRate;
    out->memory_clock_khz = prop.memoryClockRate;
    out->memory_bus_width_bits = prop.memoryBusWidth;
    out->lds_per_cu = prop.maxSharedMemoryPerMultiProcessor;
    out->lds_per_block = prop.sharedMemPerBlock;
    out->regs_per_cu = static_cast<unsigned long long>(prop.regsPerMultiprocessor);
    out->max_threads_per_cu = static_cast<unsigned long long>(prop.maxThreadsPerMultiProcessor);
    out->l2_bytes = static_cast<unsigned long long>(prop.l2CacheSize);
    out->total_mem_bytes = prop.totalGlobalMem;
    size_t free_b = 0, total_b = 0;
    int current = 0;
    if (hipGetDevice(&current) == hipSuccess && current == device_id &&
        hipMemGetInfo(&free_b, &total_b) == hipSuccess) {
        out->free_mem_bytes = free_b;
    }
    out->gpu_available = 1;
    out->binary_has_gfx950 = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
    return 0;
}

int sca_hip_mem_get_info(unsigned long long* free_bytes, unsigned long long* total_bytes) {
    size_t f = 0, t = 0;
    const int rc = FromHip(hipMemGetInfo(&f, &t), "hipMemGetInfo");
    if (rc != 0) return rc;
    if (free_bytes != nullptr) *free_bytes = f;
    if (total_bytes != nullptr) *total_bytes = t;
    return 0;
}

int sca_hip_malloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_malloc: null ptr");
    *ptr = nullptr;
    if (bytes == 0) return 0;
    return FromHip(hipMalloc(ptr, bytes), "hipMalloc");
}

int sca_hip_free(void* ptr) {
    if (ptr == nullptr) return 0;
    return FromHip(hipFree(ptr), "hipFree");
}

int sca_hip_host_malloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_host_malloc: null ptr");
    *ptr = nullptr;
    if (bytes == 0) return 0;
    return FromHip(hipHostMalloc(ptr, bytes, hipHostMallocDefault), "hipHostMalloc");
}

int sca_hip_host_free(void* ptr) {
    if (ptr == nullptr) return 0;
    return FromHip(hipHostFree(ptr), "hipHostFree");
}

static hipMemcpyKind KindOf(int kind) {
    switch (kind) {
        case SCA_COPY_H2D: return hipMemcpyHostToDevice;
        case SCA_COPY_D2H: return hipMemcpyDeviceToHost;
        case SCA_COPY_D2D: return hipMemcpyDeviceToDevice;
        case SCA_COPY_H2H: return hipMemcpyHostToHost;
        default: return hipMemcpyDefault;
    }
}

int sca_hip_memcpy(void* dst, const void* src, size_t bytes, int kind) {
    if (bytes == 0) return 0;
    if (dst == nullptr || src == nullptr) {
        return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_memcpy: null pointer");
    }
    return FromHip(hipMemcpy(dst, src, bytes, KindOf(kind)), "hipMemcpy");
}

int sca_hip_memcpy_async(void* dst, const void* src, size_t bytes, int kind, void* stream) {
    if (bytes == 0) return 0;
    if (dst == nullptr || src == nullptr) {
        return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_memcpy_async: null pointer");
    }
    return FromHip(hipMemcpyAsync(dst, src, bytes, KindOf(kind),
                                  static_cast<hipStream_t>(stream)),
                   "hipMemcpyAsync");
}

int sca_hip_zero_async(void* ptr, size_t bytes, void* stream) {
    if (bytes == 0) return 0;
    if (ptr == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_zero_async: null pointer");
    const size_t chunks = (bytes + 15) / 16;
    size_t blocks = (chunks + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks == 0) blocks = 1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(sca_hip::zero_fill_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256),
                       0, s, static_cast<uint8_t*>(ptr), bytes);
    return sca_hip::CheckLaunch("zero_fill_kernel", s);
}

int sca_hip_device_synchronize(void) {
    return FromHip(hipDeviceSynchronize(), "hipDeviceSynchronize");
}

int sca_hip_stream_create(void** stream) {
    if (stream == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_stream_create: null");
    hipStream_t s = nullptr;
    // Default priority only: streams of different priorities are never mixed by this library.
    const int rc = FromHip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking),
                           "hipStreamCreateWithFlags");
    *stream = s;
    return rc;
}

int sca_hip_stream_destroy(void* stream) {
    if (stream == nullptr) return 0;
    return FromHip(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy");
}

int sca_hip_stream_synchronize(void* stream) {
    return FromHip(hipStreamSynchronize(static_cast<hipStream_t>(stream)),
                   "hipStreamSynchronize");
}

int sca_hip_event_create(void** event) {
    if (event == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_event_create: null");
    hipEvent_t e = nullptr;
    const int rc = FromHip(hipEventCreate(&e), "hipEventCreate");
    *event = e;
    return rc;
}

int sca_hip_event_destroy(void* event) {
    if (event == nullptr) return 0;
    return FromHip(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}

int sca_hip_event_record(void* event, void* stream) {
    return FromHip(hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream)),
                   "hipEventRecord");
}

int sca_hip_event_synchronize(void* event) {
    return FromHip(hipEventSynchronize(static_cast<hipEvent_t>(event)), "hipEventSynchronize");
}

int sca_hip_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (ms == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "sca_hip_event_elapsed_ms: null");
    return FromHip(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                       static_cast<hipEvent_t>(stop)),
                   "hipEventElapsedTime");
}

}  // extern "C"

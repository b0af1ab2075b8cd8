// Internal hand-offs of the host layer: status conversion from the kernel library's C ABI, stream
// resolution, backend accessors and the split-K scratch pool. Never installed.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>

#include "core/status.hpp"
#include "core/types.hpp"
#include "device/stream.hpp"
#include "sca_hip.h"
#include "scicompute_attention/backends.hpp"
#include "scicompute_attention/status.hpp"

namespace sca {
namespace runtime {

// sca_hip_* return code -> sci::Status. Codes 2001..2010 keep their attention code (and gain the
// "[SCA-<code>]" prefix); HIP runtime errors become kCudaError with the runtime's message.
inline sci::Status StatusFromHip(int rc, const char* what) {
    if (rc == 0) return sci::Status::Ok();
    const std::string detail = std::string(what) + ": " + sca_hip_last_error_string();
    if (rc >= 2001 && rc <= 2010) return MakeStatus(static_cast<AttnStatusCode>(rc), detail);
    return sci::Status(sci::StatusCode::kCudaError,
                       "[SCA-hip " + std::to_string(rc) + "] " + detail);
}

// cfg.stream, or the calling thread's current stream when it is null.
inline void* StreamHandle(sci::Stream* stream) {
    return stream != nullptr ? stream->handle() : sci::Stream::GetCurrent().handle();
}

// Kernel-library dtype id, or -1 for a non-compute dtype.
inline int32_t KernelDtype(sci::DType dtype) {
    switch (dtype) {
        case sci::DType::kFloat32: return SCA_DTYPE_F32;
        case sci::DType::kFloat16: return SCA_DTYPE_F16;
        case sci::DType::kBFloat16: return SCA_DTYPE_BF16;
        default: return -1;
    }
}

const IAttentionBackend* NaiveBackendInstance() noexcept;
const IAttentionBackend* TiledBackendInstance() noexcept;
const IAttentionBackend* FlashBackendInstance() noexcept;
const IAttentionBackend* DecodeBackendInstance() noexcept;
const IAttentionBackend* PagedBackendInstance() noexcept;

// One FP32 scratch buffer per (device, kind), grown by 25% + 1024 elements when a request does
// not fit and otherwise reused; the pointer stays valid until the next acquisition of the same
// (device, kind). Calls are expected not to overlap (single-threaded use of the API).
enum class ScratchKind : int { kScoresFp32 = 0, kDecodePartials = 1, kGeneric = 2, kVarlenTables = 3 };
sci::Result<float*> AcquireScratchFp32(ScratchKind kind, size_t elements, int device_id);
sci::Status ReleaseScratch();
size_t ScratchHighWaterMarkBytes();
// Copies `bytes` of host data into the (device, kind) scratch buffer on `stream`, through pinned
// staging that is reused once the previous copy has completed; returns the device pointer.
sci::Result<void*> UploadToScratch(ScratchKind kind, const void* host, size_t bytes,
                                   int device_id, void* stream);

}  // namespace runtime
}  // namespace sca

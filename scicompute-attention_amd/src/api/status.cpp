// Status codes, names and the small enum helpers of the public API.
// Behaviour follows the reference's src/api/status.cpp:14-103: message format "[SCA-<code>] ...",
// the code -> sci::StatusCode table and the stable names.

#include <cstdlib>
#include <string>

#include "scicompute_attention/attention_types.hpp"
#include "scicompute_attention/status.hpp"
#include "scicompute_attention/version.hpp"

namespace sca {

const char* VersionString() noexcept { return SCI_ATTENTION_VERSION_STRING; }
const char* BuildFlavor() noexcept { return "mi355x-hip-gfx950"; }

const char* ToString(AttnStatusCode code) noexcept {
    switch (code) {
        case AttnStatusCode::kOk: return "OK";
        case AttnStatusCode::kUnsupportedHeadDim: return "UnsupportedHeadDim";
        case AttnStatusCode::kUnsupportedDtype: return "UnsupportedDtype";
        case AttnStatusCode::kUnsupportedLayout: return "UnsupportedLayout";
        case AttnStatusCode::kLayoutMismatch: return "LayoutMismatch";
        case AttnStatusCode::kShapeMismatch: return "ShapeMismatch";
        case AttnStatusCode::kSeqTooLong: return "SeqTooLong";
        case AttnStatusCode::kKVCapacityExceeded: return "KVCapacityExceeded";
        case AttnStatusCode::kWorkspaceExceeded: return "WorkspaceExceeded";
        case AttnStatusCode::kUnsupportedFeature: return "UnsupportedFeature";
        case AttnStatusCode::kDeviceCapability: return "DeviceCapability";
    }
    return "UnknownAttnStatus";
}

sci::StatusCode ToSciCode(AttnStatusCode code) noexcept {
    switch (code) {
        case AttnStatusCode::kOk: return sci::StatusCode::kOk;
        case AttnStatusCode::kUnsupportedHeadDim:
        case AttnStatusCode::kUnsupportedDtype:
        case AttnStatusCode::kUnsupportedLayout:
        case AttnStatusCode::kLayoutMismatch:
        case AttnStatusCode::kShapeMismatch:
        case AttnStatusCode::kSeqTooLong: return sci::StatusCode::kInvalidArgument;
        case AttnStatusCode::kKVCapacityExceeded:
        case AttnStatusCode::kWorkspaceExceeded: return sci::StatusCode::kResourceExhausted;
        case AttnStatusCode::kUnsupportedFeature: return sci::StatusCode::kNotImplemented;
        case AttnStatusCode::kDeviceCapability: return sci::StatusCode::kInvalidOperation;
    }
    return sci::StatusCode::kError;
}

sci::Status MakeStatus(AttnStatusCode code, std::string detail) {
    std::string message = "[SCA-";
    message += std::to_string(static_cast<int32_t>(code));
    message += "] ";
    message += detail;
    return sci::Status(ToSciCode(code), std::move(message));
}

AttnStatusCode ExtractCode(const sci::Status& status) noexcept {
    const std::string& msg = status.message();
    const size_t at = msg.find("[SCA-");
    if (at == std::string::npos) return AttnStatusCode::kOk;
    return static_cast<AttnStatusCode>(std::atoi(msg.c_str() + at + 5));
}

int SupportedHeadDimIndex(int64_t head_dim) noexcept {
    for (int64_t i = 0; i < kNumSupportedHeadDims; ++i) {
        if (kSupportedHeadDims[i] == head_dim) return static_cast<int>(i);
    }
    return -1;
}

const char* LayoutName(AttnLayout layout) noexcept {
    switch (layout) {
        case AttnLayout::kBHSD: return "bhsd";
        case AttnLayout::kBSHD: return "bshd";
    }
    return "unknown-layout";
}

const char* KvLayoutName(KvLayout layout) noexcept {
    return layout == KvLayout::kBlockMajor ? "block-major" : "unknown-kv-layout";
}

const char* BackendName(BackendKind kind) noexcept {
    switch (kind) {
        case BackendKind::kAuto: return "auto";
        case BackendKind::kNaive: return "naive";
        case BackendKind::kTiled: return "tiled";
        case BackendKind::kFlash: return "flash";
        case BackendKind::kDecode: return "decode";
        case BackendKind::kPaged: return "paged";
    }
    return "unknown-backend";
}

bool IsSupportedComputeDtype(sci::DType dtype) noexcept {
    return dtype == sci::DType::kFloat32 || dtype == sci::DType::kFloat16 ||
           dtype == sci::DType::kBFloat16;
}

int64_t DtypeSize(sci::DType dtype) noexcept {
    return static_cast<int64_t>(sci::kDTypeSize(dtype));
}

}  // namespace sca

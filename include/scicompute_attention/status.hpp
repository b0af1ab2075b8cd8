#pragma once

#include <cstdint>
#include <string>

#include "core/status.hpp"
#include "scicompute_attention/export.hpp"

namespace sca {

// Attention-specific error codes. They travel inside the message text as "[SCA-<code>] ..."
// while the sci::StatusCode carries the closest general meaning (see ToSciCode), so a caller can
// branch on either.
enum class AttnStatusCode : int32_t {
    kOk = 0,
    kUnsupportedHeadDim = 2001,
    kUnsupportedDtype = 2002,
    kUnsupportedLayout = 2003,
    kLayoutMismatch = 2004,
    kShapeMismatch = 2005,
    kSeqTooLong = 2006,
    kKVCapacityExceeded = 2007,
    kWorkspaceExceeded = 2008,
    kUnsupportedFeature = 2009,
    kDeviceCapability = 2010,
};

// Stable name of a code ("KVCapacityExceeded", ...).
SCI_ATTENTION_API const char* ToString(AttnStatusCode code) noexcept;

// General code for an attention code; total over the enum.
SCI_ATTENTION_API sci::StatusCode ToSciCode(AttnStatusCode code) noexcept;

// Status whose message is "[SCA-<code>] <detail>".
SCI_ATTENTION_API sci::Status MakeStatus(AttnStatusCode code, std::string detail);

// The attention code embedded in a status message (kOk when there is none).
SCI_ATTENTION_API AttnStatusCode ExtractCode(const sci::Status& status) noexcept;

inline bool IsOk(const sci::Status& status) noexcept { return status.ok(); }

}  // namespace sca

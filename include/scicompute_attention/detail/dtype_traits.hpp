#pragma once

#include <cstdint>

#include "core/types.hpp"

namespace sca {
namespace detail {

// Host view of the compute dtypes. Device-side conversions live in the kernel library.
template <sci::DType kDtype>
struct DTypeTraits;

template <>
struct DTypeTraits<sci::DType::kFloat32> {
    using HostType = float;
    static constexpr int64_t kBytes = 4;
    static constexpr bool kSupportsMma = false;  // served by decode only (no fp32 MFMA path)
};

template <>
struct DTypeTraits<sci::DType::kFloat16> {
    using HostType = uint16_t;
    static constexpr int64_t kBytes = 2;
    static constexpr bool kSupportsMma = true;
};

template <>
struct DTypeTraits<sci::DType::kBFloat16> {
    using HostType = uint16_t;
    static constexpr int64_t kBytes = 2;
    static constexpr bool kSupportsMma = true;
};

// CDNA4 MFMA tile used by the flash kernel: v_mfma_f32_32x32x16_{f16,bf16}.
inline constexpr int64_t kMfmaM = 32;
inline constexpr int64_t kMfmaN = 32;
inline constexpr int64_t kMfmaK = 16;

// Global loads and LDS writes move 16 bytes per lane.
inline constexpr int64_t kVectorBytes = 16;

}  // namespace detail
}  // namespace sca

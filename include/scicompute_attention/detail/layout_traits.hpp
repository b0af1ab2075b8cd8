#pragma once

#include <cstdint>

#include "scicompute_attention/attention_types.hpp"

namespace sca {
namespace detail {

// Element strides of a 4-D Q/K/V/O tensor; the head-dim stride is always 1.
struct Strides {
    int64_t s_b{0};
    int64_t s_h{0};
    int64_t s_s{0};
    int64_t s_d{0};
};

// BHSD: [B,H,S,D]; BSHD: [B,S,H,D]. Every host path derives its strides here.
inline Strides StridesFor(AttnLayout layout, int64_t seq, int64_t heads, int64_t head_dim) {
    Strides s;
    s.s_d = 1;
    if (layout == AttnLayout::kBHSD) {
        s.s_s = head_dim;
        s.s_h = seq * head_dim;
        s.s_b = heads * seq * head_dim;
    } else {
        s.s_h = head_dim;
        s.s_s = heads * head_dim;
        s.s_b = seq * heads * head_dim;
    }
    return s;
}

inline int64_t Offset(const Strides& s, int64_t b, int64_t h, int64_t t, int64_t d) noexcept {
    return b * s.s_b + h * s.s_h + t * s.s_s + d * s.s_d;
}

inline int64_t OffsetBHSD(int64_t b, int64_t h, int64_t t, int64_t d, int64_t seq, int64_t heads,
                          int64_t head_dim) noexcept {
    return ((b * heads + h) * seq + t) * head_dim + d;
}

inline int64_t OffsetBSHD(int64_t b, int64_t t, int64_t h, int64_t d, int64_t seq, int64_t heads,
                          int64_t head_dim) noexcept {
    return ((b * seq + t) * heads + h) * head_dim + d;
}

inline bool LayoutSupported(AttnLayout layout) noexcept {
    return layout == AttnLayout::kBHSD || layout == AttnLayout::kBSHD;
}

}  // namespace detail
}  // namespace sca

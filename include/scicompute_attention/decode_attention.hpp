#pragma once

#include "scicompute_attention/attention_config.hpp"
#include "scicompute_attention/attention_result.hpp"
#include "scicompute_attention/capability.hpp"
#include "scicompute_attention/export.hpp"

namespace sca {

struct DecodeConfig {
    int64_t num_splits{0};   // 0 => chosen from the shape and the device
    int64_t max_splits{64};  // cap on the automatic choice (bounds the partial scratch)
    bool use_splitk{true};   // false => one split (no combine pass)
};

SCI_ATTENTION_API DecodeConfig RecommendDecodeConfig(const AttentionShape& shape,
                                                     const DeviceCapability& cap);

// Decode (S_q == 1): every KV chunk is streamed once per KV head into FP32 (m, l, O) partials
// that a log-sum-exp combine merges.
SCI_ATTENTION_API sci::Result<AttentionResult> decode_attention(const sci::Tensor& q,
                                                                const sci::Tensor& k,
                                                                const sci::Tensor& v,
                                                                const AttentionConfig& cfg);

SCI_ATTENTION_API sci::Result<AttentionResult> decode_attention(const sci::Tensor& q,
                                                                const sci::Tensor& k,
                                                                const sci::Tensor& v,
                                                                const AttentionConfig& cfg,
                                                                const DecodeConfig& decode_cfg);

}  // namespace sca

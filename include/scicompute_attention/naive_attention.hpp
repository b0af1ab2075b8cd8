#pragma once

#include "scicompute_attention/attention_config.hpp"
#include "scicompute_attention/attention_result.hpp"
#include "scicompute_attention/export.hpp"

namespace sca {

// The reference's score-materialising backend. It is not part of the MI355X build: the call
// returns kUnsupportedFeature with a pointer to flash/decode.
SCI_ATTENTION_API sci::Result<AttentionResult> naive_attention(const sci::Tensor& q,
                                                               const sci::Tensor& k,
                                                               const sci::Tensor& v,
                                                               const AttentionConfig& cfg);

}  // namespace sca

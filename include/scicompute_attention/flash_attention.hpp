#pragma once

#include "scicompute_attention/attention_config.hpp"
#include "scicompute_attention/attention_result.hpp"
#include "scicompute_attention/export.hpp"

namespace sca {

// IO-aware prefill: scores stay on chip; the online-softmax state is rescaled per K/V tile.
// fp16/bf16 inputs; output BHSD in the input dtype.
SCI_ATTENTION_API sci::Result<AttentionResult> flash_attention(const sci::Tensor& q,
                                                               const sci::Tensor& k,
                                                               const sci::Tensor& v,
                                                               const AttentionConfig& cfg);

// Packed variable-length batches: q [total_q, H_q, D], k/v [total_kv, H_kv, D] (contiguous);
// cu_seqlens_q / cu_seqlens_kv are host int32 arrays of num_seqs + 1 offsets (see
// ValidateVarlenHost). The output is packed like q. LSE is not available on this entry point.
SCI_ATTENTION_API sci::Result<AttentionResult> flash_attention_varlen(
    const sci::Tensor& q, const sci::Tensor& k, const sci::Tensor& v, int64_t num_seqs,
    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kv, int64_t max_seq_q,
    int64_t max_seq_kv, const AttentionConfig& cfg);

// LDS bytes one workgroup of the MI355X flash kernel uses for head_dim (-1 if not built).
SCI_ATTENTION_API int64_t FlashLdsBytes(int64_t head_dim, int64_t elem_bytes);

}  // namespace sca

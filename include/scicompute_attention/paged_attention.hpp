#pragma once

#include <cstdint>

#include "scicompute_attention/attention_config.hpp"
#include "scicompute_attention/attention_result.hpp"
#include "scicompute_attention/export.hpp"
#include "scicompute_attention/paged_kv_cache.hpp"

namespace sca {

struct PagedAttentionParams {
    const int32_t* page_table{nullptr};  // device [num_seqs, max_blocks_per_seq]; null => kv's own
    const int32_t* seq_lens{nullptr};    // device [num_seqs] (including the new token); null =>
                                         // every mapped page of the row is attended in full
    int64_t num_seqs{0};
    int64_t block_size{16};
    int64_t max_blocks_per_seq{0};       // 0 => kv.MaxBlocksPerSeq()
    int64_t layer{0};                    // which KV layer to read
};

// Decode over a paged KV cache: q is [num_seqs, H_q, 1, D] BHSD.
SCI_ATTENTION_API sci::Result<AttentionResult> paged_attention(const sci::Tensor& q,
                                                               const PagedKVCache& kv,
                                                               const PagedAttentionParams& params,
                                                               const AttentionConfig& cfg);

SCI_ATTENTION_API sci::Result<AttentionResult> paged_attention(const sci::Tensor& q,
                                                               const PagedKVCache& kv,
                                                               const AttentionConfig& cfg);

}  // namespace sca

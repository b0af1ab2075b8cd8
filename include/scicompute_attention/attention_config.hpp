#pragma once

#include <cstddef>
#include <string>

#include "core/status.hpp"
#include "core/types.hpp"
#include "scicompute_attention/attention_types.hpp"
#include "scicompute_attention/detail/tile_config.hpp"
#include "scicompute_attention/export.hpp"

namespace sci {
class Stream;
}  // namespace sci

namespace sca {

struct AttentionConfig {
    BackendKind backend{BackendKind::kAuto};
    AttnLayout layout{AttnLayout::kBHSD};
    bool causal{false};               // bottom-right aligned: key j visible from row i iff
                                      // j <= i + (seq_kv - seq_q)
    bool return_lse{false};           // FP32 [B, H_q, S_q] natural-log LSE next to the output
    float scale{0.0f};                // 0 => 1/sqrt(head_dim) (see EffectiveScale)
    float softcap{0.0f};              // 0 => off; only the flash backend may accept it
    int64_t sliding_window{0};        // 0 => off; > 0 is rejected (not implemented)
    int64_t num_splits{0};            // decode split-K count; 0 => chosen by the dispatcher
    size_t workspace_limit_bytes{0};  // 0 => no explicit limit
    bool allow_fallback{false};       // never degrade silently unless the caller opts in
    // Host-resident int32 offsets (num_seqs + 1 entries) for flash_attention_varlen.
    const int32_t* cu_seqlens_q{nullptr};
    const int32_t* cu_seqlens_kv{nullptr};
    sci::Stream* stream{nullptr};     // nullptr => sci::Stream::GetCurrent()
};

// cfg.scale when it is > 0, otherwise 1/sqrt(head_dim) evaluated in double and rounded to float.
SCI_ATTENTION_API float EffectiveScale(const AttentionConfig& cfg,
                                       const AttentionShape& shape) noexcept;

// The one validation entry point of the API: geometry, head_dim, GQA divisibility, the causal
// S_kv >= S_q rule and feature availability. Messages name the offending field and its value.
SCI_ATTENTION_API sci::Status Validate(const AttentionConfig& cfg, const AttentionShape& shape,
                                       std::string* detail = nullptr);

// Tile geometry of the flash kernel for this shape (reported by Explain and the stats).
SCI_ATTENTION_API TileConfig RecommendTile(const AttentionConfig& cfg, const AttentionShape& shape);

// Checks host varlen offsets: starts at 0, strictly increasing, batch+1 entries; optionally
// returns the longest sequence.
SCI_ATTENTION_API sci::Status ValidateVarlenHost(const int32_t* host_cu_seqlens, int64_t batch,
                                                 int64_t* max_seq_out = nullptr);

}  // namespace sca

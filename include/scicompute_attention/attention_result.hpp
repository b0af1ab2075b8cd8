#pragma once

#include <cstddef>
#include <string>

#include "tensor/tensor.hpp"

#include "scicompute_attention/attention_types.hpp"
#include "scicompute_attention/detail/tile_config.hpp"
#include "scicompute_attention/export.hpp"

namespace sca {

struct AttentionRuntimeStats {
    BackendKind used_backend{BackendKind::kAuto};
    TileConfig tile{};
    size_t workspace_bytes{0};      // scratch the call used (split-K partials, ...)
    size_t kv_bytes{0};             // KV cache footprint (paged path)
    std::string note;               // how the request was served; any degradation is described
    int64_t num_splits{0};          // decode/paged split count (0 = not applicable)
    int64_t materialized_score_bytes{0};  // bytes of an S_q x S_kv score matrix written to
                                          // memory; always 0 for flash
};

struct AttentionResult {
    sci::Tensor out;   // new contiguous BHSD tensor in the input dtype
    sci::Tensor lse;   // FP32 [B, H_q, S_q] when cfg.return_lse, otherwise empty
    AttentionRuntimeStats stats;
};

}  // namespace sca

// Request validation shared by every entry point.
// Rules and message texts follow the reference's src/api/api_validate.cpp:31-174 (callers and the
// reference's tests match on the "<struct> invalid: <field>=<value>" wording); the tile report
// comes from the MI355X kernel library instead of the reference's CUDA tile table.

#include <cmath>
#include <string>

#include "runtime/internal.hpp"
#include "scicompute_attention/attention_config.hpp"
#include "scicompute_attention/detail/layout_traits.hpp"
#include "scicompute_attention/status.hpp"

namespace sca {
namespace {

std::string SupportedHeadDims() {
    std::string list;
    for (int64_t i = 0; i < kNumSupportedHeadDims; ++i) {
        if (i > 0) list += ',';
        list += std::to_string(kSupportedHeadDims[i]);
    }
    return list;
}

// Backends the softcap option is not available on (api_validate.cpp:23-26).
bool RejectsSoftcap(BackendKind kind) noexcept {
    return kind == BackendKind::kNaive || kind == BackendKind::kTiled ||
           kind == BackendKind::kDecode || kind == BackendKind::kPaged;
}

std::string AtLeastOne(const char* field, int64_t value) {
    return std::string("AttentionShape invalid: ") + field + "=" + std::to_string(value) +
           " (must be >= 1)";
}

}  // namespace

float EffectiveScale(const AttentionConfig& cfg, const AttentionShape& shape) noexcept {
    if (cfg.scale > 0.0f) return cfg.scale;
    if (shape.head_dim <= 0) return 0.0f;
    // 1/sqrt(D) in double, rounded once to float (api_validate.cpp:31-35).
    return static_cast<float>(1.0 / std::sqrt(static_cast<double>(shape.head_dim)));
}

sci::Status Validate(const AttentionConfig& cfg, const AttentionShape& shape, std::string* detail) {
    std::string why;
    AttnStatusCode code = AttnStatusCode::kOk;
    auto reject = [&](AttnStatusCode c, std::string msg) {
        code = c;
        why = std::move(msg);
    };

    if (!detail::LayoutSupported(cfg.layout)) {
        reject(AttnStatusCode::kUnsupportedLayout,
               "AttentionConfig invalid: layout=" + std::to_string(static_cast<int>(cfg.layout)) +
                   " (supported: bhsd, bshd)");
    } else if (shape.batch < 1) {
        reject(AttnStatusCode::kShapeMismatch, AtLeastOne("batch", shape.batch));
    } else if (shape.seq_q < 1) {
        reject(AttnStatusCode::kShapeMismatch, AtLeastOne("seq_q", shape.seq_q));
    } else if (shape.seq_kv < 1) {
        reject(AttnStatusCode::kShapeMismatch, AtLeastOne("seq_kv", shape.seq_kv));
    } else if (shape.num_heads < 1) {
        reject(AttnStatusCode::kShapeMismatch, AtLeastOne("num_heads", shape.num_heads));
    } else if (shape.num_kv_heads < 1) {
        reject(AttnStatusCode::kShapeMismatch, AtLeastOne("num_kv_heads", shape.num_kv_heads));
    } else if (SupportedHeadDimIndex(shape.head_dim) < 0) {
        reject(AttnStatusCode::kUnsupportedHeadDim,
               "AttentionConfig invalid: head_dim=" + std::to_string(shape.head_dim) +
                   " (supported: " + SupportedHeadDims() + ")");
    } else if (shape.num_heads % shape.num_kv_heads != 0) {
        reject(AttnStatusCode::kShapeMismatch,
               "AttentionShape invalid: num_heads=" + std::to_string(shape.num_heads) +
                   " % num_kv_heads=" + std::to_string(shape.num_kv_heads) +
                   " != 0 (GQA requires an integer group size)");
    } else if (cfg.causal && shape.seq_kv < shape.seq_q) {
        reject(AttnStatusCode::kShapeMismatch,
               "AttentionConfig invalid: causal=true but seq_kv(" + std::to_string(shape.seq_kv) +
                   ") < seq_q(" + std::to_string(shape.seq_q) + ")");
    } else if (shape.num_kv_heads > shape.num_heads) {
        reject(AttnStatusCode::kShapeMismatch,
               "AttentionShape invalid: num_kv_heads=" + std::to_string(shape.num_kv_heads) +
                   " > num_heads=" + std::to_string(shape.num_heads) +
                   " (MQA/GQA require H_kv <= H_q)");
    } else if (cfg.sliding_window > 0) {
        reject(AttnStatusCode::kUnsupportedFeature,
               "AttentionConfig invalid: sliding_window=" + std::to_string(cfg.sliding_window) +
                   " is not implemented in v1 (see README Roadmap)");
    } else if (cfg.softcap < 0.0f) {
        reject(AttnStatusCode::kShapeMismatch,
               "AttentionConfig invalid: softcap=" + std::to_string(cfg.softcap) +
                   " (must be 0 or > 0)");
    } else if (cfg.softcap > 0.0f && RejectsSoftcap(cfg.backend)) {
        reject(AttnStatusCode::kUnsupportedFeature,
               "AttentionConfig invalid: softcap=" + std::to_string(cfg.softcap) +
                   " is implemented in the flash backend only, backend=" +
                   BackendName(cfg.backend));
    } else if (cfg.scale < 0.0f) {
        reject(AttnStatusCode::kShapeMismatch,
               "AttentionConfig invalid: scale=" + std::to_string(cfg.scale) +
                   " (must be 0 for the 1/sqrt(head_dim) default or > 0)");
    } else if (cfg.num_splits < 0) {
        reject(AttnStatusCode::kShapeMismatch,
               "AttentionConfig invalid: num_splits=" + std::to_string(cfg.num_splits) +
                   " (must be >= 0)");
    } else if (cfg.cu_seqlens_q != nullptr && cfg.cu_seqlens_kv == nullptr) {
        reject(AttnStatusCode::kShapeMismatch,
               "AttentionConfig invalid: cu_seqlens_q is set but cu_seqlens_kv is null");
    }

    if (code == AttnStatusCode::kOk) {
        if (detail != nullptr) *detail = "ok";
        return sci::Status::Ok();
    }
    if (detail != nullptr) *detail = why;
    return MakeStatus(code, why);
}

TileConfig RecommendTile(const AttentionConfig& cfg, const AttentionShape& shape) {
    (void)cfg;
    TileConfig tile;
    if (SupportedHeadDimIndex(shape.head_dim) < 0) return tile;
    int32_t bm = 0, bn = 0, waves = 0, stages = 0;
    if (sca_hip_flash_tile(static_cast<int32_t>(shape.head_dim), &bm, &bn, &waves, &stages) != 0) {
        return tile;
    }
    tile.block_m = bm;
    tile.block_n = bn;
    tile.warps = waves;
    tile.stages = stages;
    tile.use_tma = false;
    return tile;
}

sci::Status ValidateVarlenHost(const int32_t* host_cu_seqlens, int64_t batch,
                               int64_t* max_seq_out) {
    if (host_cu_seqlens == nullptr) {
        return MakeStatus(AttnStatusCode::kShapeMismatch, "cu_seqlens is null");
    }
    if (batch < 1) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "varlen batch=" + std::to_string(batch) + " (must be >= 1)");
    }
    if (host_cu_seqlens[0] != 0) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "cu_seqlens[0]=" + std::to_string(host_cu_seqlens[0]) +
                              " (must start at 0)");
    }
    int64_t longest = 0;
    for (int64_t i = 0; i < batch; ++i) {
        const int32_t lo = host_cu_seqlens[i];
        const int32_t hi = host_cu_seqlens[i + 1];
        if (hi <= lo) {
            return MakeStatus(AttnStatusCode::kShapeMismatch,
                              "cu_seqlens not strictly increasing at index " + std::to_string(i) +
                                  ": [" + std::to_string(lo) + ", " + std::to_string(hi) + "]");
        }
        if (hi - lo > longest) longest = hi - lo;
    }
    if (max_seq_out != nullptr) *max_seq_out = longest;
    return sci::Status::Ok();
}

}  // namespace sca

// Top-level entry points (the reference's src/api/attention_api.cpp:1-50): infer the shape,
// validate, dispatch, execute. No exception escapes.

#include <string>

#include "scicompute_attention/attention.hpp"

namespace sca {

sci::Result<AttentionResult> attention(const sci::Tensor& q, const sci::Tensor& k,
                                       const sci::Tensor& v, const AttentionConfig& cfg) {
    const AttentionDispatcher dispatcher(cfg);
    return dispatcher.Forward(q, k, v, cfg);
}

sci::Result<AttentionResult> decode(const sci::Tensor& q, const sci::Tensor& k,
                                    const sci::Tensor& v, const AttentionConfig& cfg) {
    AttentionConfig c = cfg;
    c.backend = BackendKind::kDecode;
    return attention(q, k, v, c);
}

sci::Result<AttentionResult> paged(const sci::Tensor& q, const PagedKVCache& kv,
                                   const AttentionConfig& cfg) {
    AttentionConfig c = cfg;
    c.backend = BackendKind::kPaged;
    // The cache's own page size (the params default of 16 would misread other page sizes).
    PagedAttentionParams params;
    params.block_size = kv.BlockSize();
    return paged_attention(q, kv, params, c);
}

std::string ExplainAttention(const sci::Tensor& q, const sci::Tensor& k, const sci::Tensor& v,
                             const AttentionConfig& cfg) {
    const sci::Result<AttentionShape> shape = InferShape(q, k, v, cfg.layout);
    if (!shape.ok()) return "invalid: " + shape.message();
    return AttentionDispatcher(cfg).Explain(cfg, *shape);
}

}  // namespace sca

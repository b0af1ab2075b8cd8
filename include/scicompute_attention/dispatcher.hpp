#pragma once

#include <cstddef>
#include <string>

#include "core/status.hpp"

#include "scicompute_attention/attention_config.hpp"
#include "scicompute_attention/attention_result.hpp"
#include "scicompute_attention/export.hpp"

namespace sca {

struct DispatchDecision {
    BackendKind backend{BackendKind::kAuto};   // kAuto = the request was invalid
    TileConfig tile{};
    size_t workspace_bytes{0};
    // "<auto|explicit|fallback|invalid>: <why> [table=<rev>, ...]"
    std::string reason;
};

// Table-driven backend selection plus execution. Explain() renders the decision of the very same
// Select() that Forward() executes, so the two cannot disagree.
class SCI_ATTENTION_API AttentionDispatcher {
public:
    AttentionDispatcher() = default;
    explicit AttentionDispatcher(const AttentionConfig& default_cfg) : default_cfg_(default_cfg) {}

    DispatchDecision Select(const AttentionConfig& cfg, const AttentionShape& shape) const;

    sci::Result<AttentionResult> Forward(const sci::Tensor& q, const sci::Tensor& k,
                                         const sci::Tensor& v, const AttentionConfig& cfg) const;
    sci::Result<AttentionResult> Forward(const sci::Tensor& q, const sci::Tensor& k,
                                         const sci::Tensor& v) const;

    // "backend=<name>; tile={<tile>}; workspace=<n> B; reason=<reason>"
    std::string Explain(const AttentionConfig& cfg, const AttentionShape& shape) const;

    // nullptr keeps the compiled-in table; loading a table from a file is not implemented.
    static sci::Status ReloadDispatchTable(const char* path = nullptr);

    const AttentionConfig& DefaultConfig() const noexcept { return default_cfg_; }

private:
    AttentionConfig default_cfg_{};
};

// Attention shape of q/k/v read through the tensors in the given layout (4-D, contiguous,
// same compute dtype, GPU-resident).
SCI_ATTENTION_API sci::Result<AttentionShape> InferShape(const sci::Tensor& q, const sci::Tensor& k,
                                                         const sci::Tensor& v, AttnLayout layout);

}  // namespace sca

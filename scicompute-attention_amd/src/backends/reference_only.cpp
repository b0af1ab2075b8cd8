// The reference's score-materialising backends (naive: the full S_q x S_kv FP32 score matrix in
// HBM; tiled: SIMT tiles for short sequences). Neither is built for the MI355X: the flash kernel
// serves every sequence length without a score workspace. Their registry entries answer
// Supports() with the reason and their entry points return kUnsupportedFeature, so a request that
// names them explicitly fails loudly instead of being rerouted.

#include <string>

#include "runtime/internal.hpp"
#include "scicompute_attention/naive_attention.hpp"
#include "scicompute_attention/tiled_attention.hpp"

namespace sca {
namespace {

class ReferenceOnlyBackend final : public IAttentionBackend {
public:
    explicit ReferenceOnlyBackend(BackendKind kind) : kind_(kind) {}
    BackendKind Kind() const noexcept override { return kind_; }
    const char* Name() const noexcept override { return BackendName(kind_); }

    CapabilityReport Supports(const AttentionConfig&, const AttentionShape&) const override {
        CapabilityReport report;
        report.supported = false;
        report.recommended_backend = BackendKind::kFlash;
        report.reason = Reason();
        return report;
    }
    size_t WorkspaceBytes(const AttentionConfig&, const AttentionShape&) const override { return 0; }
    sci::Result<AttentionResult> Forward(const sci::Tensor&, const sci::Tensor&, const sci::Tensor&,
                                         const AttentionConfig&) const override {
        return sci::MakeUnexpected<AttentionResult>(
            MakeStatus(AttnStatusCode::kUnsupportedFeature, Reason()));
    }
    sci::Result<AttentionResult> ForwardVarlen(const sci::Tensor&, const sci::Tensor&,
                                               const sci::Tensor&, int64_t, const int32_t*,
                                               const int32_t*, int64_t, int64_t,
                                               const AttentionConfig&) const override {
        return sci::MakeUnexpected<AttentionResult>(
            MakeStatus(AttnStatusCode::kUnsupportedFeature, Reason()));
    }

private:
    std::string Reason() const {
        return std::string(BackendName(kind_)) +
               " backend is not built for MI355X (score-materialising reference kernel); use "
               "backend=flash (prefill) or decode/paged (S_q=1)";
    }
    BackendKind kind_;
};

const ReferenceOnlyBackend kNaive(BackendKind::kNaive);
const ReferenceOnlyBackend kTiled(BackendKind::kTiled);

}  // namespace

namespace runtime {
const IAttentionBackend* NaiveBackendInstance() noexcept { return &kNaive; }
const IAttentionBackend* TiledBackendInstance() noexcept { return &kTiled; }
}  // namespace runtime

sci::Result<AttentionResult> naive_attention(const sci::Tensor& q, const sci::Tensor& k,
                                             const sci::Tensor& v, const AttentionConfig& cfg) {
    return kNaive.Forward(q, k, v, cfg);
}

sci::Result<AttentionResult> tiled_attention(const sci::Tensor& q, const sci::Tensor& k,
                                             const sci::Tensor& v, const AttentionConfig& cfg) {
    return kTiled.Forward(q, k, v, cfg);
}

}  // namespace sca

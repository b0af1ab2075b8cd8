// Shape inference, table-driven backend selection and execution.
// Decision procedure, reason-string grammar and fallback chains follow the reference's
// src/runtime/dispatcher.cpp:19-232 so that Explain() output parses the same way; the thresholds
// are the MI355X table of runtime/dispatch_table.hpp.

#include <string>
#include <vector>

#include "runtime/dispatch_table.hpp"
#include "runtime/internal.hpp"
#include "scicompute_attention/detail/layout_traits.hpp"
#include "scicompute_attention/dispatcher.hpp"

namespace sca {
namespace {

// Backends tried, in order, when the preferred one cannot serve and the caller allowed fallback.
std::vector<BackendKind> FallbackChain(BackendKind preferred) {
    switch (preferred) {
        case BackendKind::kFlash: return {BackendKind::kTiled, BackendKind::kNaive};
        case BackendKind::kDecode:
            return {BackendKind::kFlash, BackendKind::kTiled, BackendKind::kNaive};
        case BackendKind::kPaged:
            return {BackendKind::kDecode, BackendKind::kTiled, BackendKind::kNaive};
        case BackendKind::kTiled: return {BackendKind::kNaive};
        default: return {};
    }
}

std::string ShapeText(const AttentionShape& s) {
    return "B=" + std::to_string(s.batch) + ",Hq=" + std::to_string(s.num_heads) +
           ",Hkv=" + std::to_string(s.num_kv_heads) + ",Sq=" + std::to_string(s.seq_q) +
           ",Skv=" + std::to_string(s.seq_kv) + ",D=" + std::to_string(s.head_dim);
}

std::string Dims(const sci::Tensor& t) {
    std::string out = "[";
    for (sci::index_t i = 0; i < t.ndims(); ++i) {
        if (i > 0) out += ",";
        out += std::to_string(t.dim(static_cast<size_t>(i)));
    }
    return out + "]";
}

sci::Result<AttentionShape> ShapeError(AttnStatusCode code, std::string msg) {
    return sci::MakeUnexpected<AttentionShape>(MakeStatus(code, std::move(msg)));
}

}  // namespace

sci::Result<AttentionShape> InferShape(const sci::Tensor& q, const sci::Tensor& k,
                                       const sci::Tensor& v, AttnLayout layout) {
    if (!detail::LayoutSupported(layout)) {
        return ShapeError(AttnStatusCode::kUnsupportedLayout,
                          std::string("layout=") + LayoutName(layout) + " (supported: bhsd, bshd)");
    }
    for (const sci::Tensor* t : {&q, &k, &v}) {
        if (t->ndims() != 4) {
            return ShapeError(AttnStatusCode::kShapeMismatch,
                              "tensor ndims=" + std::to_string(t->ndims()) + " (expected 4)");
        }
        if (!t->is_contiguous()) {
            return ShapeError(AttnStatusCode::kLayoutMismatch,
                              "non-contiguous input rejected; call .clone() or pass a contiguous "
                              "tensor");
        }
        if (!IsSupportedComputeDtype(t->dtype())) {
            return ShapeError(AttnStatusCode::kUnsupportedDtype,
                              std::string("dtype=") + sci::kDTypeName(t->dtype()) +
                                  " (supported: float32, float16, bfloat16)");
        }
        if (t->device_type() != sci::DeviceType::kGPU) {
            return ShapeError(AttnStatusCode::kUnsupportedFeature,
                              std::string("device=") + sci::kDeviceTypeName(t->device_type()) +
                                  " (attention kernels execute on the GPU only)");
        }
    }
    if (q.dtype() != k.dtype() || q.dtype() != v.dtype()) {
        return ShapeError(AttnStatusCode::kUnsupportedDtype,
                          std::string("dtype mismatch: q=") + sci::kDTypeName(q.dtype()) +
                              ", k=" + sci::kDTypeName(k.dtype()) +
                              ", v=" + sci::kDTypeName(v.dtype()));
    }
    // Axis positions of (S, H) in the two layouts.
    const size_t s_axis = layout == AttnLayout::kBHSD ? 2 : 1;
    const size_t h_axis = layout == AttnLayout::kBHSD ? 1 : 2;
    AttentionShape shape;
    shape.batch = q.dim(0);
    shape.num_heads = q.dim(h_axis);
    shape.seq_q = q.dim(s_axis);
    shape.head_dim = q.dim(3);
    shape.num_kv_heads = k.dim(h_axis);
    shape.seq_kv = k.dim(s_axis);
    if (v.dim(h_axis) != shape.num_kv_heads || v.dim(s_axis) != shape.seq_kv ||
        v.dim(3) != shape.head_dim || k.dim(3) != shape.head_dim) {
        return ShapeError(AttnStatusCode::kShapeMismatch,
                          std::string("k/v shape mismatch (") + LayoutName(layout) + "): q=" +
                              Dims(q) + ", k=" + Dims(k) + ", v=" + Dims(v));
    }
    if (k.dim(0) != shape.batch || v.dim(0) != shape.batch) {
        return ShapeError(AttnStatusCode::kShapeMismatch,
                          "batch mismatch: q=" + std::to_string(shape.batch) +
                              ", k=" + std::to_string(k.dim(0)) + ", v=" + std::to_string(v.dim(0)));
    }
    return sci::Ok(shape);
}

DispatchDecision AttentionDispatcher::Select(const AttentionConfig& cfg,
                                             const AttentionShape& shape) const {
    DispatchDecision decision;
    std::string invalid;
    if (!Validate(cfg, shape, &invalid).ok()) {
        decision.backend = BackendKind::kAuto;
        decision.reason = "invalid: " + invalid;
        return decision;
    }
    const auto& th = detail::kDispatchThresholds;
    const std::string table = std::string(" [table=") + th.revision;

    BackendKind preferred = cfg.backend;
    std::string rule;
    if (preferred != BackendKind::kAuto) {
        rule = std::string("explicit: backend=") + BackendName(preferred);
    } else if (shape.seq_q <= th.decode_max_seq_q && shape.seq_kv >= th.decode_min_seq_kv) {
        preferred = BackendKind::kDecode;
        rule = "auto: seq_q=" + std::to_string(shape.seq_q) + " <=" +
               std::to_string(th.decode_max_seq_q) + " and seq_kv=" + std::to_string(shape.seq_kv) +
               " >= " + std::to_string(th.decode_min_seq_kv) + " => decode (low arithmetic intensity)";
    } else if (shape.seq_q * 8 <= shape.seq_kv && shape.seq_kv >= th.decode_min_seq_kv) {
        preferred = BackendKind::kFlash;
        rule = "auto: seq_q*8=" + std::to_string(shape.seq_q * 8) + " <= seq_kv=" +
               std::to_string(shape.seq_kv) +
               " => grouped small-q prefill on flash (decode kernel is S_q=1 only)";
    } else if (shape.seq_kv <= th.short_max_seq_kv) {
        preferred = BackendKind::kFlash;
        rule = "auto: seq_kv=" + std::to_string(shape.seq_kv) + " <= " +
               std::to_string(th.short_max_seq_kv) +
               " => flash (short sequence, one KV tile pass, no score workspace)";
    } else {
        preferred = BackendKind::kFlash;
        rule = "auto: seq_q=" + std::to_string(shape.seq_q) + ", seq_kv=" +
               std::to_string(shape.seq_kv) + " => flash (tile + online softmax)";
    }

    decision.backend = preferred;
    decision.tile = RecommendTile(cfg, shape);
    const CapabilityReport report = GetBackend(preferred)->Supports(cfg, shape);
    decision.workspace_bytes = report.workspace_bytes;
    if (report.supported) {
        if (!report.tile.Empty()) decision.tile = report.tile;
        decision.reason = rule + table + ", workspace=" + std::to_string(report.workspace_bytes) +
                          " B]";
        return decision;
    }
    const std::string refusal = rule + " => unsupported(" + BackendName(preferred) +
                                "): " + report.reason;
    if (!cfg.allow_fallback) {
        decision.reason = refusal + table + ", allow_fallback=false]";
        return decision;
    }
    for (BackendKind candidate : FallbackChain(preferred)) {
        const CapabilityReport alt = GetBackend(candidate)->Supports(cfg, shape);
        if (!alt.supported) continue;
        decision.backend = candidate;
        if (!alt.tile.Empty()) decision.tile = alt.tile;
        decision.workspace_bytes = alt.workspace_bytes;
        decision.reason = std::string("fallback: ") + BackendName(preferred) + " unsupported (" +
                          report.reason + ") => " + BackendName(candidate) + "; " + rule + table +
                          ", allow_fallback=true]";
        return decision;
    }
    decision.reason = refusal + "; no fallback backend supports shape " + ShapeText(shape);
    return decision;
}

std::string AttentionDispatcher::Explain(const AttentionConfig& cfg,
                                         const AttentionShape& shape) const {
    const DispatchDecision d = Select(cfg, shape);
    return std::string("backend=") + BackendName(d.backend) + "; tile={" + d.tile.ToString() +
           "}; workspace=" + std::to_string(d.workspace_bytes) + " B; reason=" + d.reason;
}

sci::Result<AttentionResult> AttentionDispatcher::Forward(const sci::Tensor& q,
                                                          const sci::Tensor& k,
                                                          const sci::Tensor& v,
                                                          const AttentionConfig& cfg) const {
    const sci::Result<AttentionShape> shape = InferShape(q, k, v, cfg.layout);
    if (!shape.ok()) return sci::MakeUnexpected<AttentionResult>(shape.error());
    const DispatchDecision decision = Select(cfg, *shape);
    if (decision.backend == BackendKind::kAuto) {
        return sci::MakeUnexpected<AttentionResult>(
            MakeStatus(AttnStatusCode::kShapeMismatch, decision.reason));
    }
    const IAttentionBackend* backend = GetBackend(decision.backend);
    const CapabilityReport report = backend->Supports(cfg, *shape);
    if (!report.supported) {
        return sci::MakeUnexpected<AttentionResult>(
            MakeStatus(AttnStatusCode::kDeviceCapability, report.reason));
    }
    return backend->Forward(q, k, v, cfg);
}

sci::Result<AttentionResult> AttentionDispatcher::Forward(const sci::Tensor& q,
                                                          const sci::Tensor& k,
                                                          const sci::Tensor& v) const {
    return Forward(q, k, v, default_cfg_);
}

sci::Status AttentionDispatcher::ReloadDispatchTable(const char* path) {
    if (path == nullptr) return sci::Status::Ok();
    return sci::Status::NotImplemented(
        std::string("loading a dispatch table from a file is not implemented; the compiled-in "
                    "table \"") +
        detail::kDispatchThresholds.revision + "\" is in use");
}

// ---- backend registry ----------------------------------------------------------------------

const IAttentionBackend* GetBackend(BackendKind kind) noexcept {
    switch (kind) {
        case BackendKind::kTiled: return runtime::TiledBackendInstance();
        case BackendKind::kFlash: return runtime::FlashBackendInstance();
        case BackendKind::kDecode: return runtime::DecodeBackendInstance();
        case BackendKind::kPaged: return runtime::PagedBackendInstance();
        case BackendKind::kNaive:
        case BackendKind::kAuto: break;
    }
    return runtime::NaiveBackendInstance();
}

const char* BackendTypeName(BackendKind kind) noexcept { return BackendName(kind); }

bool ParseBackendName(const char* name, BackendKind* out) noexcept {
    if (name == nullptr || out == nullptr) return false;
    for (BackendKind kind : {BackendKind::kAuto, BackendKind::kNaive, BackendKind::kTiled,
                             BackendKind::kFlash, BackendKind::kDecode, BackendKind::kPaged}) {
        if (std::string(name) == BackendName(kind)) {
            *out = kind;
            return true;
        }
    }
    return false;
}

}  // namespace sca

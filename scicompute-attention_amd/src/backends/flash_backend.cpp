// Flash prefill backend: host adapter of the gfx950 MFMA kernel (sca_hip_flash_fwd).
// Request checks, output allocation (always contiguous BHSD, optional FP32 LSE) and the varlen
// contract follow the reference's src/backends/flash/flash_backend.cpp:43-376.
//
// Guarantees: the S_q x S_kv score matrix never reaches HBM (workspace_bytes == 0 and
// materialized_score_bytes == 0 on every result).

#include <algorithm>
#include <vector>
#include <string>

#include "runtime/internal.hpp"
#include "scicompute_attention/capability.hpp"
#include "scicompute_attention/detail/layout_traits.hpp"
#include "scicompute_attention/dispatcher.hpp"
#include "scicompute_attention/flash_attention.hpp"

namespace sca {
namespace {

// Why flash cannot serve (cfg, shape) on this device, or "" when it can.
std::string FlashRefusal(const AttentionConfig& cfg, const AttentionShape& shape) {
    if (!DeviceCapability::GpuAvailable()) return "no GPU device available";
    const int64_t lds = sca_hip_flash_lds_bytes(static_cast<int32_t>(shape.head_dim), 2);
    if (lds < 0) {
        return "head_dim=" + std::to_string(shape.head_dim) +
               " has no flash tile (supported: 32,64,96,128,160,192,256)";
    }
    if (cfg.sliding_window > 0) {
        return "sliding_window=" + std::to_string(cfg.sliding_window) + " not implemented";
    }
    if (cfg.softcap > 0.0f) {
        return "softcap=" + std::to_string(cfg.softcap) +
               " is not implemented by the MI355X flash kernel";
    }
    const size_t limit = DeviceCapability::SmemLimitPerBlock(DeviceCapability::ForDevice(0));
    if (limit != 0 && static_cast<size_t>(lds) > limit) {
        return "flash tile needs " + std::to_string(lds) + " B of LDS > limit " +
               std::to_string(limit) + " B for head_dim=" + std::to_string(shape.head_dim);
    }
    return "";
}

sci::Status CheckDtype(sci::DType dtype) {
    if (dtype == sci::DType::kFloat16 || dtype == sci::DType::kBFloat16) return sci::Status::Ok();
    return MakeStatus(AttnStatusCode::kUnsupportedDtype,
                      std::string("flash backend computes in fp16/bf16; dtype=") +
                          sci::kDTypeName(dtype) +
                          " is served by the naive (reference) or tiled backend");
}

void FillStats(AttentionRuntimeStats* stats, const TileConfig& tile, const std::string& note) {
    stats->used_backend = BackendKind::kFlash;
    stats->tile = tile;
    stats->workspace_bytes = 0;
    stats->materialized_score_bytes = 0;
    stats->note = note;
}

class FlashBackend final : public IAttentionBackend {
public:
    BackendKind Kind() const noexcept override { return BackendKind::kFlash; }
    const char* Name() const noexcept override { return "flash"; }

    CapabilityReport Supports(const AttentionConfig& cfg,
                              const AttentionShape& shape) const override {
        CapabilityReport report;
        report.recommended_backend = BackendKind::kFlash;
        report.workspace_bytes = 0;
        const std::string refusal = FlashRefusal(cfg, shape);
        report.supported = refusal.empty();
        if (report.supported) {
            report.tile = RecommendTile(cfg, shape);
            report.reason = "online softmax in registers (workspace 0 B), tile " +
                            report.tile.ToString();
        } else {
            report.reason = refusal;
        }
        return report;
    }

    size_t WorkspaceBytes(const AttentionConfig&, const AttentionShape&) const override { return 0; }

    sci::Result<AttentionResult> Forward(const sci::Tensor& q, const sci::Tensor& k,
                                         const sci::Tensor& v,
                                         const AttentionConfig& cfg) const override {
        const sci::Result<AttentionShape> inferred = InferShape(q, k, v, cfg.layout);
        if (!inferred.ok()) return sci::MakeUnexpected<AttentionResult>(inferred.error());
        const AttentionShape shape = *inferred;
        sci::Status status = Validate(cfg, shape);
        if (status.ok()) status = CheckDtype(q.dtype());
        if (!status.ok()) return sci::MakeUnexpected<AttentionResult>(status);
        const std::string refusal = FlashRefusal(cfg, shape);
        if (!refusal.empty()) {
            return sci::MakeUnexpected<AttentionResult>(MakeStatus(
                AttnStatusCode::kUnsupportedFeature, "flash backend: " + refusal));
        }

        sci::Device& device = q.device();
        AttentionResult result;
        result.out = sci::Tensor(sci::TensorShape({shape.batch, shape.num_heads, shape.seq_q,
                                                   shape.head_dim}),
                                 q.dtype(), device);
        if (result.out.data() == nullptr) {
            return sci::MakeUnexpected<AttentionResult>(MakeStatus(
                AttnStatusCode::kWorkspaceExceeded, "allocation of the attention output failed"));
        }
        if (cfg.return_lse) {
            result.lse = sci::Tensor(sci::TensorShape({shape.batch, shape.num_heads, shape.seq_q}),
                                     sci::DType::kFloat32, device);
            if (result.lse.data() == nullptr) {
                return sci::MakeUnexpected<AttentionResult>(MakeStatus(
                    AttnStatusCode::kWorkspaceExceeded, "allocation of the LSE buffer failed"));
            }
        }

        const detail::Strides qs =
            detail::StridesFor(cfg.layout, shape.seq_q, shape.num_heads, shape.head_dim);
        const detail::Strides ks =
            detail::StridesFor(cfg.layout, shape.seq_kv, shape.num_kv_heads, shape.head_dim);
        const detail::Strides os =
            detail::StridesFor(AttnLayout::kBHSD, shape.seq_q, shape.num_heads, shape.head_dim);
        sca_flash_params p{};
        p.q = q.data();
        p.k = k.data();
        p.v = v.data();
        p.out = result.out.data();
        p.lse = cfg.return_lse ? static_cast<float*>(result.lse.data()) : nullptr;
        p.batch = shape.batch;
        p.num_heads = shape.num_heads;
        p.num_kv_heads = shape.num_kv_heads;
        p.seq_q = shape.seq_q;
        p.seq_kv = shape.seq_kv;
        p.head_dim = shape.head_dim;
        p.q_sb = qs.s_b, p.q_sh = qs.s_h, p.q_ss = qs.s_s;
        p.k_sb = ks.s_b, p.k_sh = ks.s_h, p.k_ss = ks.s_s;
        p.v_sb = ks.s_b, p.v_sh = ks.s_h, p.v_ss = ks.s_s;
        p.o_sb = os.s_b, p.o_sh = os.s_h, p.o_ss = os.s_s;
        p.scale = EffectiveScale(cfg, shape);
        p.causal = cfg.causal ? 1 : 0;
        p.dtype = runtime::KernelDtype(q.dtype());
        p.diagonal = cfg.causal ? shape.seq_kv - shape.seq_q : 0;
        status = runtime::StatusFromHip(sca_hip_flash_fwd(&p, runtime::StreamHandle(cfg.stream)),
                                        "flash forward");
        if (!status.ok()) return sci::MakeUnexpected<AttentionResult>(status);

        const TileConfig tile = RecommendTile(cfg, shape);
        FillStats(&result.stats, tile,
                  "flash: gfx950 MFMA 32x32x16, tile " + tile.ToString() +
                      ", S/P in registers; layout=" + LayoutName(cfg.layout));
        return sci::Ok(std::move(result));
    }

    // Packed [T, H, D] inputs with host cu_seqlens: one kernel launch per sequence over the
    // packed buffers (token-major strides, batch 1).
    sci::Result<AttentionResult> ForwardVarlen(const sci::Tensor& q, const sci::Tensor& k,
                                               const sci::Tensor& v, int64_t num_seqs,
                                               const int32_t* cu_q, const int32_t* cu_kv,
                                               int64_t max_seq_q, int64_t max_seq_kv,
                                               const AttentionConfig& cfg) const override {
        auto fail = [](AttnStatusCode code, std::string msg) {
            return sci::MakeUnexpected<AttentionResult>(MakeStatus(code, std::move(msg)));
        };
        if (cu_q == nullptr || cu_kv == nullptr) {
            return fail(AttnStatusCode::kShapeMismatch,
                        "varlen requires host-resident cu_seqlens_q/kv");
        }
        if (num_seqs < 1) {
            return fail(AttnStatusCode::kShapeMismatch,
                        "varlen num_seqs=" + std::to_string(num_seqs) + " (must be >= 1)");
        }
        if (cfg.return_lse) {
            return fail(AttnStatusCode::kUnsupportedFeature,
                        "varlen does not expose LSE yet; call the per-sequence entry point if it "
                        "is needed");
        }
        if (cfg.causal && max_seq_kv < max_seq_q) {
            return fail(AttnStatusCode::kShapeMismatch,
                        "varlen causal requires max_seq_kv >= max_seq_q");
        }
        for (const sci::Tensor* t : {&q, &k, &v}) {
            if (t->ndims() != 3) {
                return fail(AttnStatusCode::kShapeMismatch,
                            "varlen expects packed [T, H, D] tensors; got ndims=" +
                                std::to_string(t->ndims()));
            }
            if (t->device_type() != sci::DeviceType::kGPU) {
                return fail(AttnStatusCode::kUnsupportedFeature, "varlen requires GPU tensors");
            }
        }
        if (!CheckDtype(q.dtype()).ok()) {
            return fail(AttnStatusCode::kUnsupportedDtype, "flash varlen supports fp16/bf16 only");
        }
        if (q.dtype() != k.dtype() || q.dtype() != v.dtype()) {
            return fail(AttnStatusCode::kUnsupportedDtype,
                        "varlen requires q/k/v to share one dtype");
        }
        const int64_t num_heads = q.dim(1);
        const int64_t head_dim = q.dim(2);
        const int64_t num_kv_heads = k.dim(1);
        if (k.dim(2) != head_dim || v.dim(2) != head_dim || v.dim(1) != num_kv_heads) {
            return fail(AttnStatusCode::kShapeMismatch,
                        "varlen expects k/v head dims to match q; got D=" +
                            std::to_string(head_dim));
        }
        if (num_kv_heads < 1 || num_heads % num_kv_heads != 0) {
            return fail(AttnStatusCode::kShapeMismatch, "varlen requires H_q % H_kv == 0");
        }
        AttentionShape probe;
        probe.batch = 1;
        probe.seq_q = max_seq_q;
        probe.seq_kv = max_seq_kv;
        probe.num_heads = num_heads;
        probe.num_kv_heads = num_kv_heads;
        probe.head_dim = head_dim;
        const std::string refusal = FlashRefusal(cfg, probe);
        if (!refusal.empty()) {
            return fail(SupportedHeadDimIndex(head_dim) < 0 ? AttnStatusCode::kUnsupportedHeadDim
                                                            : AttnStatusCode::kUnsupportedFeature,
                        "flash backend: " + refusal);
        }
        // Every sequence must lie inside the packed tensors.
        for (int64_t s = 0; s < num_seqs; ++s) {
            const int64_t sq = cu_q[s + 1] - cu_q[s];
            const int64_t skv = cu_kv[s + 1] - cu_kv[s];
            if (sq <= 0 || skv <= 0) {
                return fail(AttnStatusCode::kShapeMismatch,
                            "varlen sequence " + std::to_string(s) + " has S_q=" +
                                std::to_string(sq) + ", S_kv=" + std::to_string(skv) +
                                " (both must be > 0)");
            }
            if (cu_q[s] < 0 || cu_q[s + 1] > q.dim(0) || cu_kv[s] < 0 ||
                cu_kv[s + 1] > k.dim(0) || cu_kv[s + 1] > v.dim(0)) {
                return fail(AttnStatusCode::kShapeMismatch,
                            "varlen sequence " + std::to_string(s) +
                                " exceeds the packed tensors (T_q=" + std::to_string(q.dim(0)) +
                                ", T_kv=" + std::to_string(k.dim(0)) + ")");
            }
            if (cfg.causal && skv < sq) {
                return fail(AttnStatusCode::kShapeMismatch,
                            "varlen sequence " + std::to_string(s) + ": causal needs S_kv(" +
                                std::to_string(skv) + ") >= S_q(" + std::to_string(sq) + ")");
            }
        }

        AttentionResult result;
        result.out = sci::Tensor(sci::TensorShape({q.dim(0), num_heads, head_dim}), q.dtype(),
                                 q.device());
        if (result.out.data() == nullptr) {
            return fail(AttnStatusCode::kWorkspaceExceeded,
                        "allocation of the varlen output failed");
        }
        const int64_t eb = DtypeSize(q.dtype());
        const int64_t q_token = num_heads * head_dim;
        const int64_t kv_token = num_kv_heads * head_dim;
        const float scale = EffectiveScale(cfg, probe);
        void* stream = runtime::StreamHandle(cfg.stream);
        if (sca_hip_flash_varlen_supported(static_cast<int32_t>(head_dim))) {
            // One launch over the whole packing: cu_seqlens and the longest-first tile list go
            // up together into a scratch buffer.
            const int32_t causal = cfg.causal ? 1 : 0;
            const int64_t n_tiles =
                sca_hip_flash_varlen_tiles(cu_q, cu_kv, num_seqs, causal, nullptr);
            if (n_tiles < 0) {
                return fail(AttnStatusCode::kShapeMismatch, sca_hip_last_error_string());
            }
            std::vector<int32_t> table(static_cast<size_t>(2 * (num_seqs + 1) + 2 * n_tiles));
            std::copy(cu_q, cu_q + num_seqs + 1, table.begin());
            std::copy(cu_kv, cu_kv + num_seqs + 1, table.begin() + (num_seqs + 1));
            sca_hip_flash_varlen_tiles(cu_q, cu_kv, num_seqs, causal,
                                       table.data() + 2 * (num_seqs + 1));
            int64_t max_kv = 0;
            for (int64_t s = 0; s < num_seqs; ++s) {
                max_kv = std::max<int64_t>(max_kv, cu_kv[s + 1] - cu_kv[s]);
            }
            sci::Result<void*> dev =
                runtime::UploadToScratch(runtime::ScratchKind::kVarlenTables, table.data(),
                                         table.size() * sizeof(int32_t), q.device().id(), stream);
            if (!dev.ok()) return sci::MakeUnexpected<AttentionResult>(dev.error());
            const int32_t* d = static_cast<const int32_t*>(*dev);
            sca_flash_varlen_params vp{};
            vp.q = q.data();
            vp.k = k.data();
            vp.v = v.data();
            vp.out = result.out.data();
            vp.cu_seqlens_q = d;
            vp.cu_seqlens_kv = d + (num_seqs + 1);
            vp.tiles = d + 2 * (num_seqs + 1);
            vp.num_seqs = num_seqs;
            vp.num_tiles = n_tiles;
            vp.max_seq_kv = max_kv;
            vp.num_heads = num_heads;
            vp.num_kv_heads = num_kv_heads;
            vp.head_dim = head_dim;
            vp.q_sh = head_dim, vp.q_ss = q_token;
            vp.k_sh = head_dim, vp.k_ss = kv_token;
            vp.v_sh = head_dim, vp.v_ss = kv_token;
            vp.o_sh = head_dim, vp.o_ss = q_token;
            vp.scale = scale;
            vp.causal = causal;
            vp.dtype = runtime::KernelDtype(q.dtype());
            const sci::Status status = runtime::StatusFromHip(
                sca_hip_flash_fwd_varlen(&vp, stream), "flash varlen forward");
            if (!status.ok()) return sci::MakeUnexpected<AttentionResult>(status);
            const TileConfig tile = RecommendTile(cfg, probe);
            FillStats(&result.stats, tile,
                      "varlen: one launch over " + std::to_string(num_seqs) + " packed sequences, " +
                          std::to_string(n_tiles) + " row tiles longest first (tile " +
                          tile.ToString() + ")");
            return sci::Ok(std::move(result));
        }
        for (int64_t s = 0; s < num_seqs; ++s) {
            const int64_t sq = cu_q[s + 1] - cu_q[s];
            const int64_t skv = cu_kv[s + 1] - cu_kv[s];
            sca_flash_params p{};
            p.q = static_cast<const char*>(q.data()) + cu_q[s] * q_token * eb;
            p.k = static_cast<const char*>(k.data()) + cu_kv[s] * kv_token * eb;
            p.v = static_cast<const char*>(v.data()) + cu_kv[s] * kv_token * eb;
            p.out = static_cast<char*>(result.out.data()) + cu_q[s] * q_token * eb;
            p.lse = nullptr;
            p.batch = 1;
            p.num_heads = num_heads;
            p.num_kv_heads = num_kv_heads;
            p.seq_q = sq;
            p.seq_kv = skv;
            p.head_dim = head_dim;
            p.q_sb = sq * q_token, p.q_sh = head_dim, p.q_ss = q_token;
            p.k_sb = skv * kv_token, p.k_sh = head_dim, p.k_ss = kv_token;
            p.v_sb = p.k_sb, p.v_sh = p.k_sh, p.v_ss = p.k_ss;
            p.o_sb = sq * q_token, p.o_sh = head_dim, p.o_ss = q_token;
            p.scale = scale;
            p.causal = cfg.causal ? 1 : 0;
            p.dtype = runtime::KernelDtype(q.dtype());
            p.diagonal = cfg.causal ? skv - sq : 0;
            const sci::Status status =
                runtime::StatusFromHip(sca_hip_flash_fwd(&p, stream), "flash varlen forward");
            if (!status.ok()) return sci::MakeUnexpected<AttentionResult>(status);
        }
        const TileConfig tile = RecommendTile(cfg, probe);
        FillStats(&result.stats, tile,
                  "varlen: " + std::to_string(num_seqs) +
                      " per-sequence launches over packed buffers (tile " + tile.ToString() + ")");
        return sci::Ok(std::move(result));
    }
};

const FlashBackend kFlashBackend;

}  // namespace

namespace runtime {
const IAttentionBackend* FlashBackendInstance() noexcept { return &kFlashBackend; }
}  // namespace runtime

sci::Result<AttentionResult> flash_attention(const sci::Tensor& q, const sci::Tensor& k,
                                             const sci::Tensor& v, const AttentionConfig& cfg) {
    return kFlashBackend.Forward(q, k, v, cfg);
}

sci::Result<AttentionResult> flash_attention_varlen(const sci::Tensor& q, const sci::Tensor& k,
                                                    const sci::Tensor& v, int64_t num_seqs,
                                                    const int32_t* cu_seqlens_q,
                                                    const int32_t* cu_seqlens_kv, int64_t max_seq_q,
                                                    int64_t max_seq_kv,
                                                    const AttentionConfig& cfg) {
    return kFlashBackend.ForwardVarlen(q, k, v, num_seqs, cu_seqlens_q, cu_seqlens_kv, max_seq_q,
                                       max_seq_kv, cfg);
}

int64_t FlashLdsBytes(int64_t head_dim, int64_t elem_bytes) {
    return sca_hip_flash_lds_bytes(static_cast<int32_t>(head_dim), elem_bytes);
}

}  // namespace sca

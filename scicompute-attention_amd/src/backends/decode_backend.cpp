// Split-K decode backend (S_q == 1) and the paged decode entry points: host adapters of
// sca_hip_decode_splitk / sca_hip_decode_splitk_paged.
// Request checks and partial-scratch layout follow the reference's
// src/backends/decode/decode_backend.cpp:53-214 and src/backends/paged/paged_backend.cpp:40-253;
// the split count comes from the MI355X dispatch table (runtime/dispatch_table.hpp).

#include <string>
#include <vector>

#include "runtime/dispatch_table.hpp"
#include "runtime/internal.hpp"
#include "scicompute_attention/capability.hpp"
#include "scicompute_attention/decode_attention.hpp"
#include "scicompute_attention/detail/layout_traits.hpp"
#include "scicompute_attention/dispatcher.hpp"
#include "scicompute_attention/paged_attention.hpp"

namespace sca {
namespace {

constexpr int64_t kNativeSeqQ = 1;

int64_t PartialElements(int64_t batch, int64_t heads, int64_t splits, int64_t head_dim) {
    return sca_hip_decode_partial_elements(batch, heads, splits, head_dim);
}

// Explicit split counts are honoured up to the table's cap; otherwise the table decides.
int64_t ResolveSplits(int64_t requested, int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                      int64_t seq_kv, int64_t head_dim, int slot_waves = 4) {
    const auto& th = detail::kDispatchThresholds;
    if (requested > 0) return requested < th.max_splits ? requested : th.max_splits;
    return detail::DecodeSplits(batch, num_heads, num_kv_heads, seq_kv,
                                DeviceCapability::ForDevice(0).sm_count, slot_waves, head_dim);
}

// Points the partial pointers of `p` into the pooled FP32 scratch (m | l | O).
// Binds the FP32 partials (splits > 1) and, for ragged lengths, the 2*batch int32 schedule the
// kernels sort the sequences into, both from the decode scratch buffer.
sci::Status BindPartials(sca_decode_params* p, int64_t splits, int device_id, size_t* bytes) {
    const int64_t partials =
        splits == 1 ? 0 : PartialElements(p->batch, p->num_heads, splits, p->head_dim);
    const int64_t order = p->seq_lens != nullptr ? 2 * p->batch : 0;
    const int64_t elements = partials + order;
    *bytes = static_cast<size_t>(partials) * sizeof(float);
    p->partial_m = p->partial_l = p->partial_o = nullptr;
    p->batch_order = nullptr;
    if (elements == 0) return sci::Status::Ok();  // splits == 1 writes the output directly
    sci::Result<float*> scratch = runtime::AcquireScratchFp32(
        runtime::ScratchKind::kDecodePartials, static_cast<size_t>(elements), device_id);
    if (!scratch.ok()) return scratch.error();
    if (partials > 0) {
        const int64_t base = p->batch * p->num_heads * splits;
        p->partial_m = *scratch;
        p->partial_l = *scratch + base;
        p->partial_o = *scratch + 2 * base;
    }
    if (order > 0) {
        // partials is even (base * (2 + head_dim) with an even head_dim): 8-byte aligned.
        p->batch_order = reinterpret_cast<int32_t*>(*scratch + partials);
    }
    return sci::Status::Ok();
}

class DecodeBackend final : public IAttentionBackend {
public:
    BackendKind Kind() const noexcept override { return BackendKind::kDecode; }
    const char* Name() const noexcept override { return "decode"; }

    CapabilityReport Supports(const AttentionConfig& cfg,
                              const AttentionShape& shape) const override {
        CapabilityReport report;
        report.recommended_backend = BackendKind::kDecode;
        const int64_t splits = ResolveSplits(cfg.num_splits, shape.batch, shape.num_heads,
                                             shape.num_kv_heads, shape.seq_kv, shape.head_dim);
        report.workspace_bytes = WorkspaceBytes(cfg, shape);
        std::string reason;
        if (!DeviceCapability::GpuAvailable()) {
            reason = "no GPU device available";
        } else if (shape.seq_q != kNativeSeqQ) {
            reason = "decode kernel handles seq_q=1; seq_q=" + std::to_string(shape.seq_q) +
                     " is routed to the flash backend (grouped decode is a Roadmap item)";
        } else if (SupportedHeadDimIndex(shape.head_dim) < 0) {
            reason = "head_dim=" + std::to_string(shape.head_dim) + " is unsupported";
        } else if (shape.head_dim % 32 != 0) {
            reason = "decode requires head_dim % 32 == 0; head_dim=" +
                     std::to_string(shape.head_dim);
        } else if (cfg.sliding_window > 0) {
            reason = "sliding_window is not implemented by the decode backend";
        }
        report.supported = reason.empty();
        report.reason = report.supported
                            ? "split-K decode with " + std::to_string(splits) +
                                  " splits, workspace " + std::to_string(report.workspace_bytes) +
                                  " B (FP32 partials)"
                            : reason;
        return report;
    }

    size_t WorkspaceBytes(const AttentionConfig& cfg, const AttentionShape& shape) const override {
        const int64_t splits = ResolveSplits(cfg.num_splits, shape.batch, shape.num_heads,
                                             shape.num_kv_heads, shape.seq_kv, shape.head_dim);
        if (splits <= 1) return 0;
        return static_cast<size_t>(
                   PartialElements(shape.batch, shape.num_heads, splits, shape.head_dim)) *
               sizeof(float);
    }

    sci::Result<AttentionResult> Forward(const sci::Tensor& q, const sci::Tensor& k,
                                         const sci::Tensor& v,
                                         const AttentionConfig& cfg) const override {
        auto fail = [](AttnStatusCode code, std::string msg) {
            return sci::MakeUnexpected<AttentionResult>(MakeStatus(code, std::move(msg)));
        };
        const sci::Result<AttentionShape> inferred = InferShape(q, k, v, cfg.layout);
        if (!inferred.ok()) return sci::MakeUnexpected<AttentionResult>(inferred.error());
        const AttentionShape shape = *inferred;
        const sci::Status valid = Validate(cfg, shape);
        if (!valid.ok()) return sci::MakeUnexpected<AttentionResult>(valid);
        if (shape.seq_q != kNativeSeqQ) {
            return fail(AttnStatusCode::kUnsupportedFeature,
                        "decode backend requires seq_q=1; seq_q=" + std::to_string(shape.seq_q) +
                            " belongs to the flash backend");
        }
        if (shape.head_dim % 32 != 0) {
            return fail(AttnStatusCode::kUnsupportedHeadDim,
                        "decode requires head_dim % 32 == 0; head_dim=" +
                            std::to_string(shape.head_dim));
        }
        if (!DeviceCapability::GpuAvailable()) {
            return fail(AttnStatusCode::kUnsupportedFeature, "decode backend: no GPU device");
        }
        const int64_t splits = ResolveSplits(cfg.num_splits, shape.batch, shape.num_heads,
                                             shape.num_kv_heads, shape.seq_kv, shape.head_dim);

        AttentionResult result;
        result.out = sci::Tensor(sci::TensorShape({shape.batch, shape.num_heads, shape.seq_q,
                                                   shape.head_dim}),
                                 q.dtype(), q.device());
        if (result.out.data() == nullptr) {
            return fail(AttnStatusCode::kWorkspaceExceeded,
                        "allocation of the decode output failed");
        }
        const detail::Strides qs =
            detail::StridesFor(cfg.layout, shape.seq_q, shape.num_heads, shape.head_dim);
        const detail::Strides ks =
            detail::StridesFor(cfg.layout, shape.seq_kv, shape.num_kv_heads, shape.head_dim);
        const detail::Strides os =
            detail::StridesFor(AttnLayout::kBHSD, shape.seq_q, shape.num_heads, shape.head_dim);
        sca_decode_params p{};
        p.q = q.data();
        p.k = k.data();
        p.v = v.data();
        p.out = result.out.data();
        p.batch = shape.batch;
        p.num_heads = shape.num_heads;
        p.num_kv_heads = shape.num_kv_heads;
        p.seq_kv = shape.seq_kv;
        p.head_dim = shape.head_dim;
        p.num_splits = splits;
        p.q_sb = qs.s_b, p.q_sh = qs.s_h;
        p.k_sb = ks.s_b, p.k_sh = ks.s_h, p.k_ss = ks.s_s;
        p.v_sb = ks.s_b, p.v_sh = ks.s_h, p.v_ss = ks.s_s;
        p.o_sb = os.s_b, p.o_sh = os.s_h;
        p.scale = EffectiveScale(cfg, shape);
        p.dtype = runtime::KernelDtype(q.dtype());
        size_t partial_bytes = 0;
        sci::Status status = BindPartials(&p, splits, q.device().id(), &partial_bytes);
        if (status.ok()) {
            status = runtime::StatusFromHip(
                sca_hip_decode_splitk(&p, runtime::StreamHandle(cfg.stream)), "decode forward");
        }
        if (!status.ok()) return sci::MakeUnexpected<AttentionResult>(status);
        result.stats.used_backend = BackendKind::kDecode;
        result.stats.workspace_bytes = partial_bytes;
        result.stats.num_splits = splits;
        result.stats.note = "split-K decode: " + std::to_string(splits) +
                            " splits, FP32 partials in workspace; layout=" +
                            std::string(LayoutName(cfg.layout));
        return sci::Ok(std::move(result));
    }

    sci::Result<AttentionResult> ForwardVarlen(const sci::Tensor&, const sci::Tensor&,
                                               const sci::Tensor&, int64_t, const int32_t*,
                                               const int32_t*, int64_t, int64_t,
                                               const AttentionConfig&) const override {
        return sci::MakeUnexpected<AttentionResult>(MakeStatus(
            AttnStatusCode::kUnsupportedFeature,
            "decode backend does not implement varlen; use flash_attention_varlen"));
    }
};

// Paged decode is reached through paged_attention(q, kv, ...); the registry entry answers
// capability questions for the dispatcher.
class PagedBackend final : public IAttentionBackend {
public:
    BackendKind Kind() const noexcept override { return BackendKind::kPaged; }
    const char* Name() const noexcept override { return "paged"; }

    CapabilityReport Supports(const AttentionConfig&, const AttentionShape& shape) const override {
        CapabilityReport report;
        report.recommended_backend = BackendKind::kDecode;
        report.workspace_bytes = 0;
        std::string reason;
        if (!DeviceCapability::GpuAvailable()) {
            reason = "no GPU device available";
        } else if (shape.seq_q != kNativeSeqQ) {
            reason = "paged attention implements the decode form only (seq_q=1)";
        } else if (shape.head_dim % 32 != 0) {
            reason = "paged attention requires head_dim % 32 == 0";
        }
        report.supported = reason.empty();
        report.reason = report.supported
                            ? "paged decode over non-contiguous pages (page-table addressing)"
                            : reason;
        return report;
    }

    // An estimate from the shape alone (one wave per slot over seq_kv keys); a run under the
    // cache's length-aware plan binds, and reports in stats.workspace_bytes, what it uses.
    size_t WorkspaceBytes(const AttentionConfig& cfg, const AttentionShape& shape) const override {
        const int64_t splits = ResolveSplits(cfg.num_splits, shape.batch, shape.num_heads,
                                             shape.num_kv_heads, shape.seq_kv, shape.head_dim,
                                             /*slot_waves=*/1);
        if (splits <= 1) return 0;
        return static_cast<size_t>(
                   PartialElements(shape.batch, shape.num_heads, splits, shape.head_dim)) *
               sizeof(float);
    }

    sci::Result<AttentionResult> Forward(const sci::Tensor&, const sci::Tensor&, const sci::Tensor&,
                                         const AttentionConfig&) const override {
        return sci::MakeUnexpected<AttentionResult>(MakeStatus(
            AttnStatusCode::kUnsupportedFeature,
            "paged attention needs the KV cache: call sca::paged_attention(q, kv, params, cfg)"));
    }

    sci::Result<AttentionResult> ForwardVarlen(const sci::Tensor&, const sci::Tensor&,
                                               const sci::Tensor&, int64_t, const int32_t*,
                                               const int32_t*, int64_t, int64_t,
                                               const AttentionConfig&) const override {
        return sci::MakeUnexpected<AttentionResult>(MakeStatus(
            AttnStatusCode::kUnsupportedFeature,
            "paged backend does not implement varlen; use flash_attention_varlen"));
    }
};

const DecodeBackend kDecodeBackend;
const PagedBackend kPagedBackend;

sci::Result<AttentionResult> RunPaged(const sci::Tensor& q, const PagedKVCache& kv,
                                      const PagedAttentionParams& params,
                                      const AttentionConfig& cfg) {
    auto fail = [](AttnStatusCode code, std::string msg) {
        return sci::MakeUnexpected<AttentionResult>(MakeStatus(code, std::move(msg)));
    };
    if (q.ndims() != 4) {
        return fail(AttnStatusCode::kShapeMismatch,
                    "paged_attention expects q=[num_seqs, H_q, seq_q, D]; got ndims=" +
                        std::to_string(q.ndims()));
    }
    const int64_t num_seqs = q.dim(0);
    const int64_t num_heads = q.dim(1);
    const int64_t seq_q = q.dim(2);
    const int64_t head_dim = q.dim(3);
    if (seq_q != kNativeSeqQ) {
        return fail(AttnStatusCode::kUnsupportedFeature,
                    "paged attention implements the decode form only (seq_q=1); got seq_q=" +
                        std::to_string(seq_q));
    }
    if (num_seqs <= 0 || num_seqs > kv.MaxNumSeqs()) {
        return fail(AttnStatusCode::kShapeMismatch,
                    "paged_attention num_seqs=" + std::to_string(num_seqs) +
                        " exceeds the cache's max_num_seqs=" + std::to_string(kv.MaxNumSeqs()));
    }
    const KVCacheConfig& kv_cfg = kv.Storage().Config();
    if (params.layer < 0 || params.layer >= kv_cfg.num_layers) {
        return fail(AttnStatusCode::kShapeMismatch,
                    "paged_attention layer=" + std::to_string(params.layer) + " out of range [0," +
                        std::to_string(kv_cfg.num_layers) + ")");
    }
    if (!IsSupportedComputeDtype(q.dtype())) {
        return fail(AttnStatusCode::kUnsupportedDtype,
                    std::string("dtype=") + sci::kDTypeName(q.dtype()) + " is not a compute dtype");
    }
    if (q.dtype() != kv_cfg.dtype) {
        return fail(AttnStatusCode::kUnsupportedDtype,
                    std::string("paged_attention dtype mismatch: q=") + sci::kDTypeName(q.dtype()) +
                        ", cache=" + sci::kDTypeName(kv_cfg.dtype));
    }
    if (head_dim % 32 != 0 || SupportedHeadDimIndex(head_dim) < 0) {
        return fail(AttnStatusCode::kUnsupportedHeadDim,
                    "paged attention requires head_dim % 32 == 0 within {32..256}; got " +
                        std::to_string(head_dim));
    }
    if (head_dim != kv_cfg.head_dim) {
        return fail(AttnStatusCode::kShapeMismatch,
                    "paged_attention head_dim=" + std::to_string(head_dim) +
                        " differs from the cache's head_dim=" + std::to_string(kv_cfg.head_dim));
    }
    if (num_heads < kv_cfg.num_kv_heads || num_heads % kv_cfg.num_kv_heads != 0) {
        return fail(AttnStatusCode::kShapeMismatch,
                    "paged_attention num_heads=" + std::to_string(num_heads) +
                        " is not a multiple of the cache's num_kv_heads=" +
                        std::to_string(kv_cfg.num_kv_heads));
    }
    if (q.device_type() != sci::DeviceType::kGPU) {
        return fail(AttnStatusCode::kUnsupportedFeature, "paged_attention requires a GPU query");
    }
    const int32_t* page_table =
        params.page_table != nullptr ? params.page_table : kv.PageTableDevicePtr();
    if (page_table == nullptr) {
        return fail(AttnStatusCode::kShapeMismatch,
                    "paged_attention has no page table (call PagedKVCache::SyncPageTable first)");
    }
    const int64_t block_size = params.block_size > 0 ? params.block_size : kv.BlockSize();
    const int64_t max_blocks =
        params.max_blocks_per_seq > 0 ? params.max_blocks_per_seq : kv.MaxBlocksPerSeq();
    // Upper bound of a sequence's length; the kernel reads the true lengths from seq_lens.
    const int64_t seq_kv_bound = kv_cfg.num_blocks * block_size;
    int64_t splits =
        ResolveSplits(cfg.num_splits, num_seqs, num_heads, kv_cfg.num_kv_heads, seq_kv_bound,
                      head_dim, /*slot_waves=*/1);
    int32_t slot_waves = 0;
    // With the cache's own page table, its host-side lengths say how ragged the batch is; the
    // MFMA kernel (fp16/bf16, head_dim 64 or 128, power-of-two pages) then takes the split count
    // and slot work split of the length-aware plan. Lengths the caller passes in
    // params.seq_lens (device memory) do not feed the plan: the kernel reads them, so results
    // follow them exactly, while the plan is fitted to the cache's host lengths (which a decode
    // loop passing its own lengths, with this step's token, tracks to within a token).
    const bool mfma_shape = kv_cfg.dtype != sci::DType::kFloat32 &&
                            (head_dim == 64 || head_dim == 128) &&
                            (block_size & (block_size - 1)) == 0;
    if (cfg.num_splits <= 0 && params.page_table == nullptr && mfma_shape) {
        std::vector<int64_t> lengths(static_cast<size_t>(num_seqs));
        for (int64_t b = 0; b < num_seqs; ++b) lengths[static_cast<size_t>(b)] = kv.SeqLength(b);
        const auto plan = detail::PagedDecodePlan(lengths.data(), num_seqs, num_heads,
                                                  kv_cfg.num_kv_heads,
                                                  DeviceCapability::ForDevice(0).sm_count);
        if (plan.slot_waves != 0) {
            splits = plan.splits;
            slot_waves = plan.slot_waves;
        }
    }

    AttentionResult result;
    result.out = sci::Tensor(sci::TensorShape({num_seqs, num_heads, seq_q, head_dim}), q.dtype(),
                             q.device());
    if (result.out.data() == nullptr) {
        return fail(AttnStatusCode::kWorkspaceExceeded, "allocation of the paged output failed");
    }
    AttentionShape shape;
    shape.head_dim = head_dim;
    sca_decode_params p{};
    p.q = q.data();
    p.k = kv.Storage().K(params.layer).data();
    p.v = kv.Storage().V(params.layer).data();
    p.out = result.out.data();
    p.batch = num_seqs;
    p.num_heads = num_heads;
    p.num_kv_heads = kv_cfg.num_kv_heads;
    p.seq_kv = seq_kv_bound;
    p.head_dim = head_dim;
    p.num_splits = splits;
    p.q_sb = num_heads * head_dim, p.q_sh = head_dim;
    p.k_sb = 0, p.k_sh = head_dim, p.k_ss = kv_cfg.num_kv_heads * head_dim;
    p.v_sb = 0, p.v_sh = head_dim, p.v_ss = kv_cfg.num_kv_heads * head_dim;
    p.o_sb = num_heads * head_dim, p.o_sh = head_dim;
    p.scale = EffectiveScale(cfg, shape);
    p.dtype = runtime::KernelDtype(q.dtype());
    p.page_table = page_table;
    p.block_size = block_size;
    p.max_blocks_per_seq = max_blocks;
    p.num_kv_blocks = kv_cfg.num_blocks;
    p.seq_lens = params.seq_lens;
    p.slot_waves = slot_waves;
    size_t partial_bytes = 0;
    sci::Status status = BindPartials(&p, splits, q.device().id(), &partial_bytes);
    if (status.ok()) {
        status = runtime::StatusFromHip(
            sca_hip_decode_splitk_paged(&p, runtime::StreamHandle(cfg.stream)), "paged decode");
    }
    if (!status.ok()) return sci::MakeUnexpected<AttentionResult>(status);
    result.stats.used_backend = BackendKind::kPaged;
    result.stats.workspace_bytes = partial_bytes;
    result.stats.num_splits = splits;
    result.stats.kv_bytes = kv.Storage().MemoryBytes();
    result.stats.note = "paged decode: " + std::to_string(splits) + " splits, " +
                        (slot_waves == 4 ? "four waves" : "one wave") + " per head slot, block_size=" +
                        std::to_string(block_size) + ", layer=" + std::to_string(params.layer);
    return sci::Ok(std::move(result));
}

}  // namespace

namespace runtime {
const IAttentionBackend* DecodeBackendInstance() noexcept { return &kDecodeBackend; }
const IAttentionBackend* PagedBackendInstance() noexcept { return &kPagedBackend; }
}  // namespace runtime

DecodeConfig RecommendDecodeConfig(const AttentionShape& shape, const DeviceCapability& cap) {
    DecodeConfig cfg;
    cfg.max_splits = detail::kDispatchThresholds.max_splits;
    cfg.num_splits = detail::DecodeSplits(shape.batch, shape.num_heads, shape.num_kv_heads,
                                          shape.seq_kv, cap.sm_count, 4, shape.head_dim);
    return cfg;
}

sci::Result<AttentionResult> decode_attention(const sci::Tensor& q, const sci::Tensor& k,
                                              const sci::Tensor& v, const AttentionConfig& cfg) {
    return kDecodeBackend.Forward(q, k, v, cfg);
}

sci::Result<AttentionResult> decode_attention(const sci::Tensor& q, const sci::Tensor& k,
                                              const sci::Tensor& v, const AttentionConfig& cfg,
                                              const DecodeConfig& decode_cfg) {
    AttentionConfig resolved = cfg;
    if (!decode_cfg.use_splitk) {
        resolved.num_splits = 1;
    } else {
        int64_t splits = decode_cfg.num_splits;
        if (splits > 0 && decode_cfg.max_splits > 0 && splits > decode_cfg.max_splits) {
            splits = decode_cfg.max_splits;
        }
        resolved.num_splits = splits;
    }
    return kDecodeBackend.Forward(q, k, v, resolved);
}

sci::Result<AttentionResult> paged_attention(const sci::Tensor& q, const PagedKVCache& kv,
                                             const PagedAttentionParams& params,
                                             const AttentionConfig& cfg) {
    return RunPaged(q, kv, params, cfg);
}

sci::Result<AttentionResult> paged_attention(const sci::Tensor& q, const PagedKVCache& kv,
                                             const AttentionConfig& cfg) {
    PagedAttentionParams params;
    params.page_table = kv.PageTableDevicePtr();
    params.num_seqs = kv.MaxNumSeqs();
    params.block_size = kv.BlockSize();
    params.max_blocks_per_seq = kv.MaxBlocksPerSeq();
    params.layer = 0;
    return RunPaged(q, kv, params, cfg);
}

}  // namespace sca

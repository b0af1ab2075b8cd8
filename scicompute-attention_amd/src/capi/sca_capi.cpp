// C ABI over the sca:: C++ API (declared in include/sca_capi.h). Thin forwarding only: every
// decision is made by the C++ layer; this file converts PODs, owns nothing beyond the handles it
// returns, and records the last failure per thread.

#include "sca_capi.h"

#include <cstring>
#include <string>
#include <vector>

#include "device/device.hpp"
#include "runtime/dispatch_table.hpp"
#include "runtime/internal.hpp"
#include "scicompute_attention/attention.hpp"

namespace {

thread_local std::string g_last_error;

int Fail(const sci::Status& st) {
    g_last_error = st.message();
    const int code = static_cast<int>(sca::ExtractCode(st));
    return code != 0 ? code : 1;
}

int Check(const sci::Status& st) {
    if (st.ok()) return 0;
    return Fail(st);
}

void CopyText(const std::string& text, char* out, size_t len) {
    if (out == nullptr || len == 0) return;
    const size_t n = text.size() < len - 1 ? text.size() : len - 1;
    std::memcpy(out, text.data(), n);
    out[n] = '\0';
}

sci::Device& DeviceOf(int32_t kind) {
    return kind == 1 ? sci::GpuDevice(0) : sci::HostDevice();
}

// Streams passed in a config are wrapped per call (non-owning).
struct CfgHolder {
    sca::AttentionConfig cfg;
    sci::Stream stream;
};

void ToCfg(const ScaConfig* c, CfgHolder* h) {
    sca::AttentionConfig& cfg = h->cfg;
    if (c == nullptr) return;
    cfg.backend = static_cast<sca::BackendKind>(c->backend);
    cfg.layout = static_cast<sca::AttnLayout>(c->layout);
    cfg.causal = c->causal != 0;
    cfg.return_lse = c->return_lse != 0;
    cfg.scale = c->scale;
    cfg.softcap = c->softcap;
    cfg.sliding_window = c->sliding_window;
    cfg.num_splits = c->num_splits;
    cfg.allow_fallback = c->allow_fallback != 0;
    cfg.cu_seqlens_q = c->cu_seqlens_q;
    cfg.cu_seqlens_kv = c->cu_seqlens_kv;
    if (c->stream != nullptr) {
        h->stream = sci::Stream(c->stream);
        cfg.stream = &h->stream;
    }
}

sca::AttentionShape ToShape(const ScaShape* s) {
    sca::AttentionShape shape;
    if (s == nullptr) return shape;
    shape.batch = s->batch;
    shape.seq_q = s->seq_q;
    shape.seq_kv = s->seq_kv;
    shape.num_heads = s->num_heads;
    shape.num_kv_heads = s->num_kv_heads;
    shape.head_dim = s->head_dim;
    return shape;
}

sca::KVCacheConfig ToKvCfg(const ScaKvConfig* c) {
    sca::KVCacheConfig cfg;
    cfg.num_layers = c->num_layers;
    cfg.num_kv_heads = c->num_kv_heads;
    cfg.head_dim = c->head_dim;
    cfg.block_size = c->block_size;
    cfg.num_blocks = c->num_blocks;
    cfg.max_num_seqs = c->max_num_seqs;
    cfg.dtype = static_cast<sci::DType>(c->dtype);
    cfg.layout = static_cast<sca::KvLayout>(c->layout);
    return cfg;
}

void ToStats(const sca::AttentionRuntimeStats& s, ScaStats* out) {
    if (out == nullptr) return;
    out->used_backend = static_cast<int32_t>(s.used_backend);
    out->tile[0] = s.tile.block_m;
    out->tile[1] = s.tile.block_n;
    out->tile[2] = s.tile.warps;
    out->tile[3] = s.tile.stages;
    out->workspace_bytes = s.workspace_bytes;
    out->kv_bytes = s.kv_bytes;
    out->num_splits = s.num_splits;
    out->materialized_score_bytes = s.materialized_score_bytes;
    CopyText(s.note, out->note, sizeof(out->note));
}

sci::Stream* StreamArg(void* handle, sci::Stream* holder) {
    if (handle == nullptr) return nullptr;
    *holder = sci::Stream(handle);
    return holder;
}

const sci::Tensor& T(const ScaTensor* t) { return *reinterpret_cast<const sci::Tensor*>(t); }
ScaTensor* Wrap(sci::Tensor&& t) {
    return reinterpret_cast<ScaTensor*>(new sci::Tensor(std::move(t)));
}
sca::PagedKVCache& P(ScaPagedKV* c) { return *reinterpret_cast<sca::PagedKVCache*>(c); }
const sca::PagedKVCache& P(const ScaPagedKV* c) {
    return *reinterpret_cast<const sca::PagedKVCache*>(c);
}
sca::BlockManager& B(ScaBlockManager* b) { return *reinterpret_cast<sca::BlockManager*>(b); }
const sca::BlockManager& B(const ScaBlockManager* b) {
    return *reinterpret_cast<const sca::BlockManager*>(b);
}
sca::Workspace& W(ScaWorkspace* w) { return *reinterpret_cast<sca::Workspace*>(w); }
const sca::Workspace& W(const ScaWorkspace* w) { return *reinterpret_cast<const sca::Workspace*>(w); }

sci::TensorShape ShapeOf(const int64_t* dims, int32_t ndims) {
    std::vector<sci::index_t> d(dims, dims + (ndims > 0 ? ndims : 0));
    return sci::TensorShape(d);
}

int Finish(sci::Result<sca::AttentionResult>&& r, bool want_lse, ScaTensor** out, ScaTensor** lse,
           ScaStats* stats) {
    if (!r.ok()) return Fail(r.error());
    ToStats(r->stats, stats);
    if (out != nullptr) *out = Wrap(std::move(r->out));
    if (lse != nullptr) *lse = want_lse ? Wrap(std::move(r->lse)) : nullptr;
    return 0;
}

}  // namespace

extern "C" {

const char* sca_last_error(void) { return g_last_error.c_str(); }

const char* sca_version(void) { return sca::VersionString(); }
const char* sca_build_flavor(void) { return sca::BuildFlavor(); }
const char* sca_status_name(int code) { return sca::ToString(static_cast<sca::AttnStatusCode>(code)); }
int sca_to_sci_code(int code) {
    return static_cast<int>(sca::ToSciCode(static_cast<sca::AttnStatusCode>(code)));
}
int sca_make_status(int code, const char* detail, char* msg, size_t len) {
    const sci::Status st =
        sca::MakeStatus(static_cast<sca::AttnStatusCode>(code), detail != nullptr ? detail : "");
    CopyText(st.message(), msg, len);
    return static_cast<int>(st.code());
}
int sca_extract_code(const char* message) {
    return static_cast<int>(
        sca::ExtractCode(sci::Status(sci::StatusCode::kError, message != nullptr ? message : "")));
}
const char* sca_backend_name(int kind) { return sca::BackendName(static_cast<sca::BackendKind>(kind)); }
const char* sca_layout_name(int layout) { return sca::LayoutName(static_cast<sca::AttnLayout>(layout)); }
int sca_parse_backend(const char* name, int32_t* kind) {
    sca::BackendKind k = sca::BackendKind::kAuto;
    if (!sca::ParseBackendName(name, &k)) return 0;
    if (kind != nullptr) *kind = static_cast<int32_t>(k);
    return 1;
}
int sca_supported_head_dim_index(int64_t head_dim) { return sca::SupportedHeadDimIndex(head_dim); }
int64_t sca_tile_smem_bytes_flash(int32_t head_dim, int64_t elem_bytes, int32_t block_m,
                                  int32_t block_n, int32_t warps, int32_t stages) {
    return sca::TileConfig::SmemBytesFlash(head_dim, elem_bytes, block_m, block_n, warps, stages);
}
int64_t sca_flash_lds_bytes(int64_t head_dim, int64_t elem_bytes) {
    return sca::FlashLdsBytes(head_dim, elem_bytes);
}

int sca_validate(const ScaConfig* cfg, const ScaShape* shape, char* detail, size_t len) {
    CfgHolder h;
    ToCfg(cfg, &h);
    std::string text;
    const sci::Status st = sca::Validate(h.cfg, ToShape(shape), &text);
    CopyText(text, detail, len);
    return Check(st);
}
float sca_effective_scale(const ScaConfig* cfg, const ScaShape* shape) {
    CfgHolder h;
    ToCfg(cfg, &h);
    return sca::EffectiveScale(h.cfg, ToShape(shape));
}
int sca_validate_varlen(const int32_t* cu, int64_t batch, int64_t* max_seq) {
    return Check(sca::ValidateVarlenHost(cu, batch, max_seq));
}
int sca_select(const ScaConfig* cfg, const ScaShape* shape, int32_t* backend, int32_t* tile4,
               uint64_t* workspace_bytes, char* reason, size_t len) {
    CfgHolder h;
    ToCfg(cfg, &h);
    const sca::DispatchDecision d = sca::AttentionDispatcher().Select(h.cfg, ToShape(shape));
    if (backend != nullptr) *backend = static_cast<int32_t>(d.backend);
    if (tile4 != nullptr) {
        tile4[0] = d.tile.block_m;
        tile4[1] = d.tile.block_n;
        tile4[2] = d.tile.warps;
        tile4[3] = d.tile.stages;
    }
    if (workspace_bytes != nullptr) *workspace_bytes = d.workspace_bytes;
    CopyText(d.reason, reason, len);
    return 0;
}
void sca_explain(const ScaConfig* cfg, const ScaShape* shape, char* out, size_t len) {
    CfgHolder h;
    ToCfg(cfg, &h);
    CopyText(sca::AttentionDispatcher().Explain(h.cfg, ToShape(shape)), out, len);
}
void sca_recommend_tile(const ScaConfig* cfg, const ScaShape* shape, int32_t* tile4) {
    CfgHolder h;
    ToCfg(cfg, &h);
    const sca::TileConfig t = sca::RecommendTile(h.cfg, ToShape(shape));
    tile4[0] = t.block_m;
    tile4[1] = t.block_n;
    tile4[2] = t.warps;
    tile4[3] = t.stages;
}
int64_t sca_decode_splits(const ScaShape* s, int64_t cu_count) {
    return sca::detail::DecodeSplits(s->batch, s->num_heads, s->num_kv_heads, s->seq_kv, cu_count,
                                     4, s->head_dim);
}
int sca_paged_decode_plan(const int64_t* lengths, int64_t batch, int64_t num_heads,
                          int64_t num_kv_heads, int64_t cu_count, int64_t* splits,
                          int32_t* slot_waves) {
    if (lengths == nullptr || splits == nullptr || slot_waves == nullptr || batch < 1 ||
        num_kv_heads < 1 || num_heads < num_kv_heads || num_heads % num_kv_heads != 0) {
        return Fail(sca::MakeStatus(sca::AttnStatusCode::kShapeMismatch,
                                    "sca_paged_decode_plan: null pointer or invalid heads/batch"));
    }
    const auto plan =
        sca::detail::PagedDecodePlan(lengths, batch, num_heads, num_kv_heads, cu_count);
    *splits = plan.splits;
    *slot_waves = plan.slot_waves;
    return 0;
}

int sca_compute_slot_mapping(const int32_t* row, int64_t seq_start, int64_t num_tokens,
                             int64_t block_size, int64_t max_blocks, int32_t* slots) {
    const auto r = sca::ComputeSlotMapping(row, seq_start, num_tokens, block_size, max_blocks);
    if (!r.ok()) return Fail(r.error());
    if (slots != nullptr) std::memcpy(slots, r->data(), r->size() * sizeof(int32_t));
    return 0;
}
int sca_kv_cache_bytes(const ScaKvConfig* cfg, uint64_t* bytes) {
    const auto r = sca::KvCacheBytes(ToKvCfg(cfg));
    if (!r.ok()) return Fail(r.error());
    if (bytes != nullptr) *bytes = *r;
    return 0;
}
int64_t sca_max_blocks_for_budget(const ScaKvConfig* cfg, uint64_t budget_bytes) {
    return sca::MaxBlocksForBudget(ToKvCfg(cfg), budget_bytes);
}

// ---- tensors ----
ScaTensor* sca_tensor_new(const int64_t* dims, int32_t ndims, int32_t dtype, int32_t device_kind) {
    sci::Tensor t(ShapeOf(dims, ndims), static_cast<sci::DType>(dtype), DeviceOf(device_kind));
    if (t.data() == nullptr && t.num_bytes() > 0) {
        g_last_error = "tensor allocation failed";
        return nullptr;
    }
    return Wrap(std::move(t));
}
ScaTensor* sca_tensor_wrap(void* data, const int64_t* dims, int32_t ndims, int32_t dtype,
                           int32_t device_kind) {
    return Wrap(sci::Tensor(ShapeOf(dims, ndims), static_cast<sci::DType>(dtype),
                            DeviceOf(device_kind), data, false));
}
void sca_tensor_free(ScaTensor* t) { delete reinterpret_cast<sci::Tensor*>(t); }
void* sca_tensor_data(ScaTensor* t) { return reinterpret_cast<sci::Tensor*>(t)->data(); }
uint64_t sca_tensor_nbytes(const ScaTensor* t) { return T(t).num_bytes(); }
int32_t sca_tensor_ndims(const ScaTensor* t) { return static_cast<int32_t>(T(t).ndims()); }
int64_t sca_tensor_dim(const ScaTensor* t, int32_t i) { return T(t).dim(static_cast<size_t>(i)); }
int sca_tensor_upload(ScaTensor* t, const void* host, uint64_t bytes) {
    reinterpret_cast<sci::Tensor*>(t)->copy_from(host, bytes);
    return 0;
}
int sca_tensor_download(const ScaTensor* t, void* host, uint64_t bytes) {
    T(t).copy_to_host(host, bytes);
    return 0;
}

// ---- attention ----
int sca_run_attention(int32_t entry, const ScaTensor* q, const ScaTensor* k, const ScaTensor* v,
                      const ScaConfig* cfg, ScaTensor** out, ScaTensor** lse, ScaStats* stats) {
    CfgHolder h;
    ToCfg(cfg, &h);
    const sci::Tensor& tq = T(q);
    const sci::Tensor& tk = T(k);
    const sci::Tensor& tv = T(v);
    switch (entry) {
        case 0: return Finish(sca::attention(tq, tk, tv, h.cfg), h.cfg.return_lse, out, lse, stats);
        case 1:
            return Finish(sca::flash_attention(tq, tk, tv, h.cfg), h.cfg.return_lse, out, lse, stats);
        case 2:
            return Finish(sca::decode_attention(tq, tk, tv, h.cfg), false, out, lse, stats);
        case 3: return Finish(sca::decode(tq, tk, tv, h.cfg), false, out, lse, stats);
        case 4: return Finish(sca::naive_attention(tq, tk, tv, h.cfg), false, out, lse, stats);
        case 5: return Finish(sca::tiled_attention(tq, tk, tv, h.cfg), false, out, lse, stats);
        default: break;
    }
    return Fail(sca::MakeStatus(sca::AttnStatusCode::kUnsupportedFeature,
                                "sca_run_attention: unknown entry " + std::to_string(entry)));
}
int sca_run_flash_varlen(const ScaTensor* q, const ScaTensor* k, const ScaTensor* v,
                         int64_t num_seqs, const int32_t* cu_q, const int32_t* cu_kv,
                         int64_t max_seq_q, int64_t max_seq_kv, const ScaConfig* cfg,
                         ScaTensor** out, ScaStats* stats) {
    CfgHolder h;
    ToCfg(cfg, &h);
    return Finish(sca::flash_attention_varlen(T(q), T(k), T(v), num_seqs, cu_q, cu_kv, max_seq_q,
                                              max_seq_kv, h.cfg),
                  false, out, nullptr, stats);
}
void sca_explain_tensors(const ScaTensor* q, const ScaTensor* k, const ScaTensor* v,
                         const ScaConfig* cfg, char* out, size_t len) {
    CfgHolder h;
    ToCfg(cfg, &h);
    CopyText(sca::ExplainAttention(T(q), T(k), T(v), h.cfg), out, len);
}

// ---- paged KV cache ----
ScaPagedKV* sca_pkv_create(const ScaKvConfig* cfg, int32_t device_kind) {
    auto r = sca::PagedKVCache::Create(ToKvCfg(cfg), DeviceOf(device_kind));
    if (!r.ok()) {
        Fail(r.error());
        return nullptr;
    }
    return reinterpret_cast<ScaPagedKV*>(new sca::PagedKVCache(std::move(*r)));
}
void sca_pkv_destroy(ScaPagedKV* c) { delete reinterpret_cast<sca::PagedKVCache*>(c); }
int sca_pkv_append(ScaPagedKV* c, int64_t seq_id, int64_t layer, const ScaTensor* k_new,
                   const ScaTensor* v_new, void* stream) {
    sci::Stream holder;
    return Check(P(c).AppendTokens(seq_id, layer, T(k_new), T(v_new), StreamArg(stream, &holder)));
}
int sca_pkv_append_batch(ScaPagedKV* c, const int64_t* seq_ids, int64_t num_entries,
                         int64_t layer, const ScaTensor* k_new, const ScaTensor* v_new,
                         void* stream) {
    sci::Stream holder;
    return Check(P(c).AppendTokensBatch(seq_ids, num_entries, layer, T(k_new), T(v_new),
                                        StreamArg(stream, &holder)));
}
int sca_pkv_reserve(ScaPagedKV* c, int64_t seq_id, int64_t num_tokens, void* stream) {
    sci::Stream holder;
    return Check(P(c).ReserveTokens(seq_id, num_tokens, StreamArg(stream, &holder)));
}
int sca_pkv_reserve_batch(ScaPagedKV* c, const int64_t* seq_ids, int64_t num_entries,
                          void* stream) {
    sci::Stream holder;
    return Check(P(c).ReserveTokensBatch(seq_ids, num_entries, StreamArg(stream, &holder)));
}
int sca_pkv_write_layer(ScaPagedKV* c, int64_t layer, const ScaTensor* k_new,
                        const ScaTensor* v_new, void* stream) {
    sci::Stream holder;
    return Check(P(c).WriteReservedLayer(layer, T(k_new), T(v_new), StreamArg(stream, &holder)));
}
int sca_pkv_append_batch_all_layers(ScaPagedKV* c, const int64_t* seq_ids, int64_t num_entries,
                                    const ScaTensor* k_layers, const ScaTensor* v_layers,
                                    void* stream) {
    sci::Stream holder;
    return Check(P(c).AppendTokensBatchAllLayers(seq_ids, num_entries, T(k_layers), T(v_layers),
                                                 StreamArg(stream, &holder)));
}
int sca_pkv_reset(ScaPagedKV* c, int64_t seq_id, void* stream) {
    sci::Stream holder;
    return Check(P(c).ResetSeq(seq_id, StreamArg(stream, &holder)));
}
int sca_pkv_sync(ScaPagedKV* c, void* stream) {
    sci::Stream holder;
    return Check(P(c).SyncPageTable(StreamArg(stream, &holder)));
}
int sca_pkv_force_sync(ScaPagedKV* c, void* stream) {
    sci::Stream holder;
    return Check(P(c).ForceSyncPageTable(StreamArg(stream, &holder)));
}
const int32_t* sca_pkv_page_table_device(const ScaPagedKV* c) { return P(c).PageTableDevicePtr(); }
void sca_pkv_page_table_host(const ScaPagedKV* c, int32_t* out) {
    const auto& t = P(c).PageTableHost();
    std::memcpy(out, t.data(), t.size() * sizeof(int32_t));
}
int64_t sca_pkv_seq_len(const ScaPagedKV* c, int64_t seq_id) { return P(c).SeqLength(seq_id); }
int64_t sca_pkv_block_count(const ScaPagedKV* c, int64_t seq_id) {
    return P(c).LogicalBlockCount(seq_id);
}
int64_t sca_pkv_max_blocks_per_seq(const ScaPagedKV* c) { return P(c).MaxBlocksPerSeq(); }
uint64_t sca_pkv_revision(const ScaPagedKV* c) { return P(c).Revision(); }
uint64_t sca_pkv_synced_revision(const ScaPagedKV* c) { return P(c).SyncedRevision(); }
void sca_pkv_stats(const ScaPagedKV* c, ScaKvStats* out) {
    const sca::KVCacheStats s = P(c).Stats();
    out->num_blocks = s.num_blocks;
    out->used_blocks = s.used_blocks;
    out->free_blocks = s.free_blocks;
    out->num_appends = s.num_appends;
    out->num_resets = s.num_resets;
    out->peak_bytes = s.peak_bytes;
    out->bytes = s.bytes;
}
void* sca_pkv_layer_k(const ScaPagedKV* c, int64_t layer) {
    return const_cast<void*>(P(c).Storage().K(layer).data());
}
void* sca_pkv_layer_v(const ScaPagedKV* c, int64_t layer) {
    return const_cast<void*>(P(c).Storage().V(layer).data());
}
const ScaBlockManager* sca_pkv_blocks(const ScaPagedKV* c) {
    return reinterpret_cast<const ScaBlockManager*>(&P(c).Blocks());
}
int sca_pkv_gather(const ScaPagedKV* c, int32_t is_key, int64_t layer, const int32_t* block_ids,
                   int64_t num_blocks, void* stream, ScaTensor** out) {
    sci::Stream holder;
    sci::Stream* s = StreamArg(stream, &holder);
    auto r = is_key ? P(c).Storage().GatherK(layer, block_ids, num_blocks, s)
                    : P(c).Storage().GatherV(layer, block_ids, num_blocks, s);
    if (!r.ok()) return Fail(r.error());
    *out = Wrap(std::move(*r));
    return 0;
}
int sca_run_paged(const ScaTensor* q, const ScaPagedKV* kv, const ScaPagedParams* params,
                  const ScaConfig* cfg, ScaTensor** out, ScaStats* stats) {
    CfgHolder h;
    ToCfg(cfg, &h);
    if (params == nullptr) {
        return Finish(sca::paged_attention(T(q), P(kv), h.cfg), false, out, nullptr, stats);
    }
    sca::PagedAttentionParams p;
    p.page_table = params->page_table;
    p.seq_lens = params->seq_lens;
    p.num_seqs = params->num_seqs;
    p.block_size = params->block_size;
    p.max_blocks_per_seq = params->max_blocks_per_seq;
    p.layer = params->layer;
    return Finish(sca::paged_attention(T(q), P(kv), p, h.cfg), false, out, nullptr, stats);
}

// ---- BlockManager ----
ScaBlockManager* sca_bm_create(int64_t num_blocks, int64_t max_num_seqs,
                               int64_t max_blocks_per_seq, int32_t device_kind) {
    auto r = sca::BlockManager::Create(num_blocks, max_num_seqs, max_blocks_per_seq,
                                       DeviceOf(device_kind));
    if (!r.ok()) {
        Fail(r.error());
        return nullptr;
    }
    return reinterpret_cast<ScaBlockManager*>(new sca::BlockManager(std::move(*r)));
}
void sca_bm_destroy(ScaBlockManager* bm) { delete reinterpret_cast<sca::BlockManager*>(bm); }
int sca_bm_allocate(ScaBlockManager* bm, int64_t count, int32_t* out) {
    auto r = B(bm).Allocate(count);
    if (!r.ok()) return Fail(r.error());
    if (out != nullptr) std::memcpy(out, r->data(), r->size() * sizeof(int32_t));
    return 0;
}
void sca_bm_free(ScaBlockManager* bm, const int32_t* ids, int64_t count) { B(bm).Free(ids, count); }
int sca_bm_append_to_table(ScaBlockManager* bm, int64_t seq_id, const int32_t* ids, int64_t count) {
    return Check(B(bm).AppendToTable(seq_id, ids, count));
}
int sca_bm_reset_seq(ScaBlockManager* bm, int64_t seq_id) { return Check(B(bm).ResetSeq(seq_id)); }
int sca_bm_sync(ScaBlockManager* bm, void* stream) {
    sci::Stream holder;
    return Check(B(bm).SyncTableToDevice(StreamArg(stream, &holder)));
}
int64_t sca_bm_num_free(const ScaBlockManager* bm) { return B(bm).NumFreeBlocks(); }
int64_t sca_bm_num_total(const ScaBlockManager* bm) { return B(bm).NumTotalBlocks(); }
int64_t sca_bm_failures(const ScaBlockManager* bm) { return B(bm).AllocationFailures(); }
int64_t sca_bm_double_frees(const ScaBlockManager* bm) { return B(bm).DoubleFreeEvents(); }
uint64_t sca_bm_revision(const ScaBlockManager* bm) { return B(bm).Table().revision; }
uint64_t sca_bm_synced_revision(const ScaBlockManager* bm) { return B(bm).Table().synced_revision; }
void sca_bm_table(const ScaBlockManager* bm, int32_t* out) {
    const auto& t = B(bm).Table().host;
    std::memcpy(out, t.data(), t.size() * sizeof(int32_t));
}
int sca_bm_table_device(const ScaBlockManager* bm, int32_t* out) {
    const sci::Tensor& t = B(bm).Table().device;
    if (t.data() == nullptr) return Fail(sci::Status(sci::StatusCode::kError, "no device table"));
    t.device().synchronize();
    t.copy_to_host(out, t.num_bytes());
    return 0;
}

// ---- Workspace ----
ScaWorkspace* sca_ws_create(uint64_t bytes, int32_t device_kind) {
    auto r = sca::Workspace::Create(bytes, DeviceOf(device_kind));
    if (!r.ok()) {
        Fail(r.error());
        return nullptr;
    }
    return reinterpret_cast<ScaWorkspace*>(new sca::Workspace(*r));
}
void sca_ws_destroy(ScaWorkspace* ws) { delete reinterpret_cast<sca::Workspace*>(ws); }
int sca_ws_slice(ScaWorkspace* ws, uint64_t offset, uint64_t bytes, uint64_t align,
                 uint64_t* relative_offset) {
    auto r = W(ws).Slice(offset, bytes, align);
    if (!r.ok()) return Fail(r.error());
    if (relative_offset != nullptr) {
        *relative_offset = static_cast<uint64_t>(static_cast<unsigned char*>(*r) -
                                                 static_cast<unsigned char*>(W(ws).Data()));
    }
    return 0;
}
int sca_ws_reset(ScaWorkspace* ws) { return Check(W(ws).Reset()); }
uint64_t sca_ws_peak(const ScaWorkspace* ws) { return W(ws).PeakBytes(); }
uint64_t sca_ws_slices(const ScaWorkspace* ws) { return W(ws).AllocatedSlices(); }

// ---- pool, scratch, capability ----
uint64_t sca_gpu_empty_cache(void) { return sci::GpuEmptyCache(0); }
uint64_t sca_gpu_cached_bytes(void) { return sci::GpuCachedBytes(0); }
uint64_t sca_gpu_allocated_bytes(void) { return sci::GpuAllocatedBytes(0); }
int sca_release_scratch(void) { return Check(sca::runtime::ReleaseScratch()); }
uint64_t sca_scratch_high_water_bytes(void) { return sca::runtime::ScratchHighWaterMarkBytes(); }
int sca_gpu_available(void) { return sca::DeviceCapability::GpuAvailable() ? 1 : 0; }
int sca_device_cu_count(void) { return sca::DeviceCapability::ForDevice(0).sm_count; }
int sca_synchronize(void) {
    return Check(sca::runtime::StatusFromHip(sca_hip_device_synchronize(), "synchronize"));
}

}  // extern "C"

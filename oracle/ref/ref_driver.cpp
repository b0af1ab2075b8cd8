// Trace driver over the reference's own host code, compiled in its CPU (STUB) mode.
// TEST INFRASTRUCTURE ONLY: it is built into oracle/_ref/libsca_ref.so from the sources under
// /root/reference and used to (1) generate the golden fixtures under tests/golden/ and (2) check
// the oracle restatement and this repository's host layer against the reference, when present.
//
// The driver only calls the reference's public host API; it replaces nothing of the reference.

#include <cstdint>
#include <cstring>
#include <string>
#include <vector>

#include "backends/decode/decode_config.hpp"
#include "device/device.hpp"
#include "scicompute_attention/attention_config.hpp"
#include "scicompute_attention/backends.hpp"
#include "scicompute_attention/block_manager.hpp"
#include "scicompute_attention/dispatcher.hpp"
#include "scicompute_attention/kv_cache.hpp"
#include "scicompute_attention/status.hpp"
#include "scicompute_attention/workspace.hpp"
#include "scicompute_attention/detail/tile_config.hpp"

namespace {

void CopyMsg(const std::string& text, char* out, size_t len) {
    if (out == nullptr || len == 0) return;
    std::strncpy(out, text.c_str(), len - 1);
    out[len - 1] = '\0';
}

int CodeOf(const sci::Status& s) { return s.ok() ? 0 : static_cast<int>(sca::ExtractCode(s)); }

}  // namespace

extern "C" {

struct RefCfg {
    int32_t backend;
    int32_t layout;
    int32_t causal;
    int32_t return_lse;
    float scale;
    float softcap;
    int64_t sliding_window;
    int64_t num_splits;
    int32_t allow_fallback;
    int32_t has_cu_seqlens_q;
    int32_t has_cu_seqlens_kv;
};

struct RefShape {
    int64_t batch, seq_q, seq_kv, num_heads, num_kv_heads, head_dim;
};

static sca::AttentionConfig ToCfg(const RefCfg* c) {
    static const int32_t dummy_cu[2] = {0, 1};
    sca::AttentionConfig cfg;
    cfg.backend = static_cast<sca::BackendKind>(c->backend);
    cfg.layout = static_cast<sca::AttnLayout>(c->layout);
    cfg.causal = c->causal != 0;
    cfg.return_lse = c->return_lse != 0;
    cfg.scale = c->scale;
    cfg.softcap = c->softcap;
    cfg.sliding_window = c->sliding_window;
    cfg.num_splits = c->num_splits;
    cfg.allow_fallback = c->allow_fallback != 0;
    cfg.cu_seqlens_q = c->has_cu_seqlens_q ? dummy_cu : nullptr;
    cfg.cu_seqlens_kv = c->has_cu_seqlens_kv ? dummy_cu : nullptr;
    return cfg;
}

static sca::AttentionShape ToShape(const RefShape* s) {
    sca::AttentionShape shape;
    shape.batch = s->batch;
    shape.seq_q = s->seq_q;
    shape.seq_kv = s->seq_kv;
    shape.num_heads = s->num_heads;
    shape.num_kv_heads = s->num_kv_heads;
    shape.head_dim = s->head_dim;
    return shape;
}

// ---- validation / scale / varlen ---------------------------------------------------------------
int ref_validate(const RefCfg* c, const RefShape* s, char* msg, size_t len) {
    std::string detail;
    const sci::Status st = sca::Validate(ToCfg(c), ToShape(s), &detail);
    CopyMsg(st.ok() ? detail : st.message(), msg, len);
    return CodeOf(st);
}

float ref_effective_scale(const RefCfg* c, const RefShape* s) {
    return sca::EffectiveScale(ToCfg(c), ToShape(s));
}

int ref_validate_varlen(const int32_t* cu, int64_t batch, int64_t* max_seq, char* msg,
                        size_t len) {
    const sci::Status st = sca::ValidateVarlenHost(cu, batch, max_seq);
    CopyMsg(st.message(), msg, len);
    return CodeOf(st);
}

// ---- dispatcher ----------------------------------------------------------------------------------
int ref_select(const RefCfg* c, const RefShape* s, int32_t* backend, int32_t* tile4,
               uint64_t* workspace, char* reason, size_t len) {
    const sca::AttentionDispatcher dispatcher;
    const sca::DispatchDecision d = dispatcher.Select(ToCfg(c), ToShape(s));
    *backend = static_cast<int32_t>(d.backend);
    tile4[0] = d.tile.block_m;
    tile4[1] = d.tile.block_n;
    tile4[2] = d.tile.warps;
    tile4[3] = d.tile.stages;
    *workspace = d.workspace_bytes;
    CopyMsg(d.reason, reason, len);
    return 0;
}

void ref_explain(const RefCfg* c, const RefShape* s, char* out, size_t len) {
    const sca::AttentionDispatcher dispatcher;
    CopyMsg(dispatcher.Explain(ToCfg(c), ToShape(s)), out, len);
}

// ---- status / names ------------------------------------------------------------------------------
int ref_make_status(int code, const char* detail, char* msg, size_t len) {
    const sci::Status st = sca::MakeStatus(static_cast<sca::AttnStatusCode>(code), detail);
    CopyMsg(st.message(), msg, len);
    return static_cast<int>(st.code());
}

const char* ref_status_name(int code) { return sca::ToString(static_cast<sca::AttnStatusCode>(code)); }
int ref_to_sci_code(int code) {
    return static_cast<int>(sca::ToSciCode(static_cast<sca::AttnStatusCode>(code)));
}
int ref_extract_code(const char* msg) {
    return static_cast<int>(sca::ExtractCode(sci::Status(sci::StatusCode::kError, msg)));
}
const char* ref_backend_name(int kind) { return sca::BackendName(static_cast<sca::BackendKind>(kind)); }
const char* ref_layout_name(int layout) { return sca::LayoutName(static_cast<sca::AttnLayout>(layout)); }
int ref_parse_backend(const char* name, int32_t* out) {
    sca::BackendKind kind = sca::BackendKind::kAuto;
    const bool ok = sca::ParseBackendName(name, &kind);
    if (ok) *out = static_cast<int32_t>(kind);
    return ok ? 1 : 0;
}
int ref_supported_head_dim_index(int64_t d) { return sca::SupportedHeadDimIndex(d); }
int64_t ref_tile_smem_bytes_flash(int32_t d, int64_t eb, int32_t bm, int32_t bn, int32_t w,
                                  int32_t st) {
    return sca::TileConfig::SmemBytesFlash(d, eb, bm, bn, w, st);
}

// ---- KV helpers ----------------------------------------------------------------------------------
int ref_compute_slot_mapping(const int32_t* row, int64_t start, int64_t n, int64_t bs,
                             int64_t max_blocks, int32_t* slots, char* msg, size_t len) {
    const auto r = sca::ComputeSlotMapping(row, start, n, bs, max_blocks);
    if (!r.ok()) {
        CopyMsg(r.error().message(), msg, len);
        return CodeOf(r.error());
    }
    std::memcpy(slots, r->data(), sizeof(int32_t) * r->size());
    return 0;
}

int64_t ref_kv_cache_bytes(int64_t layers, int64_t heads, int64_t d, int64_t bs, int64_t nb,
                           int64_t max_seqs, int32_t dtype, char* msg, size_t len) {
    sca::KVCacheConfig cfg;
    cfg.num_layers = layers;
    cfg.num_kv_heads = heads;
    cfg.head_dim = d;
    cfg.block_size = bs;
    cfg.num_blocks = nb;
    cfg.max_num_seqs = max_seqs;
    cfg.dtype = static_cast<sci::DType>(dtype);
    const auto r = sca::KvCacheBytes(cfg);
    if (!r.ok()) {
        CopyMsg(r.error().message(), msg, len);
        return -static_cast<int64_t>(CodeOf(r.error()));
    }
    return static_cast<int64_t>(*r);
}

int64_t ref_max_blocks_for_budget(int64_t layers, int64_t heads, int64_t d, int64_t bs,
                                  int32_t dtype, uint64_t budget) {
    sca::KVCacheConfig cfg;
    cfg.num_layers = layers;
    cfg.num_kv_heads = heads;
    cfg.head_dim = d;
    cfg.block_size = bs;
    cfg.dtype = static_cast<sci::DType>(dtype);
    return sca::MaxBlocksForBudget(cfg, budget);
}

int64_t ref_splits_for(int64_t seq_kv, int64_t sms) { return sca::decode::SplitsFor(seq_kv, sms); }
int64_t ref_partial_elements(int64_t b, int64_t h, int64_t s, int64_t d) {
    return sca::decode::PartialElements(b, h, s, d);
}

// ---- BlockManager ----------------------------------------------------------------------------------
void* ref_bm_create(int64_t nb, int64_t max_seqs, int64_t max_blocks, char* msg, size_t len) {
    auto r = sca::BlockManager::Create(nb, max_seqs, max_blocks, sci::StubHostDevice());
    if (!r.ok()) {
        CopyMsg(r.error().message(), msg, len);
        return nullptr;
    }
    return new sca::BlockManager(std::move(*r));
}
void ref_bm_destroy(void* h) { delete static_cast<sca::BlockManager*>(h); }
int ref_bm_allocate(void* h, int64_t count, int32_t* out, char* msg, size_t len) {
    auto r = static_cast<sca::BlockManager*>(h)->Allocate(count);
    if (!r.ok()) {
        CopyMsg(r.error().message(), msg, len);
        return CodeOf(r.error());
    }
    std::memcpy(out, r->data(), sizeof(int32_t) * r->size());
    return 0;
}
void ref_bm_free(void* h, const int32_t* ids, int64_t count) {
    static_cast<sca::BlockManager*>(h)->Free(ids, count);
}
int ref_bm_append_to_table(void* h, int64_t seq, const int32_t* ids, int64_t count, char* msg,
                           size_t len) {
    const sci::Status st = static_cast<sca::BlockManager*>(h)->AppendToTable(seq, ids, count);
    CopyMsg(st.message(), msg, len);
    return CodeOf(st);
}
int ref_bm_reset_seq(void* h, int64_t seq, char* msg, size_t len) {
    const sci::Status st = static_cast<sca::BlockManager*>(h)->ResetSeq(seq);
    CopyMsg(st.message(), msg, len);
    return CodeOf(st);
}
int ref_bm_sync(void* h) {
    return CodeOf(static_cast<sca::BlockManager*>(h)->SyncTableToDevice(nullptr));
}
int64_t ref_bm_num_free(void* h) { return static_cast<sca::BlockManager*>(h)->NumFreeBlocks(); }
int64_t ref_bm_failures(void* h) { return static_cast<sca::BlockManager*>(h)->AllocationFailures(); }
int64_t ref_bm_double_frees(void* h) { return static_cast<sca::BlockManager*>(h)->DoubleFreeEvents(); }
uint64_t ref_bm_revision(void* h) { return static_cast<sca::BlockManager*>(h)->Table().revision; }
uint64_t ref_bm_synced_revision(void* h) {
    return static_cast<sca::BlockManager*>(h)->Table().synced_revision;
}
void ref_bm_table(void* h, int32_t* out) {
    const auto& t = static_cast<sca::BlockManager*>(h)->Table().host;
    std::memcpy(out, t.data(), sizeof(int32_t) * t.size());
}

// ---- Workspace -------------------------------------------------------------------------------------
void* ref_ws_create(uint64_t bytes, char* msg, size_t len) {
    auto r = sca::Workspace::Create(bytes, sci::StubHostDevice());
    if (!r.ok()) {
        CopyMsg(r.error().message(), msg, len);
        return nullptr;
    }
    return new sca::Workspace(*r);
}
void ref_ws_destroy(void* h) { delete static_cast<sca::Workspace*>(h); }
int ref_ws_slice(void* h, uint64_t offset, uint64_t bytes, uint64_t align, uint64_t* rel,
                 char* msg, size_t len) {
    auto* ws = static_cast<sca::Workspace*>(h);
    auto r = ws->Slice(offset, bytes, align);
    if (!r.ok()) {
        CopyMsg(r.error().message(), msg, len);
        return CodeOf(r.error());
    }
    *rel = static_cast<uint64_t>(static_cast<unsigned char*>(*r) -
                                 static_cast<unsigned char*>(ws->Data()));
    return 0;
}
int ref_ws_reset(void* h) { return CodeOf(static_cast<sca::Workspace*>(h)->Reset()); }
uint64_t ref_ws_peak(void* h) { return static_cast<sca::Workspace*>(h)->PeakBytes(); }
uint64_t ref_ws_slices(void* h) { return static_cast<sca::Workspace*>(h)->AllocatedSlices(); }

}  // extern "C"

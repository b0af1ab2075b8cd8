/*
 * sca_capi.h - C ABI of the host library `libsca_host.so`: the sca:: C++ API (dispatcher,
 * validation, flash / decode / paged attention, KV cache, BlockManager, PagedKVCache, Workspace)
 * behind plain functions, POD structs and opaque handles, for bindings that cannot call C++
 * (ctypes, cgo, JNI). The reference exposes this surface only as C++; each group below names the
 * C++ entry points it forwards to (file:line in the reference's include/scicompute_attention/).
 *
 * Conventions
 *   - Functions returning `int` return 0 on success and otherwise the attention status code
 *     (2001..2010) carried by the failing sci::Status, or 1 when the status carries none. The
 *     full message ("[SCA-<code>] ...") of the last failure on the calling thread is returned by
 *     sca_last_error().
 *   - Handles (ScaTensor*, ScaPagedKV*, ...) are owned by the caller and released with the
 *     matching *_free / *_destroy function.
 *   - Device kinds: 0 = host memory, 1 = GPU 0.
 *   - `stream` is a hipStream_t passed as void*; NULL means the calling thread's current stream.
 */
#ifndef SCA_CAPI_H_
#define SCA_CAPI_H_

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define SCA_CAPI __attribute__((visibility("default")))
#else
#define SCA_CAPI
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* sca::AttentionConfig (attention_config.hpp:20-37); cu_seqlens pointers are host arrays. */
typedef struct ScaConfig {
    int32_t backend;        /* sca::BackendKind: 0 auto, 1 naive, 2 tiled, 3 flash, 4 decode, 5 paged */
    int32_t layout;         /* 0 bhsd, 1 bshd */
    int32_t causal;
    int32_t return_lse;
    float scale;            /* 0 => 1/sqrt(head_dim) */
    float softcap;
    int64_t sliding_window;
    int64_t num_splits;
    int32_t allow_fallback;
    int32_t reserved;
    const int32_t* cu_seqlens_q;
    const int32_t* cu_seqlens_kv;
    void* stream;
} ScaConfig;

/* sca::AttentionShape (attention_types.hpp:25-37). */
typedef struct ScaShape {
    int64_t batch, seq_q, seq_kv, num_heads, num_kv_heads, head_dim;
} ScaShape;

/* sca::KVCacheConfig (kv_cache.hpp:15-25). */
typedef struct ScaKvConfig {
    int64_t num_layers, num_kv_heads, head_dim, block_size, num_blocks, max_num_seqs;
    int32_t dtype;          /* sci::DType: 0 f32, 1 f16, 2 bf16 */
    int32_t layout;         /* 0 block-major */
} ScaKvConfig;

/* sca::AttentionRuntimeStats (attention_result.hpp:14-23). */
typedef struct ScaStats {
    int32_t used_backend;
    int32_t tile[4];        /* block_m, block_n, warps (waves), stages */
    uint64_t workspace_bytes;
    uint64_t kv_bytes;
    int64_t num_splits;
    int64_t materialized_score_bytes;
    char note[256];
} ScaStats;

/* sca::KVCacheStats (kv_cache.hpp:27-35). */
typedef struct ScaKvStats {
    int64_t num_blocks, used_blocks, free_blocks, num_appends, num_resets;
    uint64_t peak_bytes, bytes;
} ScaKvStats;

/* sca::PagedAttentionParams (paged_attention.hpp:13-21). */
typedef struct ScaPagedParams {
    const int32_t* page_table;   /* device; NULL => the cache's own */
    const int32_t* seq_lens;     /* device; NULL => every mapped page of the row */
    int64_t num_seqs;
    int64_t block_size;          /* <= 0 => the cache's */
    int64_t max_blocks_per_seq;  /* <= 0 => the cache's */
    int64_t layer;
} ScaPagedParams;

typedef struct ScaTensor ScaTensor;           /* sci::Tensor */
typedef struct ScaPagedKV ScaPagedKV;         /* sca::PagedKVCache */
typedef struct ScaBlockManager ScaBlockManager; /* sca::BlockManager */
typedef struct ScaWorkspace ScaWorkspace;     /* sca::Workspace */

SCA_CAPI const char* sca_last_error(void);

/* ---- version, status, names (status.hpp:12-41, attention_types.hpp:39-58, version.hpp) ---- */
SCA_CAPI const char* sca_version(void);
SCA_CAPI const char* sca_build_flavor(void);
SCA_CAPI const char* sca_status_name(int code);
SCA_CAPI int sca_to_sci_code(int code);
SCA_CAPI int sca_make_status(int code, const char* detail, char* msg, size_t len);
SCA_CAPI int sca_extract_code(const char* message);
SCA_CAPI const char* sca_backend_name(int kind);
SCA_CAPI const char* sca_layout_name(int layout);
SCA_CAPI int sca_parse_backend(const char* name, int32_t* kind);
SCA_CAPI int sca_supported_head_dim_index(int64_t head_dim);
SCA_CAPI int64_t sca_tile_smem_bytes_flash(int32_t head_dim, int64_t elem_bytes, int32_t block_m,
                                          int32_t block_n, int32_t warps, int32_t stages);
SCA_CAPI int64_t sca_flash_lds_bytes(int64_t head_dim, int64_t elem_bytes);

/* ---- validation and dispatch (attention_config.hpp:40-58, dispatcher.hpp:24-52) ---- */
SCA_CAPI int sca_validate(const ScaConfig* cfg, const ScaShape* shape, char* detail, size_t len);
SCA_CAPI float sca_effective_scale(const ScaConfig* cfg, const ScaShape* shape);
SCA_CAPI int sca_validate_varlen(const int32_t* cu_seqlens, int64_t batch, int64_t* max_seq);
SCA_CAPI int sca_select(const ScaConfig* cfg, const ScaShape* shape, int32_t* backend,
                        int32_t* tile4, uint64_t* workspace_bytes, char* reason, size_t len);
SCA_CAPI void sca_explain(const ScaConfig* cfg, const ScaShape* shape, char* out, size_t len);
SCA_CAPI void sca_recommend_tile(const ScaConfig* cfg, const ScaShape* shape, int32_t* tile4);
SCA_CAPI int64_t sca_decode_splits(const ScaShape* shape, int64_t cu_count);
/* Length-aware work split of the paged MFMA decode kernel (no reference counterpart: the
 * reference sizes paged splits from the pool alone). lengths = the batch's host-side key counts;
 * writes the split count and the sca_decode_params.slot_waves value (1 or 4; 0 with splits 1
 * when every length is 0) the paged backend uses when the cache's own page table is attended.
 * Returns 0, or SCA_E_SHAPE_MISMATCH. */
SCA_CAPI int sca_paged_decode_plan(const int64_t* lengths, int64_t batch, int64_t num_heads,
                                   int64_t num_kv_heads, int64_t cu_count, int64_t* splits,
                                   int32_t* slot_waves);

/* ---- KV helpers (kv_cache.hpp:97-110) ---- */
SCA_CAPI int sca_compute_slot_mapping(const int32_t* row, int64_t seq_start, int64_t num_tokens,
                                      int64_t block_size, int64_t max_blocks, int32_t* slots);
SCA_CAPI int sca_kv_cache_bytes(const ScaKvConfig* cfg, uint64_t* bytes);
SCA_CAPI int64_t sca_max_blocks_for_budget(const ScaKvConfig* cfg, uint64_t budget_bytes);

/* ---- tensors (sci::Tensor) ---- */
SCA_CAPI ScaTensor* sca_tensor_new(const int64_t* dims, int32_t ndims, int32_t dtype,
                                   int32_t device_kind);
/* Non-owning view of existing memory (GPU when device_kind = 1). */
SCA_CAPI ScaTensor* sca_tensor_wrap(void* data, const int64_t* dims, int32_t ndims, int32_t dtype,
                                    int32_t device_kind);
SCA_CAPI void sca_tensor_free(ScaTensor* t);
SCA_CAPI void* sca_tensor_data(ScaTensor* t);
SCA_CAPI uint64_t sca_tensor_nbytes(const ScaTensor* t);
SCA_CAPI int32_t sca_tensor_ndims(const ScaTensor* t);
SCA_CAPI int64_t sca_tensor_dim(const ScaTensor* t, int32_t i);
SCA_CAPI int sca_tensor_upload(ScaTensor* t, const void* host, uint64_t bytes);
SCA_CAPI int sca_tensor_download(const ScaTensor* t, void* host, uint64_t bytes);

/* ---- attention (attention.hpp:31-56, flash_attention.hpp, decode_attention.hpp) ----
 * entry: 0 sca::attention, 1 flash_attention, 2 decode_attention, 3 sca::decode, 4 naive_attention,
 * 5 tiled_attention. On success *out (and *lse when cfg->return_lse) receive new tensors. */
SCA_CAPI int sca_run_attention(int32_t entry, const ScaTensor* q, const ScaTensor* k,
                               const ScaTensor* v, const ScaConfig* cfg, ScaTensor** out,
                               ScaTensor** lse, ScaStats* stats);
SCA_CAPI int sca_run_flash_varlen(const ScaTensor* q, const ScaTensor* k, const ScaTensor* v,
                                  int64_t num_seqs, const int32_t* cu_seqlens_q,
                                  const int32_t* cu_seqlens_kv, int64_t max_seq_q,
                                  int64_t max_seq_kv, const ScaConfig* cfg, ScaTensor** out,
                                  ScaStats* stats);
SCA_CAPI void sca_explain_tensors(const ScaTensor* q, const ScaTensor* k, const ScaTensor* v,
                                  const ScaConfig* cfg, char* out, size_t len);

/* ---- paged KV cache (paged_kv_cache.hpp:20-68, paged_attention.hpp:23-31) ---- */
SCA_CAPI ScaPagedKV* sca_pkv_create(const ScaKvConfig* cfg, int32_t device_kind);
SCA_CAPI void sca_pkv_destroy(ScaPagedKV* c);
SCA_CAPI int sca_pkv_append(ScaPagedKV* c, int64_t seq_id, int64_t layer, const ScaTensor* k_new,
                            const ScaTensor* v_new, void* stream);
/* One token per sequence id, in order (sca::PagedKVCache::AppendTokensBatch; no reference
 * counterpart: the reference appends one sequence per call). */
SCA_CAPI int sca_pkv_append_batch(ScaPagedKV* c, const int64_t* seq_ids, int64_t num_entries,
                                  int64_t layer, const ScaTensor* k_new, const ScaTensor* v_new,
                                  void* stream);
/* Multi-layer appends (sca::PagedKVCache::ReserveTokens / ReserveTokensBatch /
 * WriteReservedLayer; no reference counterpart): reserve pages and slots and advance the lengths
 * once, then write each layer's K/V rows into the reserved slots. */
SCA_CAPI int sca_pkv_reserve(ScaPagedKV* c, int64_t seq_id, int64_t num_tokens, void* stream);
SCA_CAPI int sca_pkv_reserve_batch(ScaPagedKV* c, const int64_t* seq_ids, int64_t num_entries,
                                   void* stream);
SCA_CAPI int sca_pkv_write_layer(ScaPagedKV* c, int64_t layer, const ScaTensor* k_new,
                                 const ScaTensor* v_new, void* stream);
/* One call for all layers (sca::PagedKVCache::AppendTokensBatchAllLayers): k_layers/v_layers
 * are [num_layers, num_entries, num_kv_heads, head_dim]. */
SCA_CAPI int sca_pkv_append_batch_all_layers(ScaPagedKV* c, const int64_t* seq_ids,
                                             int64_t num_entries, const ScaTensor* k_layers,
                                             const ScaTensor* v_layers, void* stream);
SCA_CAPI int sca_pkv_reset(ScaPagedKV* c, int64_t seq_id, void* stream);
SCA_CAPI int sca_pkv_sync(ScaPagedKV* c, void* stream);
SCA_CAPI int sca_pkv_force_sync(ScaPagedKV* c, void* stream);
SCA_CAPI const int32_t* sca_pkv_page_table_device(const ScaPagedKV* c);
SCA_CAPI void sca_pkv_page_table_host(const ScaPagedKV* c, int32_t* out);
SCA_CAPI int64_t sca_pkv_seq_len(const ScaPagedKV* c, int64_t seq_id);
SCA_CAPI int64_t sca_pkv_block_count(const ScaPagedKV* c, int64_t seq_id);
SCA_CAPI int64_t sca_pkv_max_blocks_per_seq(const ScaPagedKV* c);
SCA_CAPI uint64_t sca_pkv_revision(const ScaPagedKV* c);
SCA_CAPI uint64_t sca_pkv_synced_revision(const ScaPagedKV* c);
SCA_CAPI void sca_pkv_stats(const ScaPagedKV* c, ScaKvStats* out);
SCA_CAPI void* sca_pkv_layer_k(const ScaPagedKV* c, int64_t layer);
SCA_CAPI void* sca_pkv_layer_v(const ScaPagedKV* c, int64_t layer);
/* The cache's BlockManager (borrowed; valid while the cache lives). */
SCA_CAPI const ScaBlockManager* sca_pkv_blocks(const ScaPagedKV* c);
/* KVCache::GatherK / GatherV of the cache's storage; ids are device int32. */
SCA_CAPI int sca_pkv_gather(const ScaPagedKV* c, int32_t is_key, int64_t layer,
                            const int32_t* block_ids, int64_t num_blocks, void* stream,
                            ScaTensor** out);
SCA_CAPI int sca_run_paged(const ScaTensor* q, const ScaPagedKV* kv, const ScaPagedParams* params,
                           const ScaConfig* cfg, ScaTensor** out, ScaStats* stats);

/* ---- BlockManager (block_manager.hpp:31-61) ---- */
SCA_CAPI ScaBlockManager* sca_bm_create(int64_t num_blocks, int64_t max_num_seqs,
                                        int64_t max_blocks_per_seq, int32_t device_kind);
SCA_CAPI void sca_bm_destroy(ScaBlockManager* bm);
SCA_CAPI int sca_bm_allocate(ScaBlockManager* bm, int64_t count, int32_t* out);
SCA_CAPI void sca_bm_free(ScaBlockManager* bm, const int32_t* ids, int64_t count);
SCA_CAPI int sca_bm_append_to_table(ScaBlockManager* bm, int64_t seq_id, const int32_t* ids,
                                    int64_t count);
SCA_CAPI int sca_bm_reset_seq(ScaBlockManager* bm, int64_t seq_id);
SCA_CAPI int sca_bm_sync(ScaBlockManager* bm, void* stream);
SCA_CAPI int64_t sca_bm_num_free(const ScaBlockManager* bm);
SCA_CAPI int64_t sca_bm_num_total(const ScaBlockManager* bm);
SCA_CAPI int64_t sca_bm_failures(const ScaBlockManager* bm);
SCA_CAPI int64_t sca_bm_double_frees(const ScaBlockManager* bm);
SCA_CAPI uint64_t sca_bm_revision(const ScaBlockManager* bm);
SCA_CAPI uint64_t sca_bm_synced_revision(const ScaBlockManager* bm);
SCA_CAPI void sca_bm_table(const ScaBlockManager* bm, int32_t* out);
/* Device copy of the table (as last synced) into host memory. */
SCA_CAPI int sca_bm_table_device(const ScaBlockManager* bm, int32_t* out);

/* ---- Workspace (workspace.hpp:17-50) ---- */
SCA_CAPI ScaWorkspace* sca_ws_create(uint64_t bytes, int32_t device_kind);
SCA_CAPI void sca_ws_destroy(ScaWorkspace* ws);
SCA_CAPI int sca_ws_slice(ScaWorkspace* ws, uint64_t offset, uint64_t bytes, uint64_t align,
                          uint64_t* relative_offset);
SCA_CAPI int sca_ws_reset(ScaWorkspace* ws);
SCA_CAPI uint64_t sca_ws_peak(const ScaWorkspace* ws);
SCA_CAPI uint64_t sca_ws_slices(const ScaWorkspace* ws);

/* ---- device memory pool, scratch, capability (device.hpp, capability.hpp) ---- */
SCA_CAPI uint64_t sca_gpu_empty_cache(void);
SCA_CAPI uint64_t sca_gpu_cached_bytes(void);
SCA_CAPI uint64_t sca_gpu_allocated_bytes(void);
SCA_CAPI int sca_release_scratch(void);
SCA_CAPI uint64_t sca_scratch_high_water_bytes(void);
SCA_CAPI int sca_gpu_available(void);
SCA_CAPI int sca_device_cu_count(void);
SCA_CAPI int sca_synchronize(void);

#ifdef __cplusplus
}
#endif

#endif /* SCA_CAPI_H_ */

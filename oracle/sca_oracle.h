/*
 * sca_oracle.h - CPU oracle of the attention hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load this library, and
 * only as the checker (or, for the CPU baseline, as the thing timed on the host). The product path
 * (libsca_hip.so / libsca_host.so) never links, loads or calls it.
 *
 * Every function restates the reference's algorithm (DeRuiChen258/SciCompute-Attention) and cites
 * the file:line it follows. Layouts are contiguous BHSD unless stated otherwise.
 */
#ifndef SCA_ORACLE_H_
#define SCA_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- input generation and dtype encoders (tests/common/test_utils.hpp:24-131) -------------- */
void oracle_random_floats(float* out, size_t n, uint32_t seed, float low, float high);
uint16_t oracle_float_to_half_bits(float value);
float oracle_half_bits_to_float(uint16_t half);
uint16_t oracle_float_to_bf16_bits(float value);
float oracle_bf16_bits_to_float(uint16_t bits);
/* dtype: 1 = fp16, 2 = bf16. Writes the storage bits and the dequantised values. */
void oracle_encode(const float* values, size_t n, int dtype, uint16_t* bits, float* dequant);

/* ---- FP64 reference attention (tests/common/test_utils.hpp:229-285) ------------------------- */
/* q [B,Hq,Sq,D], k/v [B,Hkv,Skv,D] (dequantised floats). scale <= 0 means 1/sqrt(D).
 * rows: optional list of flat row ids (b*Hq + h)*Sq + i to evaluate (NULL = all rows, in order);
 * out receives n_rows*D doubles (row-major in the order of `rows`), lse n_rows doubles
 * (natural log; -inf for a fully masked row). threads <= 0 uses all cores. */
void oracle_reference_attention(const float* q, const float* k, const float* v, int64_t batch,
                                int64_t heads_q, int64_t heads_kv, int64_t seq_q, int64_t seq_kv,
                                int64_t head_dim, int causal, double scale, const int64_t* rows,
                                int64_t n_rows, double* out, double* lse, int threads);

/* ---- naive three-pass FP32 attention (src/backends/naive/attention_naive.cu:41-135) ---------- */
/* The CPU baseline: materialises scores [B,Hq,Sq,Skv] in `scores` (caller-provided), row softmax
 * with exp2((x-m)*log2e), all-masked rows -> zeros, then P.V with FP32 accumulation.
 * lse may be NULL. threads <= 0 uses all cores. */
void oracle_naive_attention_f32(const float* q, const float* k, const float* v, int64_t batch,
                                int64_t heads_q, int64_t heads_kv, int64_t seq_q, int64_t seq_kv,
                                int64_t head_dim, int causal, float scale, float* scores,
                                float* out, float* lse, int threads);

/* ---- split-K decode model (src/backends/decode/decode_splitk.cu:66-182) --------------------- */
/* q [B,Hq,1,D]; k/v [B,Hkv,Skv,D]; seq_lens optional [B]. Per (b,h,split) partials in double with
 * chunk = ceil(len/splits), then the LSE combine. part_* may be NULL. */
void oracle_splitk_decode(const float* q, const float* k, const float* v, int64_t batch,
                          int64_t heads_q, int64_t heads_kv, int64_t seq_kv, int64_t head_dim,
                          int64_t splits, double scale, const int32_t* seq_lens, double* out,
                          double* part_m, double* part_l, double* part_o);

/* ---- decode / KV-cache integer helpers -------------------------------------------------------- */
/* src/backends/decode/decode_config.hpp:24-40 */
int64_t oracle_splits_for(int64_t seq_kv, int64_t sm_count);
int64_t oracle_partial_elements(int64_t batch, int64_t heads_q, int64_t splits, int64_t head_dim);
/* src/kv_cache/kv_cache.cpp:79-132. Returns 0 or the attention status code; msg may be NULL. */
int oracle_compute_slot_mapping(const int32_t* row, int64_t seq_start, int64_t num_tokens,
                                int64_t block_size, int64_t max_blocks, int32_t* slots,
                                char* msg, size_t msg_len);
/* returns -1 when the config is invalid (same validation as kv_cache.cpp:36-77) */
int64_t oracle_kv_cache_bytes(int64_t num_layers, int64_t num_kv_heads, int64_t head_dim,
                              int64_t block_size, int64_t num_blocks, int64_t max_num_seqs,
                              int64_t elem_bytes);
int64_t oracle_max_blocks_for_budget(int64_t num_layers, int64_t num_kv_heads, int64_t head_dim,
                                     int64_t block_size, int64_t elem_bytes, uint64_t budget);

/* ---- BlockManager (src/kv_cache/block_manager.cpp:11-144) ----------------------------------- */
typedef struct oracle_block_manager oracle_block_manager;
oracle_block_manager* oracle_bm_create(int64_t num_blocks, int64_t max_num_seqs,
                                       int64_t max_blocks_per_seq);
void oracle_bm_destroy(oracle_block_manager* bm);
/* returns 0 or a status code; on success writes `count` ids. */
int oracle_bm_allocate(oracle_block_manager* bm, int64_t count, int32_t* out, char* msg,
                       size_t msg_len);
void oracle_bm_free(oracle_block_manager* bm, const int32_t* ids, int64_t count);
int oracle_bm_append_to_table(oracle_block_manager* bm, int64_t seq, const int32_t* ids,
                              int64_t count, char* msg, size_t msg_len);
int oracle_bm_reset_seq(oracle_block_manager* bm, int64_t seq, char* msg, size_t msg_len);
/* models SyncTableToDevice: returns 1 when an upload would happen, 0 when skipped */
int oracle_bm_sync(oracle_block_manager* bm);
int64_t oracle_bm_num_free(const oracle_block_manager* bm);
int64_t oracle_bm_failures(const oracle_block_manager* bm);
int64_t oracle_bm_double_frees(const oracle_block_manager* bm);
uint64_t oracle_bm_revision(const oracle_block_manager* bm);
uint64_t oracle_bm_synced_revision(const oracle_block_manager* bm);
/* copies the host table ([max_num_seqs * max_blocks_per_seq]) */
void oracle_bm_table(const oracle_block_manager* bm, int32_t* out);
/* copies the free list bottom-to-top (next allocation pops the last entry) */
int64_t oracle_bm_free_list(const oracle_block_manager* bm, int32_t* out);

/* ---- PagedKVCache host state (src/kv_cache/paged_kv_cache.cpp:13-211) ----------------------- */
/* Models the metadata only (no KV bytes): per-sequence length and owned blocks, its own page
 * table (row length = num_blocks), revision / synced revision, append/reset counters. */
typedef struct oracle_paged_kv oracle_paged_kv;
oracle_paged_kv* oracle_pkv_create(int64_t num_blocks, int64_t block_size, int64_t max_num_seqs,
                                   int64_t num_layers);
void oracle_pkv_destroy(oracle_paged_kv* c);
/* returns 0 or a status code; on success writes the slot mapping of the new tokens */
int oracle_pkv_append(oracle_paged_kv* c, int64_t seq, int64_t layer, int64_t num_tokens,
                      int32_t* slots, char* msg, size_t msg_len);
int oracle_pkv_reset(oracle_paged_kv* c, int64_t seq, char* msg, size_t msg_len);
int oracle_pkv_sync(oracle_paged_kv* c); /* 1 = upload, 0 = skipped (SyncPageTable) */
int64_t oracle_pkv_seq_len(const oracle_paged_kv* c, int64_t seq);
int64_t oracle_pkv_block_count(const oracle_paged_kv* c, int64_t seq);
void oracle_pkv_page_table(const oracle_paged_kv* c, int32_t* out);
/* stats: [used_blocks, free_blocks, num_appends, num_resets, revision, synced_revision] */
void oracle_pkv_stats(const oracle_paged_kv* c, int64_t* out6);
const oracle_block_manager* oracle_pkv_blocks(const oracle_paged_kv* c);

#ifdef __cplusplus
}
#endif

#endif /* SCA_ORACLE_H_ */

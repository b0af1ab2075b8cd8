/*
 * sca_oracle.c - CPU oracle of the attention hot path. TEST INFRASTRUCTURE ONLY.
 *
 * Loaded only by tests/, __graft_entry__.smoke() (as the checker) and bench.py's cpu_baseline leg
 * (the naive restatement is the CPU baseline that is timed). Never linked into the product.
 * Each function restates the reference's algorithm and names the file:line it follows.
 */
#include "sca_oracle.h"

#include <float.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* attention status codes (include/scicompute_attention/status.hpp:16-28) */
enum {
    kShapeMismatch = 2005,
    kKVCapacityExceeded = 2007,
    kUnsupportedFeature = 2009,
};

static void set_msg(char* msg, size_t len, const char* text) {
    if (msg != NULL && len > 0) {
        strncpy(msg, text, len - 1);
        msg[len - 1] = '\0';
    }
}

static int threads_or_all(int threads) {
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

/* ============================================================================================ */
/* input generation and encoders: tests/common/test_utils.hpp:24-101                            */
/* ============================================================================================ */

/* xorshift32 (13, 17, 5); unit = (float)state / (float)0xffffffff; value = low + unit*(high-low).
 * test_utils.hpp:24-38 */
void oracle_random_floats(float* out, size_t n, uint32_t seed, float low, float high) {
    uint32_t state = seed == 0 ? 1u : seed;
    for (size_t i = 0; i < n; ++i) {
        state ^= state << 13;
        state ^= state >> 17;
        state ^= state << 5;
        const float unit = (float)state / (float)0xffffffffu;
        out[i] = low + unit * (high - low);
    }
}

/* test_utils.hpp:48-65: results that would be fp16-subnormal flush to +-0, overflow -> +-inf,
 * round half to even on the 13 dropped mantissa bits. */
uint16_t oracle_float_to_half_bits(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    const uint32_t sign = (bits >> 16) & 0x8000u;
    const int32_t exponent = (int32_t)((bits >> 23) & 0xffu) - 127 + 15;
    const uint32_t mantissa = bits & 0x7fffffu;
    if (exponent <= 0) return (uint16_t)sign;
    if (exponent >= 31) return (uint16_t)(sign | 0x7c00u);
    uint16_t half = (uint16_t)(sign | ((uint32_t)exponent << 10) | (mantissa >> 13));
    const uint32_t remainder = mantissa & 0x1fffu;
    if (remainder > 0x1000u || (remainder == 0x1000u && (half & 1u) != 0u)) half = (uint16_t)(half + 1);
    return half;
}

/* test_utils.hpp:67-89 */
float oracle_half_bits_to_float(uint16_t half) {
    const uint32_t sign = (uint32_t)(half & 0x8000u) << 16;
    const uint32_t exponent = (half >> 10) & 0x1fu;
    const uint32_t mantissa = half & 0x3ffu;
    uint32_t bits = sign;
    if (exponent == 0) {
        if (mantissa != 0) {
            const float value = ldexpf((float)mantissa, -24);
            return sign ? -value : value;
        }
    } else if (exponent == 31) {
        bits |= 0x7f800000u | (mantissa << 13);
    } else {
        bits |= ((exponent - 15 + 127) << 23) | (mantissa << 13);
    }
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

/* test_utils.hpp:91-96: round half to even by adding 0x7fff + lsb (no NaN special case) */
uint16_t oracle_float_to_bf16_bits(float value) {
    uint32_t bits;
    memcpy(&bits, &value, sizeof(bits));
    bits += 0x7fffu + ((bits >> 16) & 1u);
    return (uint16_t)(bits >> 16);
}

/* test_utils.hpp:98-101 */
float oracle_bf16_bits_to_float(uint16_t b) {
    const uint32_t bits = (uint32_t)b << 16;
    float out;
    memcpy(&out, &bits, sizeof(out));
    return out;
}

/* test_utils.hpp:109-131 */
void oracle_encode(const float* values, size_t n, int dtype, uint16_t* bits, float* dequant) {
    for (size_t i = 0; i < n; ++i) {
        if (dtype == 1) {
            bits[i] = oracle_float_to_half_bits(values[i]);
            dequant[i] = oracle_half_bits_to_float(bits[i]);
        } else {
            bits[i] = oracle_float_to_bf16_bits(values[i]);
            dequant[i] = oracle_bf16_bits_to_float(bits[i]);
        }
    }
}

/* ============================================================================================ */
/* FP64 reference attention: tests/common/test_utils.hpp:229-285 (+ LSE as in                   */
/* tests/kernel/test_flash_correctness.cu:73-117)                                               */
/* ============================================================================================ */
void oracle_reference_attention(const float* q, const float* k, const float* v, int64_t batch,
                                int64_t heads_q, int64_t heads_kv, int64_t seq_q, int64_t seq_kv,
                                int64_t head_dim, int causal, double scale, const int64_t* rows,
                                int64_t n_rows, double* out, double* lse, int threads) {
    const int64_t group = heads_q / heads_kv;
    const int64_t diagonal = causal ? (seq_kv - seq_q) : 0;
    const double sc = scale > 0.0 ? scale : 1.0 / sqrt((double)head_dim);
    const int64_t total_rows = rows != NULL ? n_rows : batch * heads_q * seq_q;
    (void)batch;

#pragma omp parallel num_threads(threads_or_all(threads))
    {
        double* scores = (double*)malloc(sizeof(double) * (size_t)(seq_kv > 0 ? seq_kv : 1));
#pragma omp for schedule(dynamic, 4)
        for (int64_t r = 0; r < total_rows; ++r) {
            const int64_t flat = rows != NULL ? rows[r] : r;
            const int64_t i = flat % seq_q;
            const int64_t h = (flat / seq_q) % heads_q;
            const int64_t b = flat / (seq_q * heads_q);
            const int64_t h_kv = h / group;
            const float* q_row = q + ((b * heads_q + h) * seq_q + i) * head_dim;
            const float* k_head = k + (b * heads_kv + h_kv) * seq_kv * head_dim;
            const float* v_head = v + (b * heads_kv + h_kv) * seq_kv * head_dim;
            double m = -INFINITY;
            for (int64_t j = 0; j < seq_kv; ++j) {
                if (causal && j > i + diagonal) {
                    scores[j] = -INFINITY;
                    continue;
                }
                double dot = 0.0;
                const float* k_row = k_head + j * head_dim;
                for (int64_t d = 0; d < head_dim; ++d) dot += (double)q_row[d] * (double)k_row[d];
                dot *= sc;
                scores[j] = dot;
                if (dot > m) m = dot;
            }
            double sum = 0.0;
            for (int64_t j = 0; j < seq_kv; ++j) {
                if (isinf(scores[j])) continue;
                scores[j] = exp(scores[j] - m);
                sum += scores[j];
            }
            double* o = out + r * head_dim;
            for (int64_t d = 0; d < head_dim; ++d) o[d] = 0.0;
            if (sum > 0.0) {
                for (int64_t j = 0; j < seq_kv; ++j) {
                    if (isinf(scores[j])) continue;
                    const double p = scores[j] / sum;
                    const float* v_row = v_head + j * head_dim;
                    for (int64_t d = 0; d < head_dim; ++d) o[d] += p * (double)v_row[d];
                }
            }
            if (lse != NULL) lse[r] = sum > 0.0 ? m + log(sum) : -INFINITY;
        }
        free(scores);
    }
}

/* ============================================================================================ */
/* naive three-pass FP32 attention: src/backends/naive/attention_naive.cu:41-135                */
/* ============================================================================================ */
void oracle_naive_attention_f32(const float* q, const float* k, const float* v, int64_t batch,
                                int64_t heads_q, int64_t heads_kv, int64_t seq_q, int64_t seq_kv,
                                int64_t head_dim, int causal, float scale, float* scores,
                                float* out, float* lse, int threads) {
    const int64_t group = heads_q / heads_kv;
    const int64_t diagonal = causal ? (seq_kv - seq_q) : 0;
    const int64_t rows = batch * heads_q * seq_q;
    const float log2e = 1.4426950408889634f;
    const int nt = threads_or_all(threads);

    /* [1] QK^T * scale with the causal mask (attention_naive.cu:41-68) */
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t i = r % seq_q;
        const int64_t h = (r / seq_q) % heads_q;
        const int64_t b = r / (seq_q * heads_q);
        const float* q_row = q + r * head_dim;
        const float* k_head = k + (b * heads_kv + h / group) * seq_kv * head_dim;
        float* s_row = scores + r * seq_kv;
        for (int64_t j = 0; j < seq_kv; ++j) {
            const float* k_row = k_head + j * head_dim;
            float acc = 0.0f;
            for (int64_t d = 0; d < head_dim; ++d) acc += q_row[d] * k_row[d];
            acc *= scale;
            if (causal && j > i + diagonal) acc = -INFINITY;
            s_row[j] = acc;
        }
    }

    /* [2] row softmax, all-masked row -> zeros, LSE = m + log(sum) (attention_naive.cu:73-106) */
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float* s_row = scores + r * seq_kv;
        float m = -INFINITY;
        for (int64_t j = 0; j < seq_kv; ++j) m = fmaxf(m, s_row[j]);
        const int all_masked = !isfinite(m);
        float sum = 0.0f;
        if (!all_masked) {
            for (int64_t j = 0; j < seq_kv; ++j) {
                const float e = exp2f((s_row[j] - m) * log2e);
                s_row[j] = e;
                sum += e;
            }
        }
        const float inv = all_masked ? 0.0f : 1.0f / sum;
        for (int64_t j = 0; j < seq_kv; ++j) s_row[j] *= inv;
        if (lse != NULL) lse[r] = all_masked ? -INFINITY : m + logf(sum);
    }

    /* [3] P V with FP32 accumulation (attention_naive.cu:111-135) */
#pragma omp parallel for num_threads(nt) schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const int64_t h = (r / seq_q) % heads_q;
        const int64_t b = r / (seq_q * heads_q);
        const float* p_row = scores + r * seq_kv;
        const float* v_head = v + (b * heads_kv + h / group) * seq_kv * head_dim;
        float* o = out + r * head_dim;
        for (int64_t d = 0; d < head_dim; ++d) {
            float acc = 0.0f;
            for (int64_t j = 0; j < seq_kv; ++j) acc += p_row[j] * v_head[j * head_dim + d];
            o[d] = acc;
        }
    }
}

/* ============================================================================================ */
/* split-K decode model: src/backends/decode/decode_splitk.cu:66-182                            */
/* ============================================================================================ */
void oracle_splitk_decode(const float* q, const float* k, const float* v, int64_t batch,
                          int64_t heads_q, int64_t heads_kv, int64_t seq_kv, int64_t head_dim,
                          int64_t splits, double scale, const int32_t* seq_lens, double* out,
                          double* part_m, double* part_l, double* part_o) {
    const int64_t group = heads_q / heads_kv;
    const double sc = scale > 0.0 ? scale : 1.0 / sqrt((double)head_dim);
    double* acc = (double*)malloc(sizeof(double) * (size_t)head_dim);
    double* pm = (double*)malloc(sizeof(double) * (size_t)splits);
    double* pl = (double*)malloc(sizeof(double) * (size_t)splits);
    double* po = (double*)malloc(sizeof(double) * (size_t)(splits * head_dim));
    for (int64_t b = 0; b < batch; ++b) {
        const int64_t len = seq_lens != NULL ? (int64_t)seq_lens[b] : seq_kv;
        const int64_t chunk = (len + splits - 1) / splits;
        for (int64_t h = 0; h < heads_q; ++h) {
            const int64_t h_kv = h / group;
            const float* q_row = q + (b * heads_q + h) * head_dim;
            const float* k_head = k + (b * heads_kv + h_kv) * seq_kv * head_dim;
            const float* v_head = v + (b * heads_kv + h_kv) * seq_kv * head_dim;
            /* partial kernel (decode_splitk.cu:98-139) */
            for (int64_t s = 0; s < splits; ++s) {
                const int64_t j0 = s * chunk;
                const int64_t j1 = j0 + chunk < len ? j0 + chunk : len;
                double m = -INFINITY, l = 0.0;
                for (int64_t d = 0; d < head_dim; ++d) acc[d] = 0.0;
                for (int64_t j = j0; j < j1; ++j) {
                    double dot = 0.0;
                    for (int64_t d = 0; d < head_dim; ++d) {
                        dot += (double)q_row[d] * (double)k_head[j * head_dim + d];
                    }
                    dot *= sc;
                    const double m_new = dot > m ? dot : m;
                    const double alpha = isinf(m) ? 0.0 : exp(m - m_new);
                    const double p = exp(dot - m_new);
                    l = alpha * l + p;
                    for (int64_t d = 0; d < head_dim; ++d) {
                        acc[d] = alpha * acc[d] + p * (double)v_head[j * head_dim + d];
                    }
                    m = m_new;
                }
                pm[s] = m;
                pl[s] = l;
                for (int64_t d = 0; d < head_dim; ++d) po[s * head_dim + d] = acc[d];
            }
            /* combine (decode_splitk.cu:143-182) */
            double m_all = -INFINITY;
            for (int64_t s = 0; s < splits; ++s) m_all = pm[s] > m_all ? pm[s] : m_all;
            double l_all = 0.0;
            for (int64_t s = 0; s < splits; ++s) {
                if (isinf(pm[s]) && pm[s] < 0) continue;
                l_all += pl[s] * exp(pm[s] - m_all);
            }
            const double inv = l_all > 0.0 ? 1.0 / l_all : 0.0;
            double* o = out + (b * heads_q + h) * head_dim;
            for (int64_t d = 0; d < head_dim; ++d) {
                double total = 0.0;
                for (int64_t s = 0; s < splits; ++s) {
                    if (isinf(pm[s]) && pm[s] < 0) continue;
                    total += po[s * head_dim + d] * exp(pm[s] - m_all);
                }
                o[d] = total * inv;
            }
            const int64_t base = (b * heads_q + h) * splits;
            for (int64_t s = 0; s < splits; ++s) {
                if (part_m != NULL) part_m[base + s] = pm[s];
                if (part_l != NULL) part_l[base + s] = pl[s];
                if (part_o != NULL) {
                    for (int64_t d = 0; d < head_dim; ++d) {
                        part_o[(base + s) * head_dim + d] = po[s * head_dim + d];
                    }
                }
            }
        }
    }
    free(acc);
    free(pm);
    free(pl);
    free(po);
}

/* ============================================================================================ */
/* integer helpers                                                                               */
/* ============================================================================================ */

/* src/backends/decode/decode_config.hpp:24-31 (tokens per split 512, max splits 16) */
int64_t oracle_splits_for(int64_t seq_kv, int64_t sm_count) {
    if (seq_kv <= 0) return 1;
    int64_t splits = (seq_kv + 512 - 1) / 512;
    const int64_t cap = sm_count > 0 ? sm_count * 2 : 16;
    if (splits > cap) splits = cap;
    if (splits > 16) splits = 16;
    return splits < 1 ? 1 : splits;
}

/* src/backends/decode/decode_config.hpp:36-40 */
int64_t oracle_partial_elements(int64_t batch, int64_t heads_q, int64_t splits, int64_t head_dim) {
    return batch * heads_q * splits * (2 + head_dim);
}

/* src/kv_cache/kv_cache.cpp:99-132 */
int oracle_compute_slot_mapping(const int32_t* row, int64_t seq_start, int64_t num_tokens,
                                int64_t block_size, int64_t max_blocks, int32_t* slots,
                                char* msg, size_t msg_len) {
    char buf[256];
    if (row == NULL) {
        set_msg(msg, msg_len, "ComputeSlotMapping: null block table row");
        return kShapeMismatch;
    }
    if (block_size <= 0 || num_tokens <= 0) {
        set_msg(msg, msg_len, "ComputeSlotMapping: block_size/num_tokens <= 0");
        return kShapeMismatch;
    }
    for (int64_t t = 0; t < num_tokens; ++t) {
        const int64_t position = seq_start + t;
        const int64_t logical = position / block_size;
        const int64_t offset = position % block_size;
        if (logical >= max_blocks) {
            snprintf(buf, sizeof(buf), "ComputeSlotMapping: logical block %lld >= max_blocks=%lld",
                     (long long)logical, (long long)max_blocks);
            set_msg(msg, msg_len, buf);
            return kKVCapacityExceeded;
        }
        const int32_t physical = row[logical];
        if (physical < 0) {
            snprintf(buf, sizeof(buf),
                     "ComputeSlotMapping: block table slot %lld is empty (-1) for position %lld",
                     (long long)logical, (long long)position);
            set_msg(msg, msg_len, buf);
            return kShapeMismatch;
        }
        slots[t] = (int32_t)(physical * block_size + offset);
    }
    return 0;
}

static int supported_head_dim(int64_t d) {
    return d == 32 || d == 64 || d == 96 || d == 128 || d == 160 || d == 192 || d == 256;
}

static int supported_block_size(int64_t bs) {
    return bs == 1 || bs == 8 || bs == 16 || bs == 32 || bs == 64;
}

/* src/kv_cache/kv_cache.cpp:36-97 */
int64_t oracle_kv_cache_bytes(int64_t num_layers, int64_t num_kv_heads, int64_t head_dim,
                              int64_t block_size, int64_t num_blocks, int64_t max_num_seqs,
                              int64_t elem_bytes) {
    if (num_layers <= 0 || num_kv_heads <= 0 || !supported_head_dim(head_dim) ||
        !supported_block_size(block_size) || num_blocks <= 0 || max_num_seqs <= 0) {
        return -1;
    }
    const int64_t per_layer = num_blocks * block_size * num_kv_heads * head_dim;
    const int64_t total = 2 * num_layers * per_layer * elem_bytes;
    return total > 0 ? total : -1;
}

int64_t oracle_max_blocks_for_budget(int64_t num_layers, int64_t num_kv_heads, int64_t head_dim,
                                     int64_t block_size, int64_t elem_bytes, uint64_t budget) {
    const int64_t per_block = 2 * num_layers * block_size * num_kv_heads * head_dim * elem_bytes;
    if (per_block <= 0) return 0;
    return (int64_t)(budget / (uint64_t)per_block);
}

/* ============================================================================================ */
/* BlockManager: src/kv_cache/block_manager.cpp:11-144                                          */
/* ============================================================================================ */
struct oracle_block_manager {
    int64_t num_blocks;
    int32_t* free_list; /* LIFO: allocate pops from the back */
    int64_t free_count;
    uint8_t* in_use;
    int32_t* table;     /* [max_num_seqs * max_blocks_per_seq], -1 = empty */
    int64_t max_num_seqs;
    int64_t max_blocks_per_seq;
    uint64_t revision;
    uint64_t synced_revision;
    int64_t allocation_failures;
    int64_t double_free_events;
};

/* block_manager.cpp:11-44: free list seeded num_blocks-1 ... 0, table all -1 */
oracle_block_manager* oracle_bm_create(int64_t num_blocks, int64_t max_num_seqs,
                                       int64_t max_blocks_per_seq) {
    if (num_blocks <= 0 || max_num_seqs <= 0 || max_blocks_per_seq <= 0) return NULL;
    oracle_block_manager* bm = (oracle_block_manager*)calloc(1, sizeof(*bm));
    bm->num_blocks = num_blocks;
    bm->free_list = (int32_t*)malloc(sizeof(int32_t) * (size_t)num_blocks);
    bm->in_use = (uint8_t*)calloc((size_t)num_blocks, 1);
    for (int64_t i = num_blocks - 1, n = 0; i >= 0; --i, ++n) bm->free_list[n] = (int32_t)i;
    bm->free_count = num_blocks;
    bm->max_num_seqs = max_num_seqs;
    bm->max_blocks_per_seq = max_blocks_per_seq;
    bm->table = (int32_t*)malloc(sizeof(int32_t) * (size_t)(max_num_seqs * max_blocks_per_seq));
    for (int64_t i = 0; i < max_num_seqs * max_blocks_per_seq; ++i) bm->table[i] = -1;
    return bm;
}

void oracle_bm_destroy(oracle_block_manager* bm) {
    if (bm == NULL) return;
    free(bm->free_list);
    free(bm->in_use);
    free(bm->table);
    free(bm);
}

/* block_manager.cpp:46-67: all-or-nothing, failure counted, message carries free/total */
int oracle_bm_allocate(oracle_block_manager* bm, int64_t count, int32_t* out, char* msg,
                       size_t msg_len) {
    char buf[256];
    if (count <= 0) {
        snprintf(buf, sizeof(buf), "BlockManager::Allocate count=%lld", (long long)count);
        set_msg(msg, msg_len, buf);
        return kShapeMismatch;
    }
    if (count > bm->free_count) {
        ++bm->allocation_failures;
        snprintf(buf, sizeof(buf),
                 "BlockManager::Allocate requested %lld blocks but only %lld of %lld are free",
                 (long long)count, (long long)bm->free_count, (long long)bm->num_blocks);
        set_msg(msg, msg_len, buf);
        return kKVCapacityExceeded;
    }
    for (int64_t i = 0; i < count; ++i) {
        const int32_t block = bm->free_list[--bm->free_count];
        bm->in_use[block] = 1;
        out[i] = block;
    }
    return 0;
}

/* block_manager.cpp:69-84: invalid or not-in-use ids are counted and skipped */
void oracle_bm_free(oracle_block_manager* bm, const int32_t* ids, int64_t count) {
    if (ids == NULL || count <= 0) return;
    for (int64_t i = 0; i < count; ++i) {
        const int32_t block = ids[i];
        if (block < 0 || block >= bm->num_blocks) {
            ++bm->double_free_events;
            continue;
        }
        if (bm->in_use[block] == 0) {
            ++bm->double_free_events;
            continue;
        }
        bm->in_use[block] = 0;
        bm->free_list[bm->free_count++] = block;
    }
}

/* block_manager.cpp:86-109: append after the first -1 slot, revision++ */
int oracle_bm_append_to_table(oracle_block_manager* bm, int64_t seq, const int32_t* ids,
                              int64_t count, char* msg, size_t msg_len) {
    char buf[256];
    if (seq < 0 || seq >= bm->max_num_seqs) {
        snprintf(buf, sizeof(buf), "BlockManager::AppendToTable seq_id=%lld out of range [0,%lld)",
                 (long long)seq, (long long)bm->max_num_seqs);
        set_msg(msg, msg_len, buf);
        return kShapeMismatch;
    }
    if (ids == NULL || count <= 0) {
        set_msg(msg, msg_len, "BlockManager::AppendToTable requires block_ids and count > 0");
        return kShapeMismatch;
    }
    int32_t* row = bm->table + seq * bm->max_blocks_per_seq;
    int64_t used = 0;
    while (used < bm->max_blocks_per_seq && row[used] >= 0) ++used;
    if (used + count > bm->max_blocks_per_seq) {
        snprintf(buf, sizeof(buf),
                 "BlockManager::AppendToTable sequence %lld would need %lld blocks > "
                 "max_blocks_per_seq=%lld",
                 (long long)seq, (long long)(used + count), (long long)bm->max_blocks_per_seq);
        set_msg(msg, msg_len, buf);
        return kKVCapacityExceeded;
    }
    for (int64_t i = 0; i < count; ++i) row[used + i] = ids[i];
    ++bm->revision;
    return 0;
}

/* block_manager.cpp:111-126: free the row's ids in row order, clear, revision++ (always) */
int oracle_bm_reset_seq(oracle_block_manager* bm, int64_t seq, char* msg, size_t msg_len) {
    char buf[256];
    if (seq < 0 || seq >= bm->max_num_seqs) {
        snprintf(buf, sizeof(buf), "BlockManager::ResetSeq seq_id=%lld out of range",
                 (long long)seq);
        set_msg(msg, msg_len, buf);
        return kShapeMismatch;
    }
    int32_t* row = bm->table + seq * bm->max_blocks_per_seq;
    int64_t count = 0;
    for (int64_t i = 0; i < bm->max_blocks_per_seq; ++i) {
        if (row[i] >= 0) ++count;
    }
    if (count > 0) oracle_bm_free(bm, row, count);
    for (int64_t i = 0; i < bm->max_blocks_per_seq; ++i) row[i] = -1;
    ++bm->revision;
    return 0;
}

/* block_manager.cpp:128-142 */
int oracle_bm_sync(oracle_block_manager* bm) {
    if (bm->synced_revision == bm->revision) return 0;
    bm->synced_revision = bm->revision;
    return 1;
}

int64_t oracle_bm_num_free(const oracle_block_manager* bm) { return bm->free_count; }
int64_t oracle_bm_failures(const oracle_block_manager* bm) { return bm->allocation_failures; }
int64_t oracle_bm_double_frees(const oracle_block_manager* bm) { return bm->double_free_events; }
uint64_t oracle_bm_revision(const oracle_block_manager* bm) { return bm->revision; }
uint64_t oracle_bm_synced_revision(const oracle_block_manager* bm) { return bm->synced_revision; }

void oracle_bm_table(const oracle_block_manager* bm, int32_t* out) {
    memcpy(out, bm->table, sizeof(int32_t) * (size_t)(bm->max_num_seqs * bm->max_blocks_per_seq));
}

int64_t oracle_bm_free_list(const oracle_block_manager* bm, int32_t* out) {
    if (out != NULL) memcpy(out, bm->free_list, sizeof(int32_t) * (size_t)bm->free_count);
    return bm->free_count;
}

/* ============================================================================================ */
/* PagedKVCache host state: src/kv_cache/paged_kv_cache.cpp:13-211                              */
/* ============================================================================================ */
struct oracle_paged_kv {
    int64_t num_blocks;
    int64_t block_size;
    int64_t max_num_seqs;
    int64_t num_layers;
    oracle_block_manager* blocks;
    int64_t* seq_len;
    int32_t* owned;        /* [max_num_seqs * num_blocks] */
    int64_t* owned_count;
    int32_t* page_table;   /* [max_num_seqs * num_blocks] */
    uint64_t revision;
    uint64_t synced_revision;
    int64_t num_appends;
    int64_t num_resets;
};

/* paged_kv_cache.cpp:13-50: BlockManager(max_blocks_per_seq = num_blocks), revision 1/1 */
oracle_paged_kv* oracle_pkv_create(int64_t num_blocks, int64_t block_size, int64_t max_num_seqs,
                                   int64_t num_layers) {
    if (num_blocks <= 0 || block_size <= 0 || max_num_seqs <= 0 || num_layers <= 0) return NULL;
    oracle_paged_kv* c = (oracle_paged_kv*)calloc(1, sizeof(*c));
    c->num_blocks = num_blocks;
    c->block_size = block_size;
    c->max_num_seqs = max_num_seqs;
    c->num_layers = num_layers;
    c->blocks = oracle_bm_create(num_blocks, max_num_seqs, num_blocks);
    c->seq_len = (int64_t*)calloc((size_t)max_num_seqs, sizeof(int64_t));
    c->owned = (int32_t*)malloc(sizeof(int32_t) * (size_t)(max_num_seqs * num_blocks));
    c->owned_count = (int64_t*)calloc((size_t)max_num_seqs, sizeof(int64_t));
    c->page_table = (int32_t*)malloc(sizeof(int32_t) * (size_t)(max_num_seqs * num_blocks));
    for (int64_t i = 0; i < max_num_seqs * num_blocks; ++i) c->page_table[i] = -1;
    c->revision = 1;
    c->synced_revision = 1;
    return c;
}

void oracle_pkv_destroy(oracle_paged_kv* c) {
    if (c == NULL) return;
    oracle_bm_destroy(c->blocks);
    free(c->seq_len);
    free(c->owned);
    free(c->owned_count);
    free(c->page_table);
    free(c);
}

/* paged_kv_cache.cpp:52-142 */
int oracle_pkv_append(oracle_paged_kv* c, int64_t seq, int64_t layer, int64_t num_tokens,
                      int32_t* slots, char* msg, size_t msg_len) {
    char buf[256];
    if (seq < 0 || seq >= c->max_num_seqs) {
        snprintf(buf, sizeof(buf), "PagedKVCache::AppendTokens seq_id=%lld out of range [0,%lld)",
                 (long long)seq, (long long)c->max_num_seqs);
        set_msg(msg, msg_len, buf);
        return kShapeMismatch;
    }
    if (layer < 0 || layer >= c->num_layers) {
        snprintf(buf, sizeof(buf), "PagedKVCache::AppendTokens layer=%lld out of range [0,%lld)",
                 (long long)layer, (long long)c->num_layers);
        set_msg(msg, msg_len, buf);
        return kShapeMismatch;
    }
    if (num_tokens <= 0) {
        set_msg(msg, msg_len, "PagedKVCache::AppendTokens: 0 tokens");
        return kShapeMismatch;
    }
    int32_t* owned = c->owned + seq * c->num_blocks;
    const int64_t current = c->seq_len[seq];
    const int64_t needed = (current + num_tokens + c->block_size - 1) / c->block_size;
    const int64_t to_allocate = needed - c->owned_count[seq];
    int32_t* fresh = NULL;
    if (to_allocate > 0) {
        fresh = (int32_t*)malloc(sizeof(int32_t) * (size_t)to_allocate);
        const int rc = oracle_bm_allocate(c->blocks, to_allocate, fresh, NULL, 0);
        if (rc != 0) {
            free(fresh);
            snprintf(buf, sizeof(buf),
                     "PagedKVCache::AppendTokens seq=%lld needs %lld more blocks but only %lld "
                     "are free",
                     (long long)seq, (long long)to_allocate,
                     (long long)oracle_bm_num_free(c->blocks));
            set_msg(msg, msg_len, buf);
            return kKVCapacityExceeded;
        }
        const int rc2 = oracle_bm_append_to_table(c->blocks, seq, fresh, to_allocate, msg, msg_len);
        if (rc2 != 0) {
            oracle_bm_free(c->blocks, fresh, to_allocate);
            free(fresh);
            return rc2;
        }
        for (int64_t i = 0; i < to_allocate; ++i) owned[c->owned_count[seq]++] = fresh[i];
        free(fresh);
    }
    int32_t* row = c->page_table + seq * c->num_blocks;
    for (int64_t i = 0; i < c->num_blocks; ++i) row[i] = -1;
    for (int64_t i = 0; i < c->owned_count[seq]; ++i) row[i] = owned[i];
    const int rc = oracle_compute_slot_mapping(row, current, num_tokens, c->block_size,
                                               c->num_blocks, slots, msg, msg_len);
    if (rc != 0) return rc;
    c->seq_len[seq] = current + num_tokens;
    ++c->revision;
    ++c->num_appends;
    return 0;
}

/* paged_kv_cache.cpp:144-168 */
int oracle_pkv_reset(oracle_paged_kv* c, int64_t seq, char* msg, size_t msg_len) {
    char buf[256];
    if (seq < 0 || seq >= c->max_num_seqs) {
        snprintf(buf, sizeof(buf), "PagedKVCache::ResetSeq seq_id=%lld out of range",
                 (long long)seq);
        set_msg(msg, msg_len, buf);
        return kShapeMismatch;
    }
    oracle_bm_reset_seq(c->blocks, seq, NULL, 0);
    c->owned_count[seq] = 0;
    c->seq_len[seq] = 0;
    int32_t* row = c->page_table + seq * c->num_blocks;
    for (int64_t i = 0; i < c->num_blocks; ++i) row[i] = -1;
    ++c->revision;
    ++c->num_resets;
    return 0;
}

/* paged_kv_cache.cpp:182-201 */
int oracle_pkv_sync(oracle_paged_kv* c) {
    if (c->revision == c->synced_revision) return 0;
    c->synced_revision = c->revision;
    return 1;
}

int64_t oracle_pkv_seq_len(const oracle_paged_kv* c, int64_t seq) {
    return (seq < 0 || seq >= c->max_num_seqs) ? 0 : c->seq_len[seq];
}

int64_t oracle_pkv_block_count(const oracle_paged_kv* c, int64_t seq) {
    return (seq < 0 || seq >= c->max_num_seqs) ? 0 : c->owned_count[seq];
}

void oracle_pkv_page_table(const oracle_paged_kv* c, int32_t* out) {
    memcpy(out, c->page_table, sizeof(int32_t) * (size_t)(c->max_num_seqs * c->num_blocks));
}

/* paged_kv_cache.cpp:203-211 */
void oracle_pkv_stats(const oracle_paged_kv* c, int64_t* out6) {
    const int64_t free_blocks = oracle_bm_num_free(c->blocks);
    out6[0] = c->num_blocks - free_blocks;
    out6[1] = free_blocks;
    out6[2] = c->num_appends;
    out6[3] = c->num_resets;
    out6[4] = (int64_t)c->revision;
    out6[5] = (int64_t)c->synced_revision;
}

const oracle_block_manager* oracle_pkv_blocks(const oracle_paged_kv* c) { return c->blocks; }

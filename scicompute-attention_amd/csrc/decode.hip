// Split-K decode (S_q = 1) over contiguous or paged KV, plus the log-sum-exp combine.
//
// Semantics follow the reference's decode kernels (src/backends/decode/decode_splitk.cu:66-182
// and src/backends/paged/page_table.cuh:18-36):
//   per (b, h_q, split s): tokens [s*chunk, min((s+1)*chunk, len)), chunk = ceil(len/splits);
//     m_s = max_j q.k_j*scale, l_s = sum_j exp(q.k_j*scale - m_s), O_s = sum_j exp(...) v_j
//   combine: m* = max m_s, l* = sum_{m_s>-inf} l_s e^{m_s-m*}, out = sum O_s e^{m_s-m*} / l*
//   (out = 0 when l* = 0); paged rows: page_table[b*max_blocks + j/bs]*bs + j%bs, with page ids
//   < 0 or >= num_kv_blocks contributing nothing; len = seq_lens[b] or seq_kv.
// The partial scratch layout is the reference's: m | l | O with flat index ((b*H_q)+h)*splits+s,
// m in natural-log units.
//
// MI355X design (HBM-bound kernels):
//   * fp16/bf16 with head_dim 64 or 128 (power-of-two page sizes when paged) run
//     decode_mfma_kernel: the query heads of a GQA group are the 16 columns of
//     v_mfma_f32_16x16x32 tiles, K goes straight into A-operand registers, V through a small LDS
//     ring read with transposed loads; ragged batches run longest sequence first. Described at
//     its definition;
//   * every other shape (fp32, other head dims) runs decode_partial_kernel: one workgroup per
//     (b, kv head, split) streams its K/V chunk exactly once and serves kHeads query heads of the
//     group from registers; a lane owns 16 B of one token row (8 fp16/bf16 elements), QK uses
//     v_dot2_f32_{f16,bf16} and a DPP row sum, the online softmax is updated once per chunk of
//     kChunk tokens per row group, and row groups and waves are merged in registers / LDS;
//   * splits == 1 writes the normalised output directly and skips the combine kernel, which
//     otherwise runs one thread per (b, h, 4 dims).

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <string>
#include <type_traits>

#include "sca_device.hpp"

namespace sca_hip {
namespace {

constexpr int kDecodeThreads = 256;
constexpr int kDecodeWaves = kDecodeThreads / kWave;
constexpr int kChunk = 4;          // tokens per row group per iteration
constexpr int kPageSegment = 2048; // page ids staged in LDS per segment

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));

// ---- element traits --------------------------------------------------------------------------
// VE elements per 16-byte lane vector; dot4() accumulates the 16-byte product q.k into acc.
struct DecF16 {
    static constexpr int VE = 8;
    static __device__ __forceinline__ float dot(const uint4& q, const uint4& k, float acc) {
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, q.x), __builtin_bit_cast(half2v, k.x),
                                     acc, false);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, q.y), __builtin_bit_cast(half2v, k.y),
                                     acc, false);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, q.z), __builtin_bit_cast(half2v, k.z),
                                     acc, false);
        acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, q.w), __builtin_bit_cast(half2v, k.w),
                                     acc, false);
        return acc;
    }
    static __device__ __forceinline__ void unpack(const uint4& raw, float* out) {
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = F16::to_float(static_cast<uint16_t>(w[i] & 0xffffu));
            out[2 * i + 1] = F16::to_float(static_cast<uint16_t>(w[i] >> 16));
        }
    }
    static __device__ __forceinline__ void store(void* dst, const float* v) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = static_cast<uint32_t>(F16::from_float(v[2 * i])) |
                   (static_cast<uint32_t>(F16::from_float(v[2 * i + 1])) << 16);
        }
        *static_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    static __device__ __forceinline__ void store1(uint8_t* row, int d, float v) {
        reinterpret_cast<uint16_t*>(row)[d] = F16::from_float(v);
    }
};

struct DecBF16 {
    static constexpr int VE = 8;
    static __device__ __forceinline__ float dot(const uint4& q, const uint4& k, float acc) {
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, q.x),
                                              __builtin_bit_cast(bf16x2v, k.x), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, q.y),
                                              __builtin_bit_cast(bf16x2v, k.y), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, q.z),
                                              __builtin_bit_cast(bf16x2v, k.z), acc, false);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2v, q.w),
                                              __builtin_bit_cast(bf16x2v, k.w), acc, false);
        return acc;
    }
    static __device__ __forceinline__ void unpack(const uint4& raw, float* out) {
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = __builtin_bit_cast(float, w[i] << 16);
            out[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
        }
    }
    static __device__ __forceinline__ void store(void* dst, const float* v) {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = static_cast<uint32_t>(BF16::from_float(v[2 * i])) |
                   (static_cast<uint32_t>(BF16::from_float(v[2 * i + 1])) << 16);
        }
        *static_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    static __device__ __forceinline__ void store1(uint8_t* row, int d, float v) {
        reinterpret_cast<uint16_t*>(row)[d] = BF16::from_float(v);
    }
};

struct DecF32 {
    static constexpr int VE = 4;
    static __device__ __forceinline__ float dot(const uint4& q, const uint4& k, float acc) {
        acc = fmaf(__builtin_bit_cast(float, q.x), __builtin_bit_cast(float, k.x), acc);
        acc = fmaf(__builtin_bit_cast(float, q.y), __builtin_bit_cast(float, k.y), acc);
        acc = fmaf(__builtin_bit_cast(float, q.z), __builtin_bit_cast(float, k.z), acc);
        acc = fmaf(__builtin_bit_cast(float, q.w), __builtin_bit_cast(float, k.w), acc);
        return acc;
    }
    static __device__ __forceinline__ void unpack(const uint4& raw, float* out) {
        out[0] = __builtin_bit_cast(float, raw.x);
        out[1] = __builtin_bit_cast(float, raw.y);
        out[2] = __builtin_bit_cast(float, raw.z);
        out[3] = __builtin_bit_cast(float, raw.w);
    }
    static __device__ __forceinline__ void store(void* dst, const float* v) {
        *static_cast<uint4*>(dst) =
            make_uint4(__builtin_bit_cast(uint32_t, v[0]), __builtin_bit_cast(uint32_t, v[1]),
                       __builtin_bit_cast(uint32_t, v[2]), __builtin_bit_cast(uint32_t, v[3]));
    }
    static __device__ __forceinline__ void store1(uint8_t* row, int d, float v) {
        reinterpret_cast<float*>(row)[d] = v;
    }
};

constexpr int Pow2Ceil(int x) {
    int p = 1;
    while (p < x) p *= 2;
    return p;
}

// Sum over the LPR lanes of one row group (LPR is a power of two <= 64). Offsets below 16 use
// DPP (quad permutes and the two row mirrors); 16 and 32 use a cross-row shuffle.
template <int LPR>
__device__ __forceinline__ float RowGroupSum(float x) {
    if constexpr (LPR >= 2) {
        x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                           0, __builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, false));
    }
    if constexpr (LPR >= 4) {
        x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                           0, __builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, false));
    }
    if constexpr (LPR >= 8) {
        x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                           0, __builtin_bit_cast(int, x), 0x141, 0xF, 0xF, false));
    }
    if constexpr (LPR >= 16) {
        x += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                           0, __builtin_bit_cast(int, x), 0x140, 0xF, 0xF, false));
    }
    if constexpr (LPR >= 32) x += __shfl_xor(x, 16);
    if constexpr (LPR >= 64) x += __shfl_xor(x, 32);
    return x;
}

// Merges (m, l) of this lane with the state held `off` lanes away; returns the two weights.
__device__ __forceinline__ void MergeWeights(float m_a, float m_b, float* m_out, float* w_a,
                                             float* w_b) {
    const float mm = fmaxf(m_a, m_b);
    *m_out = mm;
    if (mm == neg_inf()) {
        *w_a = 0.0f;
        *w_b = 0.0f;
        return;
    }
    *w_a = (m_a == neg_inf()) ? 0.0f : fast_exp2(m_a - mm);
    *w_b = (m_b == neg_inf()) ? 0.0f : fast_exp2(m_b - mm);
}

template <typename E, int D, int kHeads, bool kPaged>
__global__ __launch_bounds__(kDecodeThreads) void decode_partial_kernel(const sca_decode_params p,
                                                                        int h_chunks) {
    constexpr int VE = E::VE;
    constexpr int NV = D / VE;           // active lanes per row
    constexpr int LPR = Pow2Ceil(NV);    // lanes per row group
    constexpr int RPW = kWave / LPR;     // row groups per wave
    constexpr int RG = kDecodeWaves * RPW;
    static_assert(LPR <= kWave, "head_dim too large for one wave row");

    __shared__ int32_t s_pages[kPaged ? kPageSegment : 1];
    __shared__ float s_m[kDecodeWaves][kHeads];
    __shared__ float s_l[kDecodeWaves][kHeads];
    __shared__ float s_o[kDecodeWaves][kHeads][D];

    const int lane = threadIdx.x % kWave;
    const int wave = threadIdx.x / kWave;
    const int sub = lane % LPR;
    const int rg = wave * RPW + lane / LPR;
    const bool active = sub < NV;

    const int64_t split = blockIdx.x;
    const int64_t h_kv = blockIdx.y / h_chunks;
    const int64_t h_chunk = blockIdx.y % h_chunks;
    const int64_t b = blockIdx.z;
    const int64_t group = p.num_heads / p.num_kv_heads;
    const int64_t h0 = h_kv * group + h_chunk * kHeads;  // first q head of this workgroup

    const float scale2 = p.scale * kLog2e;

    // Query vectors of the kHeads heads, raw 16-byte lane slices.
    uint4 qv[kHeads];
#pragma unroll
    for (int h = 0; h < kHeads; ++h) {
        const uint8_t* q_row = static_cast<const uint8_t*>(p.q) +
                               (b * p.q_sb + (h0 + h) * p.q_sh) * (16 / VE);
        qv[h] = active ? *reinterpret_cast<const uint4*>(q_row + sub * 16) : make_uint4(0, 0, 0, 0);
    }

    float acc[kHeads][VE];
    float m[kHeads], l[kHeads];
#pragma unroll
    for (int h = 0; h < kHeads; ++h) {
        m[h] = neg_inf();
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[h][e] = 0.0f;
    }

    const int64_t len = p.seq_lens != nullptr ? static_cast<int64_t>(p.seq_lens[b]) : p.seq_kv;
    const int64_t chunk = len > 0 ? (len + p.num_splits - 1) / p.num_splits : 0;
    const int64_t t_begin = split * chunk;
    const int64_t t_end = (t_begin + chunk < len) ? (t_begin + chunk) : len;

    constexpr int64_t kElemBytes = 16 / VE;
    const uint8_t* k_base = static_cast<const uint8_t*>(p.k) +
                            ((kPaged ? 0 : b * p.k_sb) + h_kv * p.k_sh) * kElemBytes + sub * 16;
    const uint8_t* v_base = static_cast<const uint8_t*>(p.v) +
                            ((kPaged ? 0 : b * p.v_sb) + h_kv * p.v_sh) * kElemBytes + sub * 16;
    const int64_t k_row_bytes = p.k_ss * kElemBytes;
    const int64_t v_row_bytes = p.v_ss * kElemBytes;

    // Segment loop (one segment for contiguous KV; page-table segments staged in LDS otherwise).
    // A paged segment ends on a page boundary, so it never spans more than kPageSegment pages
    // whatever page offset the split starts at.
    int64_t seg_end = t_begin;
    for (int64_t seg = t_begin; seg < t_end; seg = seg_end) {
        int64_t page0 = 0;
        if constexpr (kPaged) {
            page0 = seg / p.block_size;
            const int64_t cap = (page0 + kPageSegment) * p.block_size;
            seg_end = cap < t_end ? cap : t_end;
            const int64_t page_last = (seg_end - 1) / p.block_size;
            const int64_t n_pages = page_last - page0 + 1;
            __syncthreads();
            for (int64_t i = threadIdx.x; i < n_pages; i += kDecodeThreads) {
                const int64_t logical = page0 + i;
                int32_t id = -1;
                if (logical < p.max_blocks_per_seq) {
                    id = p.page_table[b * p.max_blocks_per_seq + logical];
                    if (id < 0 || id >= p.num_kv_blocks) id = -1;
                }
                s_pages[i] = id;
            }
            __syncthreads();
        } else {
            seg_end = t_end;
        }

        for (int64_t base = seg; base < seg_end; base += RG * kChunk) {
            uint4 kr[kChunk], vr[kChunk];
            bool valid[kChunk];
#pragma unroll
            for (int c = 0; c < kChunk; ++c) {
                const int64_t tok = base + c * RG + rg;
                bool ok = tok < seg_end;
                int64_t row = tok;
                if constexpr (kPaged) {
                    if (ok) {
                        const int32_t id = s_pages[tok / p.block_size - page0];
                        ok = id >= 0;
                        row = static_cast<int64_t>(id) * p.block_size + tok % p.block_size;
                    }
                }
                valid[c] = ok;
                if (ok && active) {
                    kr[c] = *reinterpret_cast<const uint4*>(k_base + row * k_row_bytes);
                    vr[c] = *reinterpret_cast<const uint4*>(v_base + row * v_row_bytes);
                } else {
                    kr[c] = make_uint4(0, 0, 0, 0);
                    vr[c] = make_uint4(0, 0, 0, 0);
                }
            }

            float s[kChunk][kHeads];
#pragma unroll
            for (int c = 0; c < kChunk; ++c) {
#pragma unroll
                for (int h = 0; h < kHeads; ++h) {
                    const float part = E::dot(qv[h], kr[c], 0.0f);
                    const float dot = RowGroupSum<LPR>(part);
                    s[c][h] = valid[c] ? dot * scale2 : neg_inf();
                }
            }

            float vf[kChunk][VE];
#pragma unroll
            for (int c = 0; c < kChunk; ++c) E::unpack(vr[c], vf[c]);

#pragma unroll
            for (int h = 0; h < kHeads; ++h) {
                float mc = s[0][h];
#pragma unroll
                for (int c = 1; c < kChunk; ++c) mc = fmaxf(mc, s[c][h]);
                const float m_new = fmaxf(m[h], mc);
                if (m_new == neg_inf()) continue;  // nothing visible yet for this row group
                const float alpha = (m[h] == neg_inf()) ? 0.0f : fast_exp2(m[h] - m_new);
                m[h] = m_new;
                l[h] *= alpha;
#pragma unroll
                for (int e = 0; e < VE; ++e) acc[h][e] *= alpha;
#pragma unroll
                for (int c = 0; c < kChunk; ++c) {
                    const float pc = fast_exp2(s[c][h] - m_new);
                    l[h] += pc;
#pragma unroll
                    for (int e = 0; e < VE; ++e) acc[h][e] = fmaf(pc, vf[c][e], acc[h][e]);
                }
            }
        }
    }

    // Merge the row groups of this wave (lanes LPR, 2*LPR, ... apart hold the same d slice).
#pragma unroll
    for (int off = LPR; off < kWave; off *= 2) {
#pragma unroll
        for (int h = 0; h < kHeads; ++h) {
            const float m_o = __shfl_xor(m[h], off);
            const float l_o = __shfl_xor(l[h], off);
            float mm, wa, wb;
            MergeWeights(m[h], m_o, &mm, &wa, &wb);
            m[h] = mm;
            l[h] = l[h] * wa + l_o * wb;
#pragma unroll
            for (int e = 0; e < VE; ++e) {
                const float o_o = __shfl_xor(acc[h][e], off);
                acc[h][e] = acc[h][e] * wa + o_o * wb;
            }
        }
    }

    // Merge the waves through LDS.
    if (lane < LPR && active) {
#pragma unroll
        for (int h = 0; h < kHeads; ++h) {
#pragma unroll
            for (int e = 0; e < VE; ++e) s_o[wave][h][sub * VE + e] = acc[h][e];
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int h = 0; h < kHeads; ++h) {
            s_m[wave][h] = m[h];
            s_l[wave][h] = l[h];
        }
    }
    __syncthreads();

    const bool direct = p.num_splits == 1;
    for (int idx = threadIdx.x; idx < kHeads * D; idx += kDecodeThreads) {
        const int h = idx / D;
        const int d = idx % D;
        float mm = neg_inf();
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) mm = fmaxf(mm, s_m[w][h]);
        float lsum = 0.0f, osum = 0.0f;
        if (mm != neg_inf()) {
#pragma unroll
            for (int w = 0; w < kDecodeWaves; ++w) {
                const float mw = s_m[w][h];
                if (mw == neg_inf()) continue;
                const float wgt = fast_exp2(mw - mm);
                lsum += s_l[w][h] * wgt;
                osum += s_o[w][h][d] * wgt;
            }
        }
        const int64_t hq = h0 + h;
        if (direct) {
            const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
            // Scalar store of one element; the output row is tiny next to the KV stream.
            uint8_t* out_row = static_cast<uint8_t*>(p.out) + (b * p.o_sb + hq * p.o_sh) * kElemBytes;
            E::store1(out_row, d, osum * inv);
        } else {
            const int64_t flat = (b * p.num_heads + hq) * p.num_splits + split;
            p.partial_o[flat * D + d] = osum;
            if (d == 0) {
                p.partial_m[flat] = (mm == neg_inf()) ? neg_inf() : mm * kLn2;
                p.partial_l[flat] = lsum;
            }
        }
    }
}

// Split merge (reference decode_splitk.cu:143-182): out = sum_s O_s e^{m_s - m*} / sum_s l_s e^{m_s - m*},
// with m* = max_s m_s, splits with m_s = -inf skipped and out = 0 when the denominator is 0.
// One thread per (b, h_q, 4 consecutive d): the split loads of a thread are independent, so
// they overlap instead of forming a chain, and neighbouring threads read neighbouring bytes.
constexpr int kCombineThreads = 256;

template <typename E, int D>
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(const sca_decode_params p) {
    constexpr int64_t kElemBytes = 16 / E::VE;
    constexpr int kQuads = D / 4;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kCombineThreads + threadIdx.x;
    const int64_t flat_bh = idx / kQuads;
    if (flat_bh >= p.batch * p.num_heads) return;
    const int d0 = static_cast<int>(idx % kQuads) * 4;
    const int64_t b = flat_bh / p.num_heads;
    const int64_t h = flat_bh % p.num_heads;
    const int ns = static_cast<int>(p.num_splits);
    const float* pm = p.partial_m + flat_bh * ns;
    const float* pl = p.partial_l + flat_bh * ns;
    const float* po = p.partial_o + flat_bh * ns * D + d0;

    float m_all = neg_inf();
#pragma unroll 8
    for (int s = 0; s < ns; ++s) m_all = fmaxf(m_all, pm[s]);
    float l_all = 0.0f;
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll 4
    for (int s = 0; s < ns; ++s) {
        const float ms = pm[s];
        const float w = (ms == neg_inf()) ? 0.0f : fast_exp2((ms - m_all) * kLog2e);
        l_all = fmaf(pl[s], w, l_all);
        const float* o = po + static_cast<int64_t>(s) * D;
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = fmaf(o[i], w, acc[i]);
    }
    const float inv = l_all > 0.0f ? 1.0f / l_all : 0.0f;
    uint8_t* out_row = static_cast<uint8_t*>(p.out) + (b * p.o_sb + h * p.o_sh) * kElemBytes;
#pragma unroll
    for (int i = 0; i < 4; ++i) E::store1(out_row, d0 + i, acc[i] * inv);
}

constexpr int kRankBatch = 256;  // ragged batches up to this size are ranked in the kernel

// ---- MFMA partial kernel (fp16/bf16, head_dim 64 or 128, power-of-two pages) -----------------
// One workgroup per (b, kv head, 16-head chunk of its q group, split); four waves take the
// 32-token tiles of the split in turn and are merged through LDS at the end.
//   S^T[32 tokens x 16 heads] = K . Q^T on v_mfma_f32_16x16x32 (two 16-token row tiles; the
//     q heads of the group fill the 16 columns, unused columns hold zero queries);
//   O^T[D x 16 heads] += V^T . P^T, one MFMA per 16 dims with the 32 tokens as the k dimension.
// Lane layout: lane l owns query head l % 16; its S^T values are tokens 16r + 4(l/16) + i.
// The PV k index 8g + i (g = l/16) maps to token 4g + i for i < 4 and 16 + 4g + (i - 4) after,
// which is exactly the register order of the two S^T tiles, so P^T needs no data movement.
// The head dimension is permuted identically for K and Q: k step j, lane group g covers
// elements (4j + g)*8 .. +8, so K goes straight from global memory into the A-operand
// registers as 64-byte row blocks. V goes global -> LDS with global_load_lds_dwordx4 into a
// two-stage ring per wave (one LDS object per stage, so the compiler's LDS-DMA tracking waits
// only for the stage being read); V rows XOR their 32-byte segments so the transposed reads
// hit distinct banks. A wave always has the next tile in flight while it computes, and the
// 64 KB ring lets two workgroups share a CU. The probabilities are rounded to fp16/bf16 for the
// PV MFMA (the reference's decode kernel keeps them in fp32; the denominator here sums the
// unrounded values), which stays inside the parity tolerance.
constexpr int kMfmaTile = 32;   // tokens per wave iteration
constexpr int kMfmaHeads = 16;  // query heads per workgroup (MFMA N)

template <typename E>
struct DecMfma;

template <>
struct DecMfma<DecF16> {
    using vec8 = half8;
    using Tr = TrRead<F16>;
    typedef _Float16 pair_t __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ floatx4 mma(const vec8& a, const vec8& b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack(float a, float b) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, pair_t));
    }
};

template <>
struct DecMfma<DecBF16> {
    using vec8 = bf16x8;
    using Tr = TrRead<BF16>;
    typedef __bf16 pair_t __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ floatx4 mma(const vec8& a, const vec8& b, floatx4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack(float a, float b) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, pair_t));
    }
};

template <int D>
struct MfmaDecGeom {
    static_assert(D == 64 || D == 128, "MFMA decode covers head_dim 64 and 128");
    static constexpr int NK = D / 32;                    // QK k steps
    static constexpr int ND = D / 16;                    // PV output tiles
    static constexpr int RB = 2 * D;                     // row bytes
    static constexpr int CPR = D / 8;                    // 16-byte chunks per row
    static constexpr int TILE_BYTES = kMfmaTile * RB;    // one V tile of one wave
    static constexpr int DMA = TILE_BYTES / 1024;        // DMA instructions per V tile
    static constexpr int ROWS_PER_DMA = 64 / CPR;
    static constexpr int SLOT_BYTES = kDecodeWaves * TILE_BYTES;  // one LDS object
    static constexpr int LOADS = DMA + 2 * NK;           // vector memory instructions per tile
    static_assert(kDecodeWaves * kMfmaHeads * D * 4 <= SLOT_BYTES, "merge buffer fits one slot");
};

// 32-byte segment swizzle of V row t (rows t and t + 16 share it, which the two transposed
// reads of a lane rely on).
template <int D>
__device__ __forceinline__ int VSwz(int t) {
    return D == 128 ? (t & 7) : ((t >> 1) & 3);
}

// kWaveHeads: each wave owns one (kv head, head chunk) slot and all tiles of the split (the
// four waves read neighbouring head slices of the same token rows); otherwise the four waves
// share the tiles of one head slot and are merged through LDS.
template <typename E, int D, bool kPaged, bool kWaveHeads>
__global__ __launch_bounds__(kDecodeThreads) void decode_mfma_kernel(const sca_decode_params p,
                                                                     int h_chunks,
                                                                     int block_shift) {
    using G = MfmaDecGeom<D>;
    using M = DecMfma<E>;
    using vec8 = typename M::vec8;

    __shared__ __align__(16) uint8_t s_v0[G::SLOT_BYTES];
    __shared__ __align__(16) uint8_t s_v1[G::SLOT_BYTES];
    // Page ids of the current segment; first the lengths of a ragged batch being ranked.
    __shared__ int32_t s_pages[kPaged ? kPageSegment : kRankBatch];
    __shared__ int32_t s_seq[2];
    __shared__ float s_m[kDecodeWaves][kMfmaHeads];
    __shared__ float s_l[kDecodeWaves][kMfmaHeads];

    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int col = lane % 16;  // query head within the chunk; row/column index of the MFMA
    const int grp = lane / 16;  // lane group

    const int64_t split = blockIdx.x;
    const int64_t slots = p.num_kv_heads * h_chunks;
    const int64_t hh = kWaveHeads ? static_cast<int64_t>(blockIdx.y) * kDecodeWaves + wave
                                  : static_cast<int64_t>(blockIdx.y);
    const bool slot_ok = hh < slots;  // false only for trailing waves of a kWaveHeads grid
    const int64_t h_kv = (slot_ok ? hh : 0) / h_chunks;
    const int64_t h_chunk = (slot_ok ? hh : 0) % h_chunks;
    // Sequence of this workgroup. Ragged batches run longest first: grid row z takes the
    // sequence of rank z (descending length, ties by index), ranked here for batches of up to
    // kRankBatch sequences and by decode_order_kernel through batch_order above that.
    int64_t b = blockIdx.z;
    int64_t len = p.seq_kv;
    if (p.seq_lens != nullptr && p.batch <= kRankBatch) {
        const int tid = threadIdx.x;
        const int nb = static_cast<int>(p.batch);
        if (tid < nb) s_pages[tid] = p.seq_lens[tid];
        __syncthreads();
        if (tid < nb) {
            const int mine = s_pages[tid];
            int rank = 0;
            for (int j = 0; j < nb; ++j) {
                const int other = s_pages[j];
                rank += (other > mine) | ((other == mine) & (j < tid));
            }
            if (rank == static_cast<int>(blockIdx.z)) {
                s_seq[0] = tid;
                s_seq[1] = mine;
            }
        }
        __syncthreads();
        b = __builtin_amdgcn_readfirstlane(s_seq[0]);
        len = __builtin_amdgcn_readfirstlane(s_seq[1]);
    } else if (p.batch_order != nullptr) {
        const int2 e = reinterpret_cast<const int2*>(p.batch_order)[blockIdx.z];
        b = e.x;
        len = e.y;
    } else if (p.seq_lens != nullptr) {
        len = p.seq_lens[b];
    }
    const int64_t group = p.num_heads / p.num_kv_heads;
    const int64_t h0 = h_kv * group + h_chunk * kMfmaHeads;
    const int hc = static_cast<int>(group - h_chunk * kMfmaHeads < kMfmaHeads
                                        ? group - h_chunk * kMfmaHeads
                                        : kMfmaHeads);
    const float scale2 = p.scale * kLog2e;
    const int64_t bs_mask = (int64_t{1} << block_shift) - 1;

    // Q^T B operand: lane (col, grp) holds head col, elements (4j + grp)*8 .. +8 for k step j.
    vec8 qb[G::NK];
    {
        const uint8_t* q_row =
            static_cast<const uint8_t*>(p.q) + (b * p.q_sb + (h0 + col) * p.q_sh) * 2;
#pragma unroll
        for (int j = 0; j < G::NK; ++j) {
            const uint4 raw = col < hc ? *reinterpret_cast<const uint4*>(q_row + (4 * j + grp) * 16)
                                       : make_uint4(0, 0, 0, 0);
            qb[j] = __builtin_bit_cast(vec8, raw);
        }
    }

    floatx4 o[G::ND];
#pragma unroll
    for (int dt = 0; dt < G::ND; ++dt) o[dt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    float m = neg_inf();  // running max of head `col` (log2 units, identical across lane groups)
    float l = 0.0f;       // this lane's share of the running denominator

    const int64_t chunk = len > 0 ? (len + p.num_splits - 1) / p.num_splits : 0;
    const int64_t t_begin = split * chunk;
    const int64_t t_end = (t_begin + chunk < len) ? (t_begin + chunk) : len;

    const uint8_t* k_base =
        static_cast<const uint8_t*>(p.k) + ((kPaged ? 0 : b * p.k_sb) + h_kv * p.k_sh) * 2;
    const uint8_t* v_base =
        static_cast<const uint8_t*>(p.v) + ((kPaged ? 0 : b * p.v_sb) + h_kv * p.v_sh) * 2;
    const int64_t k_row_bytes = p.k_ss * 2;
    const int64_t v_row_bytes = p.v_ss * 2;

    // Per-lane constants: DMA row/chunk within one instruction and the V transposed read
    // (row 4*grp + col/4, byte 8*(col%4) of a 32-byte segment).
    const int dma_row = lane / G::CPR;
    const int dma_pc = lane % G::CPR;
    const int wave_off = wave * G::TILE_BYTES;
    const int tr_row = 4 * grp + col / 4;
    const int tr_rd = wave_off + tr_row * G::RB + 8 * (col % 4);
    const int tr_x = VSwz<D>(tr_row) * 32;

    // A paged segment ends on a page boundary, so it never spans more than kPageSegment pages
    // whatever page offset the split starts at.
    int64_t seg_end = t_begin;
    for (int64_t seg = t_begin; seg < t_end; seg = seg_end) {
        int64_t page0 = 0;
        seg_end = t_end;
        if constexpr (kPaged) {
            page0 = seg >> block_shift;
            const int64_t cap = (page0 + kPageSegment) << block_shift;
            seg_end = cap < t_end ? cap : t_end;
            const int64_t n_pages = ((seg_end - 1) >> block_shift) - page0 + 1;
            __syncthreads();
            for (int64_t i = threadIdx.x; i < n_pages; i += kDecodeThreads) {
                const int64_t logical = page0 + i;
                int32_t id = -1;
                if (logical < p.max_blocks_per_seq) {
                    id = p.page_table[b * p.max_blocks_per_seq + logical];
                    if (id < 0 || id >= p.num_kv_blocks) id = -1;
                }
                s_pages[i] = id;
            }
            __syncthreads();
        }
        // Row index of token tok (< 0: the token contributes nothing); branch-free.
        auto row_of = [&](int64_t tok) -> int64_t {
            const bool in = tok < seg_end;
            if constexpr (kPaged) {
                const int rel = static_cast<int>((in ? tok : seg) - (page0 << block_shift));
                const int32_t id = s_pages[rel >> block_shift];
                const int64_t r = (static_cast<int64_t>(id) << block_shift) | (rel & bs_mask);
                return (in && id >= 0) ? r : -1;
            } else {
                return in ? tok : -1;
            }
        };
        // Masked tokens read a row that is always mapped (row 0 of the pool, or the segment's
        // first token); their scores are set to -inf and their V rows cleared before use.
        const int64_t safe_row = kPaged ? 0 : seg;

        const int n_tiles =
            slot_ok ? static_cast<int>((seg_end - seg + kMfmaTile - 1) / kMfmaTile) : 0;
        constexpr int TS = kWaveHeads ? 1 : kDecodeWaves;  // tile stride of one wave
        // V tile -> LDS stage, then the K tile -> registers (row col of each row tile).
        auto issue = [&](int tile, uint8_t* vdst, uint4 (&kr)[2][G::NK]) {
            const int64_t base = seg + static_cast<int64_t>(tile) * kMfmaTile;
#pragma unroll
            for (int i = 0; i < G::DMA; ++i) {
                const int t = i * G::ROWS_PER_DMA + dma_row;
                int64_t r = row_of(base + t);
                r = r < 0 ? safe_row : r;
                const int vc = (((dma_pc >> 1) ^ VSwz<D>(t)) << 1) | (dma_pc & 1);
                __builtin_amdgcn_global_load_lds(
                    v_base + r * v_row_bytes + vc * 16,
                    (__attribute__((address_space(3))) void*)(vdst + wave_off + i * 1024), 16, 0, 0);
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                int64_t r = row_of(base + 16 * rt + col);
                r = r < 0 ? safe_row : r;
                const uint8_t* src = k_base + r * k_row_bytes + grp * 16;
#pragma unroll
                for (int j = 0; j < G::NK; ++j) kr[rt][j] = *reinterpret_cast<const uint4*>(src + j * 64);
            }
        };
        auto compute = [&](int tile, const uint4 (&kr)[2][G::NK], uint8_t* vs) {
            const int64_t base = seg + static_cast<int64_t>(tile) * kMfmaTile;
            // Token validity of the tile: bit t for token t.
            const uint64_t b0 = __builtin_amdgcn_ballot_w64(row_of(base + col) >= 0);
            const uint64_t b1 = __builtin_amdgcn_ballot_w64(row_of(base + 16 + col) >= 0);
            const uint32_t valid_mask = static_cast<uint32_t>(b0 & 0xffffu) |
                                        (static_cast<uint32_t>(b1 & 0xffffu) << 16);
            // S^T = K . Q^T for the two 16-token row tiles.
            floatx4 s[2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
                s[rt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < G::NK; ++j) {
                    s[rt] = M::mma(__builtin_bit_cast(vec8, kr[rt][j]), qb[j], s[rt]);
                }
            }
            float sv[2][4];
            float mx = neg_inf();
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = 16 * rt + 4 * grp + i;
                    const float x = ((valid_mask >> t) & 1u) ? s[rt][i] * scale2 : neg_inf();
                    sv[rt][i] = x;
                    mx = fmaxf(mx, x);
                }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16));
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float m_new = fmaxf(m, mx);
            if (__builtin_amdgcn_ballot_w64(m_new > m) != 0) {
                const float alpha = (m == neg_inf()) ? 0.0f : fast_exp2(m - m_new);
                l *= alpha;
#pragma unroll
                for (int dt = 0; dt < G::ND; ++dt) o[dt] *= alpha;
                m = m_new;
            }
            const float m_use = (m == neg_inf()) ? 0.0f : m;
            float pr[2][4];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    pr[rt][i] = fast_exp2(sv[rt][i] - m_use);
                    l += pr[rt][i];
                }
            }
            const vec8 pb = __builtin_bit_cast(
                vec8, make_uint4(M::pack(pr[0][0], pr[0][1]), M::pack(pr[0][2], pr[0][3]),
                                 M::pack(pr[1][0], pr[1][1]), M::pack(pr[1][2], pr[1][3])));
            if (valid_mask != 0xffffffffu) {
                // Clear the V rows of masked tokens: their probabilities are zero, but the rows
                // may hold any bit pattern.
                constexpr int kLanesPerRow = kWave / kMfmaTile;
                constexpr int kChunksPerLane = G::CPR / kLanesPerRow;
                const int t = lane / kLanesPerRow;
                if (((valid_mask >> t) & 1u) == 0) {
                    uint4* rowp = reinterpret_cast<uint4*>(vs + wave_off + t * G::RB) +
                                  (lane % kLanesPerRow) * kChunksPerLane;
#pragma unroll
                    for (int c = 0; c < kChunksPerLane; ++c) rowp[c] = make_uint4(0, 0, 0, 0);
                }
            }
#pragma unroll
            for (int dt = 0; dt < G::ND; ++dt) {
                const uint8_t* a = vs + tr_rd + ((dt * 32) ^ tr_x);
                const uint2 lo = M::Tr::read(a);
                const uint2 hi = M::Tr::read(a + 16 * G::RB);
                o[dt] = M::mma(__builtin_bit_cast(vec8, make_uint4(lo.x, lo.y, hi.x, hi.y)), pb,
                               o[dt]);
            }
        };

        // Tiles wave, wave + 4, ...: stage 0 holds the even ones of this wave, stage 1 the odd.
        uint4 k0[2][G::NK], k1[2][G::NK];
        int tile = kWaveHeads ? 0 : wave;
        if (tile < n_tiles) issue(tile, s_v0, k0);
        if (tile + TS < n_tiles) issue(tile + TS, s_v1, k1);
        while (tile < n_tiles) {
            if (tile + TS < n_tiles) {
                WaitVm<G::LOADS>();
            } else {
                WaitVm<0>();
            }
            compute(tile, k0, s_v0);
            if (tile + 2 * TS < n_tiles) issue(tile + 2 * TS, s_v0, k0);
            tile += TS;
            if (tile >= n_tiles) break;
            if (tile + TS < n_tiles) {
                WaitVm<G::LOADS>();
            } else {
                WaitVm<0>();
            }
            compute(tile, k1, s_v1);
            if (tile + 2 * TS < n_tiles) issue(tile + 2 * TS, s_v1, k1);
            tile += TS;
        }
    }

    // Lane totals of l over the four lane groups.
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const bool direct = p.num_splits == 1;
    if constexpr (kWaveHeads) {
        // This wave holds the whole state of its head slot: lane (col, grp) has dims
        // dt*16 + 4*grp + i of head h0 + col.
        if (!slot_ok || col >= hc) return;
        const int64_t hq = h0 + col;
        if (direct) {
            const float inv = l > 0.0f ? 1.0f / l : 0.0f;
            uint8_t* out_row = static_cast<uint8_t*>(p.out) + (b * p.o_sb + hq * p.o_sh) * 2;
#pragma unroll
            for (int dt = 0; dt < G::ND; ++dt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) E::store1(out_row, dt * 16 + 4 * grp + i, o[dt][i] * inv);
            }
        } else {
            const int64_t flat = (b * p.num_heads + hq) * p.num_splits + split;
#pragma unroll
            for (int dt = 0; dt < G::ND; ++dt) {
                *reinterpret_cast<floatx4*>(p.partial_o + flat * D + dt * 16 + 4 * grp) = o[dt];
            }
            if (grp == 0) {
                p.partial_m[flat] = (m == neg_inf()) ? neg_inf() : m * kLn2;
                p.partial_l[flat] = l;
            }
        }
        return;
    }
    // Wave states to LDS, then one thread per (head, dim) merges the four waves.
    __syncthreads();  // every wave is done with its stages
    float* s_o = reinterpret_cast<float*>(s_v0);  // [wave][head][D]
#pragma unroll
    for (int dt = 0; dt < G::ND; ++dt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s_o[(wave * kMfmaHeads + col) * D + dt * 16 + 4 * grp + i] = o[dt][i];
        }
    }
    if (grp == 0) {
        s_m[wave][col] = m;
        s_l[wave][col] = l;
    }
    __syncthreads();

    for (int idx = threadIdx.x; idx < hc * D; idx += kDecodeThreads) {
        const int h = idx / D;
        const int d = idx % D;
        float mm = neg_inf();
#pragma unroll
        for (int w = 0; w < kDecodeWaves; ++w) mm = fmaxf(mm, s_m[w][h]);
        float lsum = 0.0f, osum = 0.0f;
        if (mm != neg_inf()) {
#pragma unroll
            for (int w = 0; w < kDecodeWaves; ++w) {
                const float mw = s_m[w][h];
                const float wgt = mw == neg_inf() ? 0.0f : fast_exp2(mw - mm);
                lsum += s_l[w][h] * wgt;
                osum += s_o[(w * kMfmaHeads + h) * D + d] * wgt;
            }
        }
        const int64_t hq = h0 + h;
        if (direct) {
            const float inv = lsum > 0.0f ? 1.0f / lsum : 0.0f;
            uint8_t* out_row = static_cast<uint8_t*>(p.out) + (b * p.o_sb + hq * p.o_sh) * 2;
            E::store1(out_row, d, osum * inv);
        } else {
            const int64_t flat = (b * p.num_heads + hq) * p.num_splits + split;
            p.partial_o[flat * D + d] = osum;
            if (d == 0) {
                p.partial_m[flat] = (mm == neg_inf()) ? neg_inf() : mm * kLn2;
                p.partial_l[flat] = lsum;
            }
        }
    }
}

template <typename E, int D, int kHeads, bool kPaged>
int LaunchPartial(const sca_decode_params& p, int h_chunks, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(p.num_splits),
                    static_cast<unsigned>(p.num_kv_heads * h_chunks),
                    static_cast<unsigned>(p.batch));
    hipLaunchKernelGGL((decode_partial_kernel<E, D, kHeads, kPaged>), grid, dim3(kDecodeThreads),
                       0, s, p, h_chunks);
    return CheckLaunch("decode_partial_kernel", s);
}

// Longest-first schedule of ragged batches larger than kRankBatch: entry r of `order` is
// (b, len_b) for the sequence of rank r (descending length, ties by index). The MFMA kernels
// take the sequence of grid row z from entry z, so the longest sequences are dispatched first.
constexpr int kMaxOrderedBatch = 8192;

__global__ __launch_bounds__(256) void decode_order_kernel(const int32_t* seq_lens, int batch,
                                                           int32_t* order) {
    const int b = blockIdx.x * 256 + threadIdx.x;
    if (b >= batch) return;
    const int mine = seq_lens[b];
    int rank = 0;
    for (int j = 0; j < batch; ++j) {
        const int other = seq_lens[j];
        rank += (other > mine) | ((other == mine) & (j < b));
    }
    order[2 * rank] = b;
    order[2 * rank + 1] = mine;
}

// One wave per head slot (true) or four waves per slot (false): the caller's slot_waves when
// set, else one wave per slot for paged KV and four for contiguous KV.
bool MfmaWaveHeads(bool paged, int32_t slot_waves) {
    if (slot_waves == 1) return true;
    if (slot_waves == kDecodeWaves) return false;
    return paged;
}

template <typename E, int D, bool kPaged>
int LaunchForDim(const sca_decode_params& p, hipStream_t s) {
    const int64_t group = p.num_heads / p.num_kv_heads;
    int rc = 0;
    int block_shift = 0;
    if constexpr (kPaged) {
        while ((int64_t{1} << block_shift) < p.block_size) ++block_shift;
    }
    const bool mfma_ok = !std::is_same_v<E, DecF32> && (D == 64 || D == 128) &&
                         (!kPaged || (int64_t{1} << block_shift) == p.block_size);
    if constexpr (!std::is_same_v<E, DecF32> && (D == 64 || D == 128)) {
        if (mfma_ok) {
            sca_decode_params q = p;
            if (q.seq_lens == nullptr || q.batch <= kRankBatch || q.batch > kMaxOrderedBatch) {
                q.batch_order = nullptr;
            }
            if (q.batch_order != nullptr) {
                hipLaunchKernelGGL(decode_order_kernel,
                                   dim3(static_cast<unsigned>((q.batch + 255) / 256)), dim3(256),
                                   0, s, q.seq_lens, static_cast<int>(q.batch), q.batch_order);
                rc = CheckLaunch("decode_order_kernel", s);
                if (rc != 0) return rc;
            }
            const int h_chunks = static_cast<int>((group + kMfmaHeads - 1) / kMfmaHeads);
            const int64_t slots = p.num_kv_heads * h_chunks;
            if (MfmaWaveHeads(kPaged, p.slot_waves)) {
                const dim3 grid(static_cast<unsigned>(p.num_splits),
                                static_cast<unsigned>((slots + kDecodeWaves - 1) / kDecodeWaves),
                                static_cast<unsigned>(p.batch));
                hipLaunchKernelGGL((decode_mfma_kernel<E, D, kPaged, true>), grid,
                                   dim3(kDecodeThreads), 0, s, q, h_chunks, block_shift);
            } else {
                const dim3 grid(static_cast<unsigned>(p.num_splits), static_cast<unsigned>(slots),
                                static_cast<unsigned>(p.batch));
                hipLaunchKernelGGL((decode_mfma_kernel<E, D, kPaged, false>), grid,
                                   dim3(kDecodeThreads), 0, s, q, h_chunks, block_shift);
            }
            rc = CheckLaunch("decode_mfma_kernel", s);
        }
    }
    if (mfma_ok) {
    } else if (group % 8 == 0) {
        rc = LaunchPartial<E, D, 8, kPaged>(p, static_cast<int>(group / 8), s);
    } else if (group % 4 == 0) {
        rc = LaunchPartial<E, D, 4, kPaged>(p, static_cast<int>(group / 4), s);
    } else if (group % 2 == 0) {
        rc = LaunchPartial<E, D, 2, kPaged>(p, static_cast<int>(group / 2), s);
    } else {
        rc = LaunchPartial<E, D, 1, kPaged>(p, static_cast<int>(group), s);
    }
    if (rc != 0 || p.num_splits == 1) return rc;
    const int64_t threads = p.batch * p.num_heads * (D / 4);
    const unsigned blocks = static_cast<unsigned>((threads + kCombineThreads - 1) / kCombineThreads);
    hipLaunchKernelGGL((decode_combine_kernel<E, D>), dim3(blocks), dim3(kCombineThreads), 0, s, p);
    return CheckLaunch("decode_combine_kernel", s);
}

template <typename E, bool kPaged>
int LaunchTyped(const sca_decode_params& p, hipStream_t s) {
    switch (p.head_dim) {
        case 32: return LaunchForDim<E, 32, kPaged>(p, s);
        case 64: return LaunchForDim<E, 64, kPaged>(p, s);
        case 96: return LaunchForDim<E, 96, kPaged>(p, s);
        case 128: return LaunchForDim<E, 128, kPaged>(p, s);
        case 160: return LaunchForDim<E, 160, kPaged>(p, s);
        case 192: return LaunchForDim<E, 192, kPaged>(p, s);
        case 256: return LaunchForDim<E, 256, kPaged>(p, s);
        default: break;
    }
    return SetError(SCA_E_UNSUPPORTED_HEAD_DIM,
                    "decode: head_dim=" + std::to_string(p.head_dim) + " is not instantiated");
}

bool Aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

int ValidateDecode(const sca_decode_params* p, bool paged) {
    if (p == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "decode: null params");
    if (p->q == nullptr || p->k == nullptr || p->v == nullptr || p->out == nullptr) {
        return SetError(SCA_E_SHAPE_MISMATCH, "decode: null pointer");
    }
    if (p->num_splits < 1) return SetError(SCA_E_SHAPE_MISMATCH, "decode: num_splits must be >= 1");
    if (p->num_splits > 65535) {
        return SetError(SCA_E_SHAPE_MISMATCH,
                        "decode: num_splits=" + std::to_string(p->num_splits) + " > 65535");
    }
    if (p->num_splits > 1 &&
        (p->partial_m == nullptr || p->partial_l == nullptr || p->partial_o == nullptr)) {
        return SetError(SCA_E_WORKSPACE, "decode: num_splits > 1 needs partial_m/l/o scratch");
    }
    if (p->batch < 1 || p->num_heads < 1 || p->num_kv_heads < 1 ||
        p->num_heads % p->num_kv_heads != 0) {
        return SetError(SCA_E_SHAPE_MISMATCH,
                        "decode: invalid heads (H_q=" + std::to_string(p->num_heads) +
                            ", H_kv=" + std::to_string(p->num_kv_heads) + ") or batch");
    }
    if (p->batch > 65535 || p->num_heads > 65535) {
        return SetError(SCA_E_SHAPE_MISMATCH, "decode: batch/num_heads exceed the grid limit");
    }
    if (p->seq_kv < 0) return SetError(SCA_E_SHAPE_MISMATCH, "decode: seq_kv < 0");
    if (p->dtype != SCA_DTYPE_F16 && p->dtype != SCA_DTYPE_BF16 && p->dtype != SCA_DTYPE_F32) {
        return SetError(SCA_E_UNSUPPORTED_DTYPE, "decode: unsupported dtype id " +
                                                     std::to_string(p->dtype));
    }
    const int64_t eb = p->dtype == SCA_DTYPE_F32 ? 4 : 2;
    const int64_t ve = 16 / eb;
    if (!Aligned16(p->q) || !Aligned16(p->k) || !Aligned16(p->v) || !Aligned16(p->out) ||
        p->q_sb % ve || p->q_sh % ve || p->k_sb % ve || p->k_sh % ve || p->k_ss % ve ||
        p->v_sb % ve || p->v_sh % ve || p->v_ss % ve || p->o_sb % ve || p->o_sh % ve) {
        return SetError(SCA_E_LAYOUT_MISMATCH,
                        "decode: pointers must be 16 B aligned and strides multiples of 16 B");
    }
    if (p->slot_waves != 0 && p->slot_waves != 1 && p->slot_waves != kDecodeWaves) {
        return SetError(SCA_E_SHAPE_MISMATCH, "decode: slot_waves must be 0, 1 or 4; got " +
                                                  std::to_string(p->slot_waves));
    }
    if ((reinterpret_cast<uintptr_t>(p->batch_order) & 7u) != 0) {
        return SetError(SCA_E_LAYOUT_MISMATCH, "decode: batch_order must be 8 B aligned");
    }
    if (paged) {
        if (p->page_table == nullptr) {
            return SetError(SCA_E_SHAPE_MISMATCH,
                            "paged attention: page_table is null (use the contiguous entry point "
                            "instead)");
        }
        if (p->block_size <= 0 || p->max_blocks_per_seq <= 0 || p->num_kv_blocks <= 0) {
            return SetError(SCA_E_SHAPE_MISMATCH,
                            "paged attention: block_size/max_blocks_per_seq/num_kv_blocks must be "
                            "positive");
        }
    }
    return 0;
}

// ---- allocation-free variant: the split partials and the ranking scratch live in a static
// device array instead of caller memory ---------------------------------------------------------

constexpr int64_t kNoAllocPartialBytes = int64_t{16} << 20;        // split-K partials
constexpr int64_t kNoAllocOrderBytes = int64_t{2} * kMaxOrderedBatch * 4;  // batch_order
constexpr int kNoAllocMaxDevices = 64;

}  // namespace
}  // namespace sca_hip

// One copy per GPU, held until the process ends. Its host-side name is not a device address:
// kernels receive the per-device address from hipGetSymbolAddress instead.
static __device__ __align__(256) unsigned char
    scratch[sca_hip::kNoAllocPartialBytes + sca_hip::kNoAllocOrderBytes];

namespace sca_hip {
namespace {

// Device address of `scratch` on the current device, looked up once per device.
int NoAllocScratch(unsigned char** out) {
    int dev = 0;
    int rc = FromHip(hipGetDevice(&dev), "hipGetDevice");
    if (rc != 0) return rc;
    if (dev < 0 || dev >= kNoAllocMaxDevices) {
        return SetError(SCA_E_DEVICE_CAPABILITY,
                        "decode (no-alloc): device " + std::to_string(dev) + " beyond the table");
    }
    static std::atomic<unsigned char*> ptrs[kNoAllocMaxDevices];
    static std::mutex mu;
    unsigned char* ptr = ptrs[dev].load(std::memory_order_acquire);
    if (ptr == nullptr) {
        std::lock_guard<std::mutex> lock(mu);
        ptr = ptrs[dev].load(std::memory_order_relaxed);
        if (ptr == nullptr) {
            void* addr = nullptr;
            rc = FromHip(hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)),
                         "hipGetSymbolAddress(scratch)");
            if (rc != 0) return rc;
            ptr = static_cast<unsigned char*>(addr);
            ptrs[dev].store(ptr, std::memory_order_release);
        }
    }
    *out = ptr;
    return 0;
}

}  // namespace
}  // namespace sca_hip

using sca_hip::SetError;

extern "C" {

int64_t sca_hip_decode_partial_elements(int64_t batch, int64_t num_heads, int64_t num_splits,
                                        int64_t head_dim) {
    return batch * num_heads * num_splits * (2 + head_dim);
}

int sca_hip_decode_splitk(const sca_decode_params* params, void* stream) {
    int rc = sca_hip::ValidateDecode(params, /*paged=*/params != nullptr && params->page_table);
    if (rc != 0) return rc;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool paged = params->page_table != nullptr;
    switch (params->dtype) {
        case SCA_DTYPE_F16:
            return paged ? sca_hip::LaunchTyped<sca_hip::DecF16, true>(*params, s)
                         : sca_hip::LaunchTyped<sca_hip::DecF16, false>(*params, s);
        case SCA_DTYPE_BF16:
            return paged ? sca_hip::LaunchTyped<sca_hip::DecBF16, true>(*params, s)
                         : sca_hip::LaunchTyped<sca_hip::DecBF16, false>(*params, s);
        default:
            return paged ? sca_hip::LaunchTyped<sca_hip::DecF32, true>(*params, s)
                         : sca_hip::LaunchTyped<sca_hip::DecF32, false>(*params, s);
    }
}

int sca_hip_decode_splitk_paged(const sca_decode_params* params, void* stream) {
    int rc = sca_hip::ValidateDecode(params, /*paged=*/true);
    if (rc != 0) return rc;
    return sca_hip_decode_splitk(params, stream);
}

int sca_hip_decode_splitk_noalloc(const sca_decode_params* params, void* stream) {
    if (params == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "decode (no-alloc): null params");
    if (params->partial_m != nullptr || params->partial_l != nullptr ||
        params->partial_o != nullptr || params->batch_order != nullptr) {
        return SetError(SCA_E_WORKSPACE,
                        "decode (no-alloc): partial_m/l/o and batch_order must be NULL (the "
                        "library's static scratch holds them)");
    }
    sca_decode_params p = *params;
    if (p.batch < 1 || p.batch > 65535 || p.num_heads < 1 || p.num_heads > 65535 ||
        p.num_splits < 1 || p.num_splits > 65535 || p.head_dim < 1 || p.head_dim > 256) {
        return SetError(SCA_E_SHAPE_MISMATCH,
                        "decode (no-alloc): batch, num_heads and num_splits must be in "
                        "[1, 65535] and head_dim in [1, 256]");
    }
    if (p.num_splits > 1) {
        const int64_t elems = p.batch * p.num_heads * p.num_splits;
        const int64_t bytes = elems * (2 + p.head_dim) * 4;
        if (bytes > sca_hip::kNoAllocPartialBytes) {
            return SetError(SCA_E_WORKSPACE,
                            "decode (no-alloc): the split partials need " + std::to_string(bytes) +
                                " bytes, more than the static scratch's " +
                                std::to_string(sca_hip::kNoAllocPartialBytes));
        }
    }
    unsigned char* base = nullptr;
    int rc = sca_hip::NoAllocScratch(&base);
    if (rc != 0) return rc;
    if (p.num_splits > 1) {
        const int64_t elems = p.batch * p.num_heads * p.num_splits;
        float* f = reinterpret_cast<float*>(base);
        p.partial_m = f;
        p.partial_l = f + elems;
        p.partial_o = f + 2 * elems;
    }
    // Every split writes its partials and the ranking kernel writes every order entry, so
    // nothing in the scratch needs clearing between calls.
    p.batch_order = reinterpret_cast<int32_t*>(base + sca_hip::kNoAllocPartialBytes);
    return sca_hip_decode_splitk(&p, stream);
}

}  // extern "C"

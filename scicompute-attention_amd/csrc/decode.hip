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
// MI355X design (HBM-bound kernel):
//   * one workgroup per (b, kv head, split) streams its K/V chunk exactly once and serves all
//     kHeads query heads of the GQA group from registers (the reference re-reads K/V per q head);
//   * a lane owns 16 B of one token row (8 fp16/bf16 elements); LPR lanes cover a row, so a wave
//     reads 64 lanes x 16 B of consecutive token rows per load instruction;
//   * QK uses v_dot2_f32_{f16,bf16} on the packed inputs, the 16-lane row sum uses DPP,
//     and the online softmax is updated once per chunk of kChunk tokens per row group;
//   * row groups and waves are merged in registers / LDS at the end; splits == 1 writes the
//     normalised output directly and skips the combine kernel.

#include <hip/hip_runtime.h>

#include <string>

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
    const int64_t seg_tokens = kPaged ? static_cast<int64_t>(kPageSegment) * p.block_size
                                      : (t_end - t_begin);
    for (int64_t seg = t_begin; seg < t_end; seg += (seg_tokens > 0 ? seg_tokens : 1)) {
        const int64_t seg_end = (seg + seg_tokens < t_end) ? seg + seg_tokens : t_end;
        int64_t page0 = 0;
        if constexpr (kPaged) {
            page0 = seg / p.block_size;
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

template <typename E, int D, int kHeads, bool kPaged>
int LaunchPartial(const sca_decode_params& p, int h_chunks, hipStream_t s) {
    const dim3 grid(static_cast<unsigned>(p.num_splits),
                    static_cast<unsigned>(p.num_kv_heads * h_chunks),
                    static_cast<unsigned>(p.batch));
    hipLaunchKernelGGL((decode_partial_kernel<E, D, kHeads, kPaged>), grid, dim3(kDecodeThreads),
                       0, s, p, h_chunks);
    return CheckLaunch("decode_partial_kernel", s);
}

template <typename E, int D, bool kPaged>
int LaunchForDim(const sca_decode_params& p, hipStream_t s) {
    const int64_t group = p.num_heads / p.num_kv_heads;
    int rc = 0;
    if (group % 8 == 0) {
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

}  // extern "C"

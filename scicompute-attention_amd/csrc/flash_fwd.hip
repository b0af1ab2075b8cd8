// Flash prefill forward for gfx950: O = softmax(scale * Q K^T + mask) V, fp16/bf16 in, fp32
// accumulation, optional natural-log LSE. No score matrix is ever written to memory.
//
// Semantics follow the reference kernel (src/backends/flash/flash_fwd_impl.cuh:45-279,
// flash_online_softmax.cuh:34-99, flash_causal_mask.cuh:14-28): bottom-right causal mask
// (key j visible from row i iff j <= i + diagonal), masked logits are exactly -inf, GQA maps
// q head h to kv head h / (H_q / H_kv), P is rounded to the input dtype before the PV product,
// out = O / l (0 when l == 0), LSE = m + ln(l) (-inf when l == 0).
//
// Three kernels share the formulation below:
//   * flash_fwd_wide_kernel (head_dim 64 and 128: every non-causal grid, large causal grids and
//     packed variable-length batches in one launch): 4 waves of 64 query rows, K/V tiles DMA'd
//     into LDS; described at its definition;
//   * flash_fwd_pair_kernel (head_dim 64 and 128, causal grids too small to balance 128-row
//     tiles): two 4-wave groups that run a complementary pair of 64-row tiles side by side, each
//     with its own DMA ring; described at its definition;
//   * flash_fwd_kernel (head_dim 32, 96, 160, 192, 256): 4 waves = 128 query rows, K/V staged
//     through registers into a double-buffered LDS ring with V transposed on the way in.
// Formulation: S^T = K Q^T with v_mfma_f32_32x32x16_{f16,bf16} (A = K rows from LDS, B = Q^T in
// registers for the whole tile). In the S^T accumulator every lane holds 16 keys of ONE query
// row, so the row max/sum need a single exchange between the two 32-lane halves and the
// online-softmax state (m, l) is one register per lane. The P^T accumulator, converted to
// fp16/bf16, is directly the B operand of O^T = V^T P^T (the key order inside an MFMA k-step
// matches the accumulator layout), so P never leaves registers. The O rescale is lazy (only when
// the running max grows by more than kRescaleSlack, decided per wave).

#include <hip/hip_runtime.h>

#include <cstdlib>
#include <algorithm>
#include <string>
#include <vector>

#include "sca_device.hpp"

namespace sca_hip {
namespace {

constexpr int kRowsPerWave = 32;
constexpr int kRowGroups = 4;
constexpr int kBlockM = kRowGroups * kRowsPerWave;  // 128 query rows per workgroup
constexpr int kKPad = 8;        // K rows padded by 16 B
constexpr int kVPad = 4;        // V^T rows padded by 8 B
constexpr float kRescaleSlack = 8.0f;  // log2 units the running max may lag behind

// Geometry per head_dim. Every wave owns 32 query rows and 32 keys of each KV tile:
// KSPLIT waves share a row group and split the tile's keys between them (their softmax states
// are merged once at the end), so a SIMD holds KSPLIT waves whose MFMA and VALU phases overlap.
template <int D>
struct FlashGeom {
    static constexpr int KSPLIT = D <= 128 ? 2 : 1;
    static constexpr int WAVES = kRowGroups * KSPLIT;
    static constexpr int THREADS = WAVES * kWave;
    static constexpr int BN = 32 * KSPLIT;               // keys per tile
    static constexpr int STAGES = 3;                     // LDS ring depth
    static constexpr int KS = D / 16;                    // QK k-steps
    static constexpr int DT = D / 32;                    // 32-row tiles of O^T
    static constexpr int KSTR = D + kKPad;               // K row stride (elements)
    static constexpr int VSTR = BN + kVPad;              // V^T row stride (elements)
    static constexpr int K_CHUNKS = BN * D / 8;          // 16 B chunks per K tile
    static constexpr int K_PER_THREAD = (K_CHUNKS + THREADS - 1) / THREADS;
    static constexpr int V_UNITS = (BN / 4) * (D / 8);   // 4 keys x 8 dims per unit
    static constexpr int V_PER_THREAD = (V_UNITS + THREADS - 1) / THREADS;
    static constexpr int K_STAGE = BN * KSTR;
    static constexpr int V_STAGE = D * VSTR;
    static constexpr int STAGE_BYTES = STAGES * (K_STAGE + V_STAGE) * 2;
    static constexpr int MERGE_FLOATS = DT * 16 + 2;     // per lane: O^T + m + l
    static constexpr int MERGE_BYTES = KSPLIT > 1 ? kRowGroups * kWave * MERGE_FLOATS * 4 : 0;
    static constexpr int LDS_BYTES = STAGE_BYTES > MERGE_BYTES ? STAGE_BYTES : MERGE_BYTES;
};

template <typename E>
struct Mfma;

template <>
struct Mfma<F16> {
    typedef _Float16 pair_t __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ floatx16 mma(const half8& a, const half8& b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    // Two floats -> packed pair (round to nearest even), as the raw 32-bit word.
    static __device__ __forceinline__ uint32_t pack(float a, float b) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, pair_t));
    }
    // acc + a.x + a.y in fp32 (v_dot2 with (1, 1)).
    static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
        const pair_t ones = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(pair_t, w), ones, acc, false);
    }
};

template <>
struct Mfma<BF16> {
    typedef __bf16 pair_t __attribute__((ext_vector_type(2)));
    static __device__ __forceinline__ floatx16 mma(const bf16x8& a, const bf16x8& b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ uint32_t pack(float a, float b) {
        typedef float f2 __attribute__((ext_vector_type(2)));
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){a, b}, pair_t));
    }
    static __device__ __forceinline__ float sum2(uint32_t w, float acc) {
        const pair_t ones = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(pair_t, w), ones, acc, false);
    }
};

__device__ __forceinline__ uint32_t Half16(const uint4& v, int t) {
    const uint32_t w = (t < 2) ? v.x : (t < 4) ? v.y : (t < 6) ? v.z : v.w;
    return (t & 1) ? (w >> 16) : (w & 0xffffu);
}

// Workgroup -> (row tile index, batch*head). The dispatcher deals workgroups to the eight XCDs
// round robin (workgroup w on XCD w % 8), and each XCD has its own L2. When the (batch, KV head)
// groups divide by eight, XCD x takes groups x, x + 8, ...: the query heads that read one KV head
// run on one XCD and share its L2 (C3, 4 x 8 groups of 4 heads: +5%). Otherwise w runs row tile
// w / bh_count of head w % bh_count. Either way row tile t starts before t + 1 (so longest-first
// orders survive), and the mapping is a bijection on [0, tiles * bh_count).
__device__ __forceinline__ void XcdOrder(const sca_flash_params& p, int64_t bh_count,
                                         int64_t* tile_linear, int64_t* bh) {
    const int64_t w = blockIdx.x;
    const int64_t groups = p.batch * p.num_kv_heads;
    if (groups % 8 != 0) {
        *tile_linear = w / bh_count;
        *bh = w % bh_count;
        return;
    }
    const int64_t gsz = p.num_heads / p.num_kv_heads;
    const int64_t per_tile = bh_count / 8;  // workgroups of one row tile on one XCD
    const int64_t pos = w / 8;
    const int64_t rem = pos % per_tile;
    *tile_linear = pos / per_tile;
    *bh = ((rem / gsz) * 8 + w % 8) * gsz + rem % gsz;
}

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedValu = 0x002;
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;


template <typename E, int D, bool kCausal>
__global__ __launch_bounds__(FlashGeom<D>::THREADS, 1) void flash_fwd_kernel(
    const sca_flash_params p, int num_q_tiles) {
    using G = FlashGeom<D>;
    using M = Mfma<E>;
    using vec8 = typename E::vec8;
    constexpr int BN = G::BN;

    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t* sK = lds;                           // [STAGES][BN][KSTR]
    uint16_t* sV = lds + G::STAGES * G::K_STAGE;  // [STAGES][D][VSTR]  (V^T)

    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int lr = lane & 31;
    const int hh = lane >> 5;
    const int rg = wave % kRowGroups;  // row group
    const int kh = wave / kRowGroups;  // which 32 keys of every tile this wave owns

    // Block -> (tile, batch*head). Causal: longest row tiles are dispatched first.
    const int64_t bh_count = p.batch * p.num_heads;
    int64_t tile_linear, bh;
    XcdOrder(p, bh_count, &tile_linear, &bh);
    const int64_t qt = kCausal ? (num_q_tiles - 1 - tile_linear) : tile_linear;
    const int64_t b = bh / p.num_heads;
    const int64_t h = bh % p.num_heads;
    const int64_t h_kv = h / (p.num_heads / p.num_kv_heads);
    const int q0 = static_cast<int>(qt) * kBlockM;
    const int wave_q0 = q0 + rg * kRowsPerWave;
    const int my_q = wave_q0 + lr;
    const int seq_q = static_cast<int>(p.seq_q);
    const int seq_kv = static_cast<int>(p.seq_kv);
    const int diag = static_cast<int>(p.diagonal);

    const uint16_t* q_ptr = static_cast<const uint16_t*>(p.q) + b * p.q_sb + h * p.q_sh;
    const uint16_t* k_ptr = static_cast<const uint16_t*>(p.k) + b * p.k_sb + h_kv * p.k_sh;
    const uint16_t* v_ptr = static_cast<const uint16_t*>(p.v) + b * p.v_sb + h_kv * p.v_sh;

    // Q^T fragments (B operand of S^T = K Q^T): lane holds Q[my_q][16*ks + 8*hh + 0..7].
    vec8 qf[G::KS];
    {
        const uint16_t* q_row = q_ptr + static_cast<int64_t>(my_q) * p.q_ss + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            uint4 raw = make_uint4(0, 0, 0, 0);
            if (my_q < seq_q) raw = *reinterpret_cast<const uint4*>(q_row + 16 * ks);
            qf[ks] = __builtin_bit_cast(vec8, raw);
        }
        // Retire the Q loads here on every path. Otherwise the waitcnt pass, which merges the
        // loop-entry state conservatively, waits for *all* outstanding loads (including the
        // next tile's prefetch) before the first MFMA of every tile.
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), expcnt/lgkmcnt unconstrained
    }

    int n_tiles = (seq_kv + BN - 1) / BN;
    // Tiles [0, n_plain) are inside seq_kv and fully visible to every row of the workgroup.
    int n_plain = seq_kv / BN;
    if (kCausal) {
        const int last_key = q0 + kBlockM - 1 + diag;
        const int causal_tiles = last_key < 0 ? 0 : last_key / BN + 1;
        if (causal_tiles < n_tiles) n_tiles = causal_tiles;
        const int plain = (q0 + diag + 1) / BN;
        if (plain < n_plain) n_plain = plain;
    }
    if (n_plain > n_tiles) n_plain = n_tiles;

    floatx16 o[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] = 0.0f;
    }
    float m_used = neg_inf();  // running max used for the exponentials (log2 units)
    float l_run = 0.0f;        // sum of this lane's rounded weights
    const float scale2 = p.scale * kLog2e;

    // ---- staging: global -> registers -> LDS ------------------------------------------------
    // Per-thread 32-bit element offsets inside one tile, fixed for the whole kernel.
    int k_off[G::K_PER_THREAD], k_row[G::K_PER_THREAD], k_lds[G::K_PER_THREAD];
#pragma unroll
    for (int i = 0; i < G::K_PER_THREAD; ++i) {
        const int c = tid + i * G::THREADS;
        const int row = c / (D / 8);
        const int col = (c % (D / 8)) * 8;
        k_row[i] = c < G::K_CHUNKS ? row : (1 << 30);
        k_off[i] = row * static_cast<int>(p.k_ss) + col;
        k_lds[i] = row * G::KSTR + col;
    }
    int v_off[G::V_PER_THREAD], v_key[G::V_PER_THREAD], v_lds[G::V_PER_THREAD];
#pragma unroll
    for (int i = 0; i < G::V_PER_THREAD; ++i) {
        const int u = tid + i * G::THREADS;
        const int kg = u / (D / 8);
        const int dc = u % (D / 8);
        v_key[i] = u < G::V_UNITS ? 4 * kg : (1 << 30);
        v_off[i] = 4 * kg * static_cast<int>(p.v_ss) + 8 * dc;
        v_lds[i] = 8 * dc * G::VSTR + 4 * kg;
    }
    const int v_ss = static_cast<int>(p.v_ss);

    uint4 k_stage[G::K_PER_THREAD];
    uint4 v_stage[G::V_PER_THREAD][4];

    auto load_tile = [&](int t) {
        const int key0 = t * BN;
        const uint16_t* kt = k_ptr + static_cast<int64_t>(key0) * p.k_ss;
        const uint16_t* vt = v_ptr + static_cast<int64_t>(key0) * p.v_ss;
        const int limit = seq_kv - key0;  // keys of this tile that exist
#pragma unroll
        for (int i = 0; i < G::K_PER_THREAD; ++i) {
            k_stage[i] = make_uint4(0, 0, 0, 0);
            if (k_row[i] < limit) k_stage[i] = *reinterpret_cast<const uint4*>(kt + k_off[i]);
        }
#pragma unroll
        for (int i = 0; i < G::V_PER_THREAD; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v_stage[i][j] = make_uint4(0, 0, 0, 0);
                if (v_key[i] + j < limit) {
                    v_stage[i][j] = *reinterpret_cast<const uint4*>(vt + v_off[i] + j * v_ss);
                }
            }
        }
    };

    auto store_tile = [&](int stage) {
        uint16_t* k_dst = sK + stage * G::K_STAGE;
        uint16_t* v_dst = sV + stage * G::V_STAGE;
#pragma unroll
        for (int i = 0; i < G::K_PER_THREAD; ++i) {
            if (k_row[i] < BN) *reinterpret_cast<uint4*>(k_dst + k_lds[i]) = k_stage[i];
        }
#pragma unroll
        for (int i = 0; i < G::V_PER_THREAD; ++i) {
            if (v_key[i] < BN) {
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const uint32_t lo = Half16(v_stage[i][0], t) | (Half16(v_stage[i][1], t) << 16);
                    const uint32_t hi = Half16(v_stage[i][2], t) | (Half16(v_stage[i][3], t) << 16);
                    *reinterpret_cast<uint2*>(v_dst + v_lds[i] + t * G::VSTR) = make_uint2(lo, hi);
                }
            }
        }
    };

    const int wkey_base = 32 * kh;  // this wave's first key inside a tile
    const uint16_t* k_frag_base = sK + (wkey_base + lr) * G::KSTR + 8 * hh;
    const uint16_t* v_frag_base = sV + lr * G::VSTR + wkey_base + 4 * hh;

    // S^T[key][q] for this wave's 32 keys x 32 rows of the tile in `stage`.
    auto qk = [&](int stage) {
        const uint16_t* k_tile = k_frag_base + stage * G::K_STAGE;
        vec8 a[G::KS];
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) a[ks] = *reinterpret_cast<const vec8*>(k_tile + 16 * ks);
        floatx16 s;
#pragma unroll
        for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) s = M::mma(a[ks], qf[ks], s);
        return s;
    };

    if (n_tiles > 0) {
        load_tile(0);
        store_tile(0);
        if (n_tiles > 1) {
            load_tile(1);
            store_tile(1);
        }
    }
    __syncthreads();
    floatx16 s_cur = qk(0);

    // One pipeline step. Tiles j and j+1 are resident in LDS, tile j+2 is being fetched:
    //   region A: QK MFMAs of tile j+1 interleaved with the softmax VALU work of tile j;
    //   O rescale (only when some lane's running max moved);
    //   region C: PV MFMAs of tile j; then tile j+2 goes to LDS and the workgroup syncs.
    auto step = [&]<bool kMask>(int j) {
        if (j + 2 < n_tiles) load_tile(j + 2);
        const int stage = j % G::STAGES;
        const int next_stage = (j + 1) % G::STAGES;

        // ---- region A (straight-line code) ----
        floatx16 s_nxt = qk(next_stage);  // for the last tile this reads a stale stage; unused
        floatx16 s = s_cur;
        if constexpr (kMask) {
            const int lim = kCausal ? min(seq_kv - 1, my_q + diag) : seq_kv - 1;
            const int kbase = j * BN + wkey_base + 4 * hh;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kbase + 8 * (i / 4) + (i % 4);
                s[i] = key > lim ? neg_inf() : s[i];
            }
        }
        float tmax = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])),
                           fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
        tmax = fmaxf(tmax, fmaxf(fmaxf(fmaxf(s[8], s[9]), fmaxf(s[10], s[11])),
                                 fmaxf(fmaxf(s[12], s[13]), fmaxf(s[14], s[15]))));
        tmax = fmaxf(tmax, xor32(tmax)) * scale2;
        // Lazy rescale: the max used for the exponentials only moves when the row max grew by
        // more than kRescaleSlack (weights stay <= 2^slack).
        const bool grow = tmax > m_used + kRescaleSlack;
        const float m_new = grow ? tmax : m_used;
        const float alpha = grow ? fast_exp2(m_used - m_new) : 1.0f;
        m_used = m_new;
        l_run *= alpha;
        const float mu = (m_used == neg_inf()) ? 0.0f : m_used;
        uint32_t pw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float p0 = fast_exp2(fmaf(s[2 * i], scale2, -mu));
            const float p1 = fast_exp2(fmaf(s[2 * i + 1], scale2, -mu));
            pw[i] = M::pack(p0, p1);
            l_run = M::sum2(pw[i], l_run);
        }
        // Materialise P here: without this use the exponentials are sunk into region C, past
        // the rescale branch, and no longer overlap the QK MFMAs.
#pragma unroll
        for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(pw[i]));
        // interleave: K-fragment reads first, then one MFMA per ~12 VALU instructions
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, G::KS, 0);
#pragma unroll
        for (int i = 0; i < G::KS; ++i) {
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedValu, 12, 0);
        }

        // ---- O rescale (rare) ----
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
            }
        }

        // ---- region C: O^T[d][q] += V^T[d][key] P^T[key][q] ----
        // k-step ps covers keys 16*ps + {0..3, 8..11} (hh = 0) or 16*ps + {4..7, 12..15} (hh = 1).
        const vec8 pb0 = __builtin_bit_cast(vec8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
        const vec8 pb1 = __builtin_bit_cast(vec8, make_uint4(pw[4], pw[5], pw[6], pw[7]));
        const uint16_t* v_tile = v_frag_base + stage * G::V_STAGE;
        vec8 va[G::DT][2];
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
            for (int ps = 0; ps < 2; ++ps) {
                const uint16_t* vrow = v_tile + 32 * dt * G::VSTR + 16 * ps;
                const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 8);
                va[dt][ps] = __builtin_bit_cast(vec8, make_uint4(lo.x, lo.y, hi.x, hi.y));
            }
        }
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
            o[dt] = M::mma(va[dt][0], pb0, o[dt]);
            o[dt] = M::mma(va[dt][1], pb1, o[dt]);
        }
        // all V^T fragment reads in flight before the first PV MFMA
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * G::DT, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2 * G::DT, 0);

        if (j + 2 < n_tiles) store_tile((j + 2) % G::STAGES);
        __syncthreads();
        s_cur = s_nxt;
    };

    int j = 0;
    for (; j < n_plain; ++j) step.template operator()<false>(j);
    for (; j < n_tiles; ++j) step.template operator()<true>(j);

    // Merge the KSPLIT partial states of each row group through LDS.
    if constexpr (G::KSPLIT > 1) {
        float* mbuf = reinterpret_cast<float*>(lds) + (rg * kWave + lane) * G::MERGE_FLOATS;
        if (kh == 1) {
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
                for (int i = 0; i < 16; ++i) mbuf[dt * 16 + i] = o[dt][i];
            }
            mbuf[G::DT * 16] = m_used;
            mbuf[G::DT * 16 + 1] = l_run;
        }
        __syncthreads();
        if (kh == 1) return;
        const float m_o = mbuf[G::DT * 16];
        const float l_o = mbuf[G::DT * 16 + 1];
        const float mm = fmaxf(m_used, m_o);
        const float wa = (m_used == neg_inf()) ? 0.0f : fast_exp2(m_used - mm);
        const float wb = (m_o == neg_inf()) ? 0.0f : fast_exp2(m_o - mm);
        m_used = mm;
        l_run = l_run * wa + l_o * wb;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) o[dt][i] = o[dt][i] * wa + mbuf[dt * 16 + i] * wb;
        }
    }

    // Epilogue: merge the two lane halves' sums, normalise, store.
    const float l_tot = l_run + xor32(l_run);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (my_q < seq_q) {
        uint16_t* out_row = static_cast<uint16_t*>(p.out) + b * p.o_sb + h * p.o_sh +
                            static_cast<int64_t>(my_q) * p.o_ss;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = 32 * dt + 8 * g + 4 * hh;
                const uint32_t lo = M::pack(o[dt][4 * g + 0] * inv, o[dt][4 * g + 1] * inv);
                const uint32_t hi = M::pack(o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv);
                *reinterpret_cast<uint2*>(out_row + d0) = make_uint2(lo, hi);
            }
        }
        if (p.lse != nullptr && hh == 0) {
            p.lse[(b * p.num_heads + h) * p.seq_q + my_q] =
                l_tot > 0.0f ? (m_used + __log2f(l_tot)) * kLn2 : neg_inf();
        }
    }
}

// ============================================================================================
// The DMA pipeline of the head_dim 64 / 128 kernels (pair and wide).
//
// K and V tiles go straight from global memory to LDS with buffer loads to LDS (16 bytes per
// lane, no VGPR staging, no transposition) through a buffer resource bounded at the sequence's
// last row, so rows past seq_kv read as zero. Loads are issued ahead of their use and retired
// with explicit vmcnt waits plus one barrier per tile. LDS rows are unpadded; 16-byte chunks are
// XOR-swizzled per row (SwzK / SwzV) so that both the K reads and the V transpose reads are
// bank-conflict free. The PV A operand (V^T fragments) comes from ds_read_b64_tr_b16: within each
// 16-lane group, lane j receives element j % 4 of the 8 bytes read by lane 4*i + j/4 (i = 0..3),
// i.e. one head-dim column over 4 consecutive keys.
// ============================================================================================

// 16-byte-chunk swizzles for 64 LDS banks (a 256-byte bank window):
//   K: the 32 rows a wave reads in one ds_read_b128 land on 16 distinct 4-bank groups;
//   V: the 8 keys x 4 chunks of one transpose read land on 16 distinct groups.
template <int D>
__device__ __forceinline__ int SwzK(int row) {
    return D == 128 ? (row & 15) : ((row >> 1) & 7);
}
template <int D>
__device__ __forceinline__ int SwzV(int row) {
    return D == 128 ? ((row & 3) << 2) : (((row >> 1) & 1) << 2);
}

// (lower-half value, upper-half value) of v for lanes l and l ^ 32, on every lane, from one
// v_permlane32_swap: it exchanges the upper 32 lanes of its first operand with the lower 32 lanes
// of its second, so with both operands holding v the first ends as (v_lo, v_lo) and the second as
// (v_hi, v_hi). Issued from inline asm with both registers as in/out operands (the builtin's
// second result is not reliably kept apart from the first), after the two wait states a VALU
// write needs before the permlane reads it.
__device__ __forceinline__ void HalfPair(float v, float* lo, float* hi) {
    uint32_t a = __builtin_bit_cast(uint32_t, v);
    uint32_t b = a;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
    *lo = __builtin_bit_cast(float, a);
    *hi = __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float HalfMax(float v) {
    float lo, hi;
    HalfPair(v, &lo, &hi);
    return fmaxf(lo, hi);
}
__device__ __forceinline__ float HalfSum(float v) {
    float lo, hi;
    HalfPair(v, &lo, &hi);
    return lo + hi;
}

// ---- Online softmax of one 32-key x 32-row S^T tile (lane: 16 keys of one row; lanes l and
// l ^ 32 hold the other 16 keys of the same row) -----------------------------------------------
// Per-lane row state: the running max used for the exponentials (m, log2 units), the raw-score
// threshold above which it must move (thr = (m + kRescaleSlack) / scale2), the exponent bias
// (-m, or 0 while no key of the row was visible) and this lane's share of the denominator.
struct RowState {
    float m;
    float thr;
    float neg_mu;
    float l;
};

__device__ __forceinline__ void ResetRow(RowState& r) {
    r.m = neg_inf();
    r.thr = neg_inf();
    r.neg_mu = 0.0f;
    r.l = 0.0f;
}

__device__ __forceinline__ float Max16(const floatx16& s) {
    const float a = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    const float b = fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7]));
    const float c = fmaxf(fmaxf(s[8], s[9]), fmaxf(s[10], s[11]));
    const float d = fmaxf(fmaxf(s[12], s[13]), fmaxf(s[14], s[15]));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Transposed 8-byte LDS read at byte address addr + OFF. Issued from inline asm so that the
// compiler's conservative LDS-DMA tracking adds no wait for DMAs still in flight; the caller
// retires the reads with WaitLdsTied before the registers are used.
template <int OFF>
__device__ __forceinline__ uint2 TrReadAsm(uint32_t addr) {
    uint2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}

// lgkmcnt(0), tied to the registers it guards so that no use of them is scheduled above it,
// and to the P operands (a, b) so that it is not hoisted above the exponentials either.
template <typename V, int N>
__device__ __forceinline__ void WaitLdsTied(V (&regs)[N], V& a, V& b) {
    if constexpr (N == 8) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(regs[0]), "+v"(regs[1]), "+v"(regs[2]), "+v"(regs[3]), "+v"(regs[4]),
                       "+v"(regs[5]), "+v"(regs[6]), "+v"(regs[7]), "+v"(a), "+v"(b));
    } else if constexpr (N == 4) {
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(regs[0]), "+v"(regs[1]), "+v"(regs[2]), "+v"(regs[3]), "+v"(a),
                       "+v"(b));
    } else {
        static_assert(N == 8 || N == 4, "tied wait covers 4 or 8 registers");
    }
}

__device__ __forceinline__ uint32_t LdsAddr(const void* p) {
    return static_cast<uint32_t>(
        reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) uint8_t*)(p)));
}

// V^T fragments of one key tile for the PV MFMAs: for O tile dt, k-step ps, the transposed
// reads at rows 16*ps and 16*ps + 8 of the lane's V position (v_addr[dt], LDS byte address of
// the slot-0 copy); SLOT_OFF selects the slot.
template <int SLOT_OFF, int ROW_BYTES, int DT, typename vec8>
__device__ __forceinline__ void ReadVFrags(const uint32_t (&v_addr)[DT], vec8 (&va)[2 * DT]) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
        const uint2 l0 = TrReadAsm<SLOT_OFF>(v_addr[dt]);
        const uint2 h0 = TrReadAsm<SLOT_OFF + 8 * ROW_BYTES>(v_addr[dt]);
        const uint2 l1 = TrReadAsm<SLOT_OFF + 16 * ROW_BYTES>(v_addr[dt]);
        const uint2 h1 = TrReadAsm<SLOT_OFF + 24 * ROW_BYTES>(v_addr[dt]);
        va[2 * dt] = __builtin_bit_cast(vec8, make_uint4(l0.x, l0.y, h0.x, h0.y));
        va[2 * dt + 1] = __builtin_bit_cast(vec8, make_uint4(l1.x, l1.y, h1.x, h1.y));
    }
}

constexpr int kSchedValuTrans = 0x402;  // VALU and transcendental

// 16-byte DMA of lane data from a raw buffer (base, num_records) at voffset + soffset into LDS
// at lds + 16 * lane. Bytes at or beyond num_records read as zero. (The buffer resource is
// built here rather than in the kernel body: a buffer-resource local in a kernel body makes the
// host pass drop the kernel's launch stub.)
__device__ __forceinline__ void DmaToLds(const uint8_t* base, int num_records, uint8_t* lds,
                                         uint32_t voffset, uint32_t soffset) {
    const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(base), 0, num_records, 0x00020000);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)(lds), 16,
                                             voffset, soffset, 0, 0);
}

// Packed variable-length launch: cumulative token offsets and the work list (2 int32 per row
// tile: sequence, tile), device-resident.
struct VarlenArgs {
    const int32_t* cu_q;
    const int32_t* cu_kv;
    const int32_t* tiles;
};

// ---- Two-group causal pair kernel ---------------------------------------------------------------
// Small causal grids: each workgroup owns the complementary 64-row tiles A = T-1-t (long) and
// B = t (short) and runs them concurrently in two groups of four waves (one wave of each group
// per SIMD), each group with its own K/V ring. Group 0 takes A's key tiles [0, x); group 1
// takes all of B, finishes B (a two-way merge and the stores), then takes A's key tiles
// [x, n_A). The two groups' A states are merged once at the end, so the short tile's setup,
// merge and stores run beside the long tile's key loop instead of after it. x balances the
// two groups' barrier intervals.
// Within a group: 2 row groups of 32 rows x 2 waves of 32 keys per 64-key tile; the pipeline
// step j computes QK of tile j+1 under the softmax of tile j, then PV of tile j.
template <int D>
struct PairGeom {
    static constexpr int GW = 4;                      // waves per group
    static constexpr int THREADS = 2 * GW * kWave;
    static constexpr int BM = 64;                     // rows per row tile
    static constexpr int BN = 64;                     // keys per key tile
    static constexpr int KS = D / 16;
    static constexpr int DT = D / 32;
    static constexpr int CPR = D / 8;
    static constexpr int ROW_BYTES = D * 2;
    static constexpr int TILE_BYTES = BN * D * 2;
    static constexpr int IPW = BN * CPR / (kWave * GW);  // DMA instructions per wave per tile
    static constexpr int RING_BYTES = 4 * TILE_BYTES;    // K slots 0, 1, then V slots 0, 1
    // Final merge: per row group, three partial states (16-byte quads) and their (m, l).
    static constexpr int MERGE_QUADS = 2 * 3 * 4 * DT * kWave;
    static constexpr int MERGE_BYTES = MERGE_QUADS * 16 + 2 * 3 * kWave * 8;
    static constexpr int LDS_BYTES = 2 * RING_BYTES > MERGE_BYTES ? 2 * RING_BYTES : MERGE_BYTES;
    static_assert(IPW >= 1 && BN * CPR == IPW * kWave * GW, "tile must split evenly into DMAs");
    static_assert(2 * 4 * DT * kWave * 16 + 2 * kWave * 8 <= RING_BYTES,
                  "the B merge fits group 1's ring");
    static_assert(TILE_BYTES < 65536, "slot offsets are DS immediates");
};

template <typename E, int D>
__global__ __launch_bounds__(PairGeom<D>::THREADS, 1) void flash_fwd_pair_kernel(
    const sca_flash_params p, int num_q_tiles) {
    using G = PairGeom<D>;
    using M = Mfma<E>;
    using vec8 = typename E::vec8;
    constexpr int BN = G::BN;
    constexpr int BM = G::BM;
    constexpr int ROW_BYTES = G::ROW_BYTES;

    extern __shared__ __align__(16) uint8_t lds8[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int lr = lane & 31;
    const int hh = lane >> 5;
    const int g = wave / G::GW;        // group
    const int w4 = wave % G::GW;       // wave within the group
    const int rg = w4 % 2;             // row group: rows 32*rg .. of the row tile
    const int kq = w4 / 2;             // keys 32*kq .. of every key tile

    // The groups share the workgroup barrier: every interval between two barriers is one
    // pipeline step (or setup / merge phase) of each group. The group with fewer intervals
    // pads with empty ones before the final merge, so both groups reach the same count.
    int syncs = 0;
    auto gsync = [&]() {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        ++syncs;
    };

    const int64_t bh_count = p.batch * p.num_heads;
    int64_t tile_linear, bh;
    XcdOrder(p, bh_count, &tile_linear, &bh);
    const int64_t b = bh / p.num_heads;
    const int64_t h = bh % p.num_heads;
    const int64_t h_kv = h / (p.num_heads / p.num_kv_heads);
    const int seq_q = static_cast<int>(p.seq_q);
    const int seq_kv = static_cast<int>(p.seq_kv);
    const int diag = static_cast<int>(p.diagonal);
    const float scale2 = p.scale * kLog2e;
    const float inv_scale2 = 1.0f / scale2;

    const uint8_t* k_bytes = reinterpret_cast<const uint8_t*>(
        static_cast<const uint16_t*>(p.k) + b * p.k_sb + h_kv * p.k_sh);
    const uint8_t* v_bytes = reinterpret_cast<const uint8_t*>(
        static_cast<const uint16_t*>(p.v) + b * p.v_sb + h_kv * p.v_sh);
    const int k_row_bytes = static_cast<int>(p.k_ss) * 2;
    const int v_row_bytes = static_cast<int>(p.v_ss) * 2;
    const int k_records = (seq_kv - 1) * k_row_bytes + ROW_BYTES;
    const int v_records = (seq_kv - 1) * v_row_bytes + ROW_BYTES;
    uint32_t dma_koff[G::IPW], dma_voff[G::IPW];
#pragma unroll
    for (int i = 0; i < G::IPW; ++i) {
        const int P = (w4 * G::IPW + i) * kWave + lane;
        const int row = P / G::CPR;
        const int pos = P % G::CPR;
        dma_koff[i] = row * k_row_bytes + (pos ^ SwzK<D>(row)) * 16;
        dma_voff[i] = row * v_row_bytes + (pos ^ SwzV<D>(row)) * 16;
    }
    uint8_t* const ring = lds8 + g * G::RING_BYTES;
    // K tile t -> K slot t & 1, V tile t -> V slot t & 1 of this group's ring.
    auto issue_k = [&](int t) {
        uint8_t* dst = ring + (t & 1) * G::TILE_BYTES + w4 * G::IPW * 1024;
        const uint32_t off = static_cast<uint32_t>(t * BN * k_row_bytes);
#pragma unroll
        for (int i = 0; i < G::IPW; ++i) DmaToLds(k_bytes, k_records, dst + i * 1024, dma_koff[i], off);
    };
    auto issue_v = [&](int t) {
        uint8_t* dst = ring + (2 + (t & 1)) * G::TILE_BYTES + w4 * G::IPW * 1024;
        const uint32_t off = static_cast<uint32_t>(t * BN * v_row_bytes);
#pragma unroll
        for (int i = 0; i < G::IPW; ++i) DmaToLds(v_bytes, v_records, dst + i * 1024, dma_voff[i], off);
    };
    // Fragment offsets, with the group's ring base folded in so slot offsets stay immediates.
    const int wkey_base = 32 * kq;
    const int k_row = wkey_base + lr;
    uint32_t k_frag[G::KS];
#pragma unroll
    for (int ks = 0; ks < G::KS; ++ks) {
        k_frag[ks] = g * G::RING_BYTES + k_row * ROW_BYTES + (((2 * ks) ^ hh ^ SwzK<D>(k_row)) * 16);
    }
    const int grp = lane >> 4;
    const int sl = lane & 15;
    const int v_key = wkey_base + 4 * hh + (sl >> 2);
    const int v_chunk = 2 * (grp & 1) + ((sl & 3) >> 1);
    const int v_half = (sl & 1) * 8;
    uint32_t v_frag[G::DT], v_addr[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt) {
        v_frag[dt] = g * G::RING_BYTES + v_key * ROW_BYTES +
                     (((4 * dt + v_chunk) ^ SwzV<D>(v_key)) * 16) + v_half;
        v_addr[dt] = LdsAddr(lds8) + v_frag[dt];
    }

    // Row tiles: A = T-1-t (long), B = t (short; none when they coincide).
    const int qa = num_q_tiles - 1 - static_cast<int>(tile_linear);
    const int qb = static_cast<int>(tile_linear);
    const bool has_b = qb < qa;
    auto key_tiles = [&](int qt, int& n, int& n_plain) {
        const int q0 = qt * BM;
        n = (seq_kv + BN - 1) / BN;
        n_plain = seq_kv / BN;
        const int last_key = q0 + BM - 1 + diag;
        const int causal_tiles = last_key < 0 ? 0 : last_key / BN + 1;
        if (causal_tiles < n) n = causal_tiles;
        const int plain = (q0 + diag + 1) / BN;
        if (plain < n_plain) n_plain = plain;
        if (n_plain > n) n_plain = n;
    };
    int n_a, plain_a, n_b = 0, plain_b = 0;
    key_tiles(qa, n_a, plain_a);
    if (has_b) key_tiles(qb, n_b, plain_b);
    // Group 0: A tiles [0, x). Group 1: B, its merge, then A tiles [x, n_a). A key range
    // [kb, ke) takes ke - kb + 2 barrier intervals (two for its prologue), B's merge two, so
    // x + 2 = (n_b + 2) + 2 + (n_a - x + 2) balances the groups.
    int x = (n_a + n_b + (has_b ? 4 : 0) + 1) / 2;
    if (x > n_a) x = n_a;
    if (x < 1) x = 1;
    const int syncs_g0 = x + 2;
    const int syncs_g1 = (has_b ? n_b + 4 : 0) + (x < n_a ? n_a - x + 2 : 0);
    const int syncs_all = syncs_g0 > syncs_g1 ? syncs_g0 : syncs_g1;

    vec8 qf[G::KS];
    auto load_q = [&](int qt) {
        const int row = qt * BM + rg * 32 + lr;
        const uint16_t* q_row = static_cast<const uint16_t*>(p.q) + b * p.q_sb + h * p.q_sh +
                                static_cast<int64_t>(row) * p.q_ss + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            uint4 raw = make_uint4(0, 0, 0, 0);
            if (row < seq_q) raw = *reinterpret_cast<const uint4*>(q_row + 16 * ks);
            qf[ks] = __builtin_bit_cast(vec8, raw);
        }
    };

    floatx16 o[G::DT];
    RowState rs;
    auto reset_state = [&]() {
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) o[dt][i] = 0.0f;
        }
        ResetRow(rs);
    };

    auto qk_slot = [&](int slot) {
        const uint8_t* base = lds8 + slot * G::TILE_BYTES;
        vec8 a[G::KS];
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) a[ks] = *reinterpret_cast<const vec8*>(base + k_frag[ks]);
        floatx16 acc;
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) acc = M::mma(a[ks], qf[ks], acc);
        return acc;
    };

    // Key tiles [kb, ke) of row tile qt into the running state (o, rs.m, rs.l).
    auto run_keys = [&](int qt, int kb, int ke, int n_plain) {
        if (kb >= ke) return;
        const int my_q = qt * BM + rg * 32 + lr;
        const int lim = min(seq_kv - 1, my_q + diag);
        // Keys above lim_j read as -inf.
        auto mask = [&](int jt, int lim_j, floatx16& sv) {
            const int kbase = jt * BN + wkey_base + 4 * hh;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kbase + 8 * (i / 4) + (i % 4);
                sv[i] = key > lim_j ? neg_inf() : sv[i];
            }
        };
        // Scores of one tile -> exponent arguments in place (t = s * scale2 - m), the first
        // half's weights (keys of pw[0..3]) and their sum. Returns the lane's raw maximum.
        auto prep = [&](floatx16& sv, uint32_t (&ph)[4], float& sh) {
            const float lm = Max16(sv);
#pragma unroll
            for (int i = 0; i < 16; ++i) sv[i] = fmaf(sv[i], scale2, rs.neg_mu);
            float a = 0.0f, c = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p0 = fast_exp2(sv[2 * i]);
                const float p1 = fast_exp2(sv[2 * i + 1]);
                ph[i] = M::pack(p0, p1);
                a += p0;
                c += p1;
            }
            sh = a + c;
            // Pinned here: otherwise they sink below the rare rescale branch, out of PV's shadow.
#pragma unroll
            for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(ph[i]));
            asm volatile("" : "+v"(sh));
            return lm;
        };
        // Lazy rescale, decided after prep ran with the current maximum: only when some lane of
        // the wave sees a raw score above its threshold does the wave exchange the two half-row
        // maxima and move m (to the row maximum, when it exceeds m by more than kRescaleSlack),
        // scaling O and l by 2^(m_old - m_new); the tile's exponent arguments and first-half
        // weights are then redone. The exponentials stay bounded by 2^kRescaleSlack.
        auto fix = [&](float lm, floatx16& sv, uint32_t (&ph)[4], float& sh) {
            if (__builtin_amdgcn_ballot_w64(lm > rs.thr) == 0) return;
            const float tmax = HalfMax(lm) * scale2;
            const bool grow = tmax > rs.m + kRescaleSlack;
            const float m_new = grow ? tmax : rs.m;
            const float alpha = grow ? fast_exp2(rs.m - m_new) : 1.0f;
            const float neg_mu_new = (m_new == neg_inf()) ? 0.0f : -m_new;
            const float delta = neg_mu_new - rs.neg_mu;
            rs.m = m_new;
            rs.l *= alpha;
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
            }
            rs.thr = (rs.m + kRescaleSlack) * inv_scale2;
            rs.neg_mu = neg_mu_new;
#pragma unroll
            for (int i = 0; i < 16; ++i) sv[i] += delta;
            float a = 0.0f, c = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float p0 = fast_exp2(sv[2 * i]);
                const float p1 = fast_exp2(sv[2 * i + 1]);
                ph[i] = M::pack(p0, p1);
                a += p0;
                c += p1;
            }
            sh = a + c;
        };
        // Prologue: K(kb), K(kb+1), V(kb); QK(kb) once K(kb) has landed.
        issue_k(kb);
        if (kb + 1 < ke) issue_k(kb + 1);
        issue_v(kb);
        if (kb + 1 < ke) {
            WaitVm<2 * G::IPW>();
        } else {
            WaitVm<G::IPW>();
        }
        gsync();
        floatx16 s_cur = qk_slot(kb & 1);
        uint32_t ph_cur[4];
        float sh_cur;
        if (kb >= n_plain) mask(kb, lim, s_cur);
        {
            const float lm = prep(s_cur, ph_cur, sh_cur);
            fix(lm, s_cur, ph_cur, sh_cur);
        }
        WaitVm<0>();
        gsync();  // K(kb) read by every wave before step kb refills its slot
        // Step j (S = j & 1): K(j+2) into K slot S and V(j+1) into V slot S^1 (both read in
        // step j-1), QK(j+1) from K slot S^1, PV(j) from V slot S. The softmax work is split
        // between the two MFMA runs of the step so that each has VALU and transcendental work
        // to hide: under QK(j+1) the second half of tile j's weights; under PV(j) tile j+1's
        // maximum, exponent arguments and first-half weights (with the current maximum; the
        // rare move of the maximum redoes them after PV). The range's last step (LAST) has no
        // next tile: it only finishes tile j's weights and runs PV(j).
        auto step = [&]<int S, bool MASK, bool LAST = false>(
                        int j, floatx16& s_in, uint32_t (&ph_in)[4], float sh_in, floatx16& s_out,
                        uint32_t (&ph_out)[4], float& sh_out) {
            vec8 kf[G::KS];
            if constexpr (!LAST) {
                const uint8_t* base = lds8 + (S ^ 1) * G::TILE_BYTES;
#pragma unroll
                for (int ks = 0; ks < G::KS; ++ks) {
                    kf[ks] = *reinterpret_cast<const vec8*>(base + k_frag[ks]);
                }
            }
            vec8 va[2 * G::DT];
            ReadVFrags<(2 + S) * G::TILE_BYTES, ROW_BYTES>(v_addr, va);
            if (j + 2 < ke) issue_k(j + 2);
            if (j + 1 < ke) issue_v(j + 1);
            uint32_t pw[8];
            {
                float a = 0.0f, c = 0.0f;
#pragma unroll
                for (int i = 4; i < 8; ++i) {
                    const float p0 = fast_exp2(s_in[2 * i]);
                    const float p1 = fast_exp2(s_in[2 * i + 1]);
                    pw[i] = M::pack(p0, p1);
                    a += p0;
                    c += p1;
                }
                rs.l += sh_in + (a + c);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) pw[i] = ph_in[i];
            if constexpr (!LAST) {
                floatx16 acc;
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
#pragma unroll
                for (int ks = 0; ks < G::KS; ++ks) acc = M::mma(kf[ks], qf[ks], acc);
                s_out = acc;
#pragma unroll
                for (int i = 0; i < G::KS; ++i) {
                    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(kSchedValuTrans, 3, 0);
                }
                if constexpr (MASK) mask(j + 1, lim, s_out);
            }
            vec8 pb0 = __builtin_bit_cast(vec8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
            vec8 pb1 = __builtin_bit_cast(vec8, make_uint4(pw[4], pw[5], pw[6], pw[7]));
            WaitLdsTied(va, pb0, pb1);
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
                o[dt] = M::mma(va[2 * dt], pb0, o[dt]);
                o[dt] = M::mma(va[2 * dt + 1], pb1, o[dt]);
            }
            if constexpr (!LAST) {
                const float lm = prep(s_out, ph_out, sh_out);
#pragma unroll
                for (int i = 0; i < 2 * G::DT; ++i) {
                    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(kSchedValuTrans, 6, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
                fix(lm, s_out, ph_out, sh_out);
            }
            WaitVm<0>();
            gsync();
        };
        floatx16 s_next;
        uint32_t ph_next[4];
        float sh_next;
        int j = kb;
        // Steps whose next tile needs no mask, then the rest up to the range's last step; each
        // run alternates the two register sets and slots by the step's parity.
        auto run = [&]<bool MASK>(int j_end) {
            if (j < j_end && (j & 1)) {
                step.template operator()<1, MASK>(j, s_cur, ph_cur, sh_cur, s_next, ph_next, sh_next);
                s_cur = s_next;
#pragma unroll
                for (int i = 0; i < 4; ++i) ph_cur[i] = ph_next[i];
                sh_cur = sh_next;
                ++j;
            }
            for (; j + 2 <= j_end; j += 2) {
                step.template operator()<0, MASK>(j, s_cur, ph_cur, sh_cur, s_next, ph_next, sh_next);
                step.template operator()<1, MASK>(j + 1, s_next, ph_next, sh_next, s_cur, ph_cur, sh_cur);
            }
            if (j < j_end) {
                step.template operator()<0, MASK>(j, s_cur, ph_cur, sh_cur, s_next, ph_next, sh_next);
                s_cur = s_next;
#pragma unroll
                for (int i = 0; i < 4; ++i) ph_cur[i] = ph_next[i];
                sh_cur = sh_next;
                ++j;
            }
        };
        run.template operator()<false>(min(ke, n_plain) - 1);
        run.template operator()<true>(ke - 1);
        if (j & 1) {
            step.template operator()<1, true, true>(j, s_cur, ph_cur, sh_cur, s_next, ph_next, sh_next);
        } else {
            step.template operator()<0, true, true>(j, s_cur, ph_cur, sh_cur, s_next, ph_next, sh_next);
        }
    };
    float4* const mquad = reinterpret_cast<float4*>(lds8);
    if (g == 0) {
        load_q(qa);
        reset_state();
        run_keys(qa, 0, x, plain_a);
    } else {
        if (has_b) {
            load_q(qb);
            reset_state();
            run_keys(qb, 0, n_b, plain_b);
            // B's two key halves meet here: the kq = 1 waves hand their state to kq = 0
            // through group 1's ring (idle now: the last step's barrier retired every read).
            float4* const bq = reinterpret_cast<float4*>(ring);
            float2* const bst = reinterpret_cast<float2*>(bq + 2 * 4 * G::DT * kWave);
            if (kq == 1) {
#pragma unroll
                for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        bq[(rg * 4 * G::DT + 4 * dt + q4) * kWave + lane] =
                            make_float4(o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2],
                                        o[dt][4 * q4 + 3]);
                    }
                }
                bst[rg * kWave + lane] = make_float2(rs.m, rs.l);
            }
            gsync();
            if (kq == 0) {
                const float2 st = bst[rg * kWave + lane];
                const float mm = fmaxf(rs.m, st.x);
                const float w0 = (rs.m == neg_inf()) ? 0.0f : fast_exp2(rs.m - mm);
                const float w1 = (st.x == neg_inf()) ? 0.0f : fast_exp2(st.x - mm);
                const float l_tot = HalfSum(rs.l * w0 + st.y * w1);
                const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
                const int row = qb * BM + rg * 32 + lr;
                const bool row_ok = row < seq_q;
                uint16_t* out_row = static_cast<uint16_t*>(p.out) + b * p.o_sb + h * p.o_sh +
                                    static_cast<int64_t>(row) * p.o_ss;
#pragma unroll
                for (int dt = 0; dt < G::DT; ++dt) {
                    float acc[16];
#pragma unroll
                    for (int q4 = 0; q4 < 4; ++q4) {
                        const float4 v = bq[(rg * 4 * G::DT + 4 * dt + q4) * kWave + lane];
                        acc[4 * q4] = o[dt][4 * q4] * w0 + v.x * w1;
                        acc[4 * q4 + 1] = o[dt][4 * q4 + 1] * w0 + v.y * w1;
                        acc[4 * q4 + 2] = o[dt][4 * q4 + 2] * w0 + v.z * w1;
                        acc[4 * q4 + 3] = o[dt][4 * q4 + 3] * w0 + v.w * w1;
                    }
                    if (row_ok) {
#pragma unroll
                        for (int q4 = 0; q4 < 4; ++q4) {
                            const int d0 = 32 * dt + 8 * q4 + 4 * hh;
                            const uint32_t lo = M::pack(acc[4 * q4] * inv, acc[4 * q4 + 1] * inv);
                            const uint32_t hi = M::pack(acc[4 * q4 + 2] * inv, acc[4 * q4 + 3] * inv);
                            *reinterpret_cast<uint2*>(out_row + d0) = make_uint2(lo, hi);
                        }
                    }
                }
                if (row_ok && p.lse != nullptr && hh == 0) {
                    p.lse[(b * p.num_heads + h) * p.seq_q + row] =
                        l_tot > 0.0f ? (mm + __log2f(l_tot)) * kLn2 : neg_inf();
                }
            }
            gsync();  // the merge buffer is the ring of the next key range
        }
        load_q(qa);
        reset_state();
        run_keys(qa, x, n_a, plain_a);
    }

    // Both groups reach the same barrier count (the counts are uniform per group).
    while (syncs < syncs_all) gsync();

    // A's four states per row group (groups 0 and 1, key halves 0 and 1) merge into the
    // (g = 0, kq = 0) wave of the row group; the other three hand theirs over through LDS.
    __syncthreads();
    float2* const mstat = reinterpret_cast<float2*>(mquad + G::MERGE_QUADS);
    const int src = g * 2 + kq;  // 0 = the merging wave
    if (src != 0) {
        float4* mbuf = mquad + ((rg * 3 + src - 1) * 4 * G::DT) * kWave + lane;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                mbuf[(4 * dt + q4) * kWave] = make_float4(o[dt][4 * q4], o[dt][4 * q4 + 1],
                                                          o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]);
            }
        }
        mstat[(rg * 3 + src - 1) * kWave + lane] = make_float2(rs.m, rs.l);
    }
    __syncthreads();
    if (src == 0) {
        float2 st[3];
#pragma unroll
        for (int q = 0; q < 3; ++q) st[q] = mstat[(rg * 3 + q) * kWave + lane];
        float mm = rs.m;
#pragma unroll
        for (int q = 0; q < 3; ++q) mm = fmaxf(mm, st[q].x);
        float wq[4];
        wq[0] = (rs.m == neg_inf()) ? 0.0f : fast_exp2(rs.m - mm);
        float l = rs.l * wq[0];
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            wq[q + 1] = (st[q].x == neg_inf()) ? 0.0f : fast_exp2(st[q].x - mm);
            l += st[q].y * wq[q + 1];
        }
        const float l_tot = HalfSum(l);
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        const int row = qa * BM + rg * 32 + lr;
        const bool row_ok = row < seq_q;
        uint16_t* out_row = static_cast<uint16_t*>(p.out) + b * p.o_sb + h * p.o_sh +
                            static_cast<int64_t>(row) * p.o_ss;
        const float4* mb = mquad + (rg * 3 * 4 * G::DT) * kWave + lane;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
            float acc[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[i] = o[dt][i] * wq[0];
#pragma unroll
            for (int q = 0; q < 3; ++q) {
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const float4 v = mb[(q * 4 * G::DT + 4 * dt + q4) * kWave];
                    acc[4 * q4] += v.x * wq[q + 1];
                    acc[4 * q4 + 1] += v.y * wq[q + 1];
                    acc[4 * q4 + 2] += v.z * wq[q + 1];
                    acc[4 * q4 + 3] += v.w * wq[q + 1];
                }
            }
            if (row_ok) {
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const int d0 = 32 * dt + 8 * q4 + 4 * hh;
                    const uint32_t lo = M::pack(acc[4 * q4] * inv, acc[4 * q4 + 1] * inv);
                    const uint32_t hi = M::pack(acc[4 * q4 + 2] * inv, acc[4 * q4 + 3] * inv);
                    *reinterpret_cast<uint2*>(out_row + d0) = make_uint2(lo, hi);
                }
            }
        }
        if (row_ok && p.lse != nullptr && hh == 0) {
            p.lse[(b * p.num_heads + h) * p.seq_q + row] =
                l_tot > 0.0f ? (mm + __log2f(l_tot)) * kLn2 : neg_inf();
        }
    }
}

// ============================================================================================
// Wide-row kernel (head_dim 64 and 128): one wave per SIMD and 64 query rows per wave.
//
// Why: the fragment reads from LDS are what bounds the 32-row kernels. Every K fragment (32 keys x
// 16 dims) and every V^T fragment feeds one MFMA per 32 query rows a wave holds, and the
// transposed V reads stream at about half the rate of ds_read_b128. With 64 rows per wave each
// fragment feeds two MFMAs, which halves the LDS bytes per FLOP. 64 rows need about 250 VGPRs
// plus 64 (D = 64) or 128 (D = 128) accumulator registers for O, which only one wave per SIMD
// has; that wave then has to overlap its own VALU work with its MFMAs. It does when O lives in
// AGPRs and the instruction stream alternates one MFMA with a few VALU instructions, so the
// step below is written in an explicit order: every MFMA, fragment read and wait is an inline
// asm statement, the C++ VALU code between them is fenced with sched_barrier, and the data
// hazards the compiler cannot see are covered by waits stated at each use (see the step).
//
// Workgroup: 4 waves = 2 row groups (64 rows each, two 32-row subtiles) x 2 key halves (32 keys
// of every 64-key tile); K and V tiles come by buffer->LDS DMA into rings of four slots each,
// three tiles ahead. The two key halves of a row group are merged through LDS at the end.
// ============================================================================================
template <int D>
struct WideGeom {
    static constexpr int WAVES = 4;
    static constexpr int THREADS = WAVES * kWave;
    static constexpr int RT = 2;                      // 32-row subtiles per wave
    static constexpr int BM = 128;                    // rows per workgroup
    static constexpr int BN = 64;                     // keys per tile
    static constexpr int KS = D / 16;                 // QK k-steps
    static constexpr int DT = D / 32;                 // O^T tiles of 32 dims
    static constexpr int CPR = D / 8;                 // 16-byte chunks per row
    static constexpr int ROW_BYTES = 2 * D;
    static constexpr int TILE_BYTES = BN * ROW_BYTES;
    static constexpr int IPW = BN * CPR / (kWave * WAVES);  // DMA instructions per wave per tile
    static constexpr int SLOTS = 4;
    static constexpr int V_BASE = SLOTS * TILE_BYTES;
    static constexpr int RING_BYTES = 2 * SLOTS * TILE_BYTES;
    // Merge: the two kq = 1 waves' O (RT*DT*16 floats per lane) and (m, l) per subtile.
    static constexpr int MERGE_FLOATS = RT * DT * 16 + 2 * RT;
    static constexpr int MERGE_BYTES = 2 * kWave * MERGE_FLOATS * 4;
    static constexpr int LDS_BYTES = RING_BYTES > MERGE_BYTES ? RING_BYTES : MERGE_BYTES;
    static_assert(IPW >= 1 && BN * CPR == IPW * kWave * WAVES, "tile must split evenly");
    static_assert((SLOTS - 1) * TILE_BYTES + 24 * ROW_BYTES < 65536, "slot offsets are DS immediates");
};

// MFMAs issued from inline asm: S^T accumulators in VGPRs, O^T accumulators in AGPRs.
template <typename E>
struct MfmaAsm;

template <>
struct MfmaAsm<F16> {
    // S^T: A (K fragment) in VGPRs, B (Q fragment) in AGPRs, accumulator in VGPRs.
    template <typename V>
    static __device__ __forceinline__ void first_v(floatx16& c, const V& a, const V& b) {
        asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "a"(b));
    }
    template <typename V>
    static __device__ __forceinline__ void acc_v(floatx16& c, const V& a, const V& b) {
        asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "a"(b));
    }
    template <typename V>
    static __device__ __forceinline__ void acc_a(floatx16& c, const V& a, const V& b) {
        asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    }
};

template <>
struct MfmaAsm<BF16> {
    // S^T: A (K fragment) in VGPRs, B (Q fragment) in AGPRs, accumulator in VGPRs.
    template <typename V>
    static __device__ __forceinline__ void first_v(floatx16& c, const V& a, const V& b) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(c) : "v"(a), "a"(b));
    }
    template <typename V>
    static __device__ __forceinline__ void acc_v(floatx16& c, const V& a, const V& b) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "a"(b));
    }
    template <typename V>
    static __device__ __forceinline__ void acc_a(floatx16& c, const V& a, const V& b) {
        asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    }
};

template <int OFF, typename V>
__device__ __forceinline__ void ReadB128Asm(V& dst, uint32_t addr) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(dst) : "v"(addr), "i"(OFF));
}

// lgkmcnt(N) tied to the register it guards (the asm uses below it cannot move above it).
template <int N, typename V>
__device__ __forceinline__ void WaitLgkmTied(V& reg) {
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(reg) : "i"(N));
}

__device__ __forceinline__ void Fence() { __builtin_amdgcn_sched_barrier(0); }

// Gives a value the AGPR register class (an empty asm with an AGPR in/out operand), so that the
// loop-carried accumulators and Q fragments stay in AGPRs instead of being copied in and out.
template <typename V>
__device__ __forceinline__ void PinAgpr(V& x) {
    asm volatile("" : "+a"(x));
}

// 32 wait states tied to the O accumulators (AGPRs): VALU access to O placed after this waits
// for the last MFMA that wrote O, which the compiler does not track for inline-asm MFMAs.
template <int DT>
__device__ __forceinline__ void SettleO(floatx16 (&o)[2][DT]) {
    if constexpr (DT == 4) {
        asm volatile("s_nop 15\n\ts_nop 15"
                     : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[0][2]), "+a"(o[0][3]), "+a"(o[1][0]),
                       "+a"(o[1][1]), "+a"(o[1][2]), "+a"(o[1][3]));
    } else {
        static_assert(DT == 2, "head_dim 64 or 128");
        asm volatile("s_nop 15\n\ts_nop 15" : "+a"(o[0][0]), "+a"(o[0][1]), "+a"(o[1][0]), "+a"(o[1][1]));
    }
}

template <typename E, int D, bool kCausal, bool kVarlen>
__global__ __launch_bounds__(WideGeom<D>::THREADS, 1) void flash_fwd_wide_kernel(
    const sca_flash_params p, int num_q_tiles, const VarlenArgs vl) {
    using G = WideGeom<D>;
    using M = Mfma<E>;
    using A = MfmaAsm<E>;
    using vec8 = typename E::vec8;
    constexpr int BN = G::BN;
    constexpr int BM = G::BM;
    constexpr int RB = G::ROW_BYTES;

    extern __shared__ __align__(16) uint8_t lds8[];
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    const int lane = tid % kWave;
    const int lr = lane & 31;
    const int hh = lane >> 5;
    const int rg = wave & 1;   // row group: rows 64*rg .. +64 of the row tile
    const int kq = wave >> 1;  // key half: keys 32*kq .. +32 of every key tile

    const int64_t bh_count = p.batch * p.num_heads;
    int64_t tile_linear, bh;
    XcdOrder(p, bh_count, &tile_linear, &bh);
    const int64_t b = bh / p.num_heads;
    const int64_t h = bh % p.num_heads;
    const int64_t h_kv = h / (p.num_heads / p.num_kv_heads);
    // Causal: longest row tiles first. A packed varlen launch takes the sequence and row tile of
    // work entry tile_linear (the list is longest first); tok_*: the sequence's first token.
    int qt = static_cast<int>(kCausal ? (num_q_tiles - 1 - tile_linear) : tile_linear);
    int seq_q = static_cast<int>(p.seq_q);
    int seq_kv = static_cast<int>(p.seq_kv);
    int diag = static_cast<int>(p.diagonal);
    int64_t tok_q = 0, tok_kv = 0;
    if constexpr (kVarlen) {
        const int seq = vl.tiles[2 * tile_linear];
        qt = vl.tiles[2 * tile_linear + 1];
        tok_q = vl.cu_q[seq];
        tok_kv = vl.cu_kv[seq];
        seq_q = vl.cu_q[seq + 1] - static_cast<int>(tok_q);
        seq_kv = vl.cu_kv[seq + 1] - static_cast<int>(tok_kv);
        diag = kCausal ? seq_kv - seq_q : 0;
    }
    const float scale2 = p.scale * kLog2e;
    const float inv_scale2 = 1.0f / scale2;
    const int q0 = qt * BM;
    const int row0 = q0 + 64 * rg + lr;  // row of subtile 0 (subtile 1: +32)

    int n_tiles = (seq_kv + BN - 1) / BN;
    int n_plain = seq_kv / BN;
    if (kCausal) {
        const int last_key = q0 + BM - 1 + diag;
        const int causal_tiles = last_key < 0 ? 0 : last_key / BN + 1;
        if (causal_tiles < n_tiles) n_tiles = causal_tiles;
        const int plain = (q0 + diag + 1) / BN;
        if (plain < n_plain) n_plain = plain;
    }
    if (n_plain > n_tiles) n_plain = n_tiles;

    // ---- Q fragments (B operand of S^T = K Q^T): subtile r, k-step ks ----
    vec8 qf[G::RT][G::KS];
#pragma unroll
    for (int r = 0; r < G::RT; ++r) {
        const int row = row0 + 32 * r;
        const uint16_t* q_row = static_cast<const uint16_t*>(p.q) + b * p.q_sb + h * p.q_sh +
                                (tok_q + row) * p.q_ss + 8 * hh;
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            uint4 raw = make_uint4(0, 0, 0, 0);
            if (row < seq_q) raw = *reinterpret_cast<const uint4*>(q_row + 16 * ks);
            qf[r][ks] = __builtin_bit_cast(vec8, raw);
        }
    }

    // ---- DMA (buffer resources bounded at the sequence's last row) ----
    const uint8_t* k_bytes = reinterpret_cast<const uint8_t*>(
        static_cast<const uint16_t*>(p.k) + b * p.k_sb + h_kv * p.k_sh + tok_kv * p.k_ss);
    const uint8_t* v_bytes = reinterpret_cast<const uint8_t*>(
        static_cast<const uint16_t*>(p.v) + b * p.v_sb + h_kv * p.v_sh + tok_kv * p.v_ss);
    const int k_row_bytes = static_cast<int>(p.k_ss) * 2;
    const int v_row_bytes = static_cast<int>(p.v_ss) * 2;
    const int k_records = (seq_kv - 1) * k_row_bytes + RB;
    const int v_records = (seq_kv - 1) * v_row_bytes + RB;
    uint32_t dma_koff[G::IPW], dma_voff[G::IPW];
#pragma unroll
    for (int i = 0; i < G::IPW; ++i) {
        const int P = (wave * G::IPW + i) * kWave + lane;
        const int row = P / G::CPR;
        const int pos = P % G::CPR;
        dma_koff[i] = row * k_row_bytes + (pos ^ SwzK<D>(row)) * 16;
        dma_voff[i] = row * v_row_bytes + (pos ^ SwzV<D>(row)) * 16;
    }
    auto issue_k = [&](int slot, int t) __attribute__((always_inline)) {
        uint8_t* dst = lds8 + slot * G::TILE_BYTES + wave * G::IPW * 1024;
        const uint32_t off = static_cast<uint32_t>(t * BN * k_row_bytes);
#pragma unroll
        for (int i = 0; i < G::IPW; ++i) DmaToLds(k_bytes, k_records, dst + i * 1024, dma_koff[i], off);
    };
    auto issue_v = [&](int slot, int t) __attribute__((always_inline)) {
        uint8_t* dst = lds8 + G::V_BASE + slot * G::TILE_BYTES + wave * G::IPW * 1024;
        const uint32_t off = static_cast<uint32_t>(t * BN * v_row_bytes);
#pragma unroll
        for (int i = 0; i < G::IPW; ++i) DmaToLds(v_bytes, v_records, dst + i * 1024, dma_voff[i], off);
    };
    // DMA instruction n (of 2*IPW: K's then V's) of the step that fetches K(t + 1) and V(t).
    auto issue_one = [&](int n, int k_slot, int v_slot, int t_k, int t_v) __attribute__((always_inline)) {
        if (n < G::IPW) {
            uint8_t* dst = lds8 + k_slot * G::TILE_BYTES + wave * G::IPW * 1024;
            DmaToLds(k_bytes, k_records, dst + n * 1024, dma_koff[n],
                     static_cast<uint32_t>(t_k * BN * k_row_bytes));
        } else {
            const int i = n - G::IPW;
            uint8_t* dst = lds8 + G::V_BASE + v_slot * G::TILE_BYTES + wave * G::IPW * 1024;
            DmaToLds(v_bytes, v_records, dst + i * 1024, dma_voff[i],
                     static_cast<uint32_t>(t_v * BN * v_row_bytes));
        }
    };

    // ---- fragment addresses (LDS byte addresses of slot 0; slots are immediate offsets) ----
    const uint32_t lds_base = LdsAddr(lds8);
    const int k_row = 32 * kq + lr;
    uint32_t k_addr[G::KS];
#pragma unroll
    for (int ks = 0; ks < G::KS; ++ks) {
        k_addr[ks] = lds_base + k_row * RB + (((2 * ks) ^ hh ^ SwzK<D>(k_row)) * 16);
    }
    const int grp = lane >> 4;
    const int sl = lane & 15;
    const int v_key = 32 * kq + 4 * hh + (sl >> 2);
    const int v_chunk = 2 * (grp & 1) + ((sl & 3) >> 1);
    const int v_half = (sl & 1) * 8;
    uint32_t v_addr[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt) {
        v_addr[dt] = lds_base + G::V_BASE + v_key * RB +
                     (((4 * dt + v_chunk) ^ SwzV<D>(v_key)) * 16) + v_half;
    }

    floatx16 o[G::RT][G::DT];
#pragma unroll
    for (int r = 0; r < G::RT; ++r) {
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
            for (int i = 0; i < 16; ++i) o[r][dt][i] = 0.0f;
            PinAgpr(o[r][dt]);
        }
    }
#pragma unroll
    for (int r = 0; r < G::RT; ++r) {
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) PinAgpr(qf[r][ks]);
    }
    // Row state (RowState); the denominator is summed in two halves (rs.l and l2), which keeps
    // the two dependency chains of its additions apart.
    RowState rs[G::RT];
    float l2[G::RT];
#pragma unroll
    for (int r = 0; r < G::RT; ++r) {
        ResetRow(rs[r]);
        l2[r] = 0.0f;
    }

    // K fragments of the next key tile, and two V^T fragment buffers (tile parity).
    vec8 kf[G::KS];
    vec8 va[2][2 * G::DT];
    auto read_k = [&]<int SLOT>() __attribute__((always_inline)) {
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) ReadB128Asm<SLOT * G::TILE_BYTES>(kf[ks], k_addr[ks]);
    };
    // Transposed V read i (of 4*DT) of the V tile in slot SLOT into buffer VB.
    auto read_v1 = [&]<int SLOT, int VB>(int i) __attribute__((always_inline)) {
        const int dt = i / 4;
        const int part = i % 4;
        uint2 r;
        switch (part) {
            case 0: r = TrReadAsm<SLOT * G::TILE_BYTES>(v_addr[dt]); break;
            case 1: r = TrReadAsm<SLOT * G::TILE_BYTES + 8 * RB>(v_addr[dt]); break;
            case 2: r = TrReadAsm<SLOT * G::TILE_BYTES + 16 * RB>(v_addr[dt]); break;
            default: r = TrReadAsm<SLOT * G::TILE_BYTES + 24 * RB>(v_addr[dt]); break;
        }
        // fragment 2*dt + ps holds (rows 16*ps, 16*ps + 8) of the lane's V column
        uint4 w = __builtin_bit_cast(uint4, va[VB][2 * dt + part / 2]);
        if (part % 2 == 0) {
            w.x = r.x;
            w.y = r.y;
        } else {
            w.z = r.x;
            w.w = r.y;
        }
        va[VB][2 * dt + part / 2] = __builtin_bit_cast(vec8, w);
    };

    // Masking of S^T subtile r of key tile t (uniform `masked`), and the lane's local maximum.
    auto mask_max = [&](floatx16& sr, int r, int t, bool masked) __attribute__((always_inline)) -> float {
        if (masked) {
            const int kbase = t * BN + 32 * kq + 4 * hh;
            const int lim = kCausal ? min(seq_kv - 1, row0 + 32 * r + diag) : seq_kv - 1;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kbase + 8 * (i / 4) + (i % 4);
                sr[i] = key > lim ? neg_inf() : sr[i];
            }
        }
        return Max16(sr);
    };
    // The rare rescale of both subtiles for a new key tile with raw lane maxima lm (RowState).
    auto rescale_if_grown = [&](float lm0, float lm1) __attribute__((always_inline)) {
        if (__builtin_amdgcn_ballot_w64((lm0 > rs[0].thr) || (lm1 > rs[1].thr)) == 0) return;
        SettleO(o);
        const float lmv[2] = {lm0, lm1};
#pragma unroll
        for (int r = 0; r < G::RT; ++r) {
            const float cmax = HalfMax(lmv[r]) * scale2;  // row maximum, log2 units
            const bool grow = cmax > rs[r].m + kRescaleSlack;
            const float m_new = grow ? cmax : rs[r].m;
            const float alpha = grow ? fast_exp2(rs[r].m - m_new) : 1.0f;  // 0 when m was -inf
            rs[r].m = m_new;
            rs[r].l *= alpha;
            l2[r] *= alpha;
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
                Fence();  // one O tile at a time through VGPRs
#pragma unroll
                for (int i = 0; i < 16; ++i) o[r][dt][i] *= alpha;
                PinAgpr(o[r][dt]);
            }
            Fence();
            rs[r].thr = (m_new + kRescaleSlack) * inv_scale2;
            rs[r].neg_mu = (m_new == neg_inf()) ? 0.0f : -m_new;
        }
        asm volatile("s_nop 4");
    };

    // ---- prologue: K(0..3), V(0..2) in flight; S(0), its maxima and rescale; K(1) and V(0)
    //      fragments read for step 0; K(2) and V(1) landed before step 0 ----
    issue_k(0, 0);
    issue_k(1, 1);
    issue_v(0, 0);
    issue_k(2, 2);
    issue_v(1, 1);
    issue_k(3, 3);
    issue_v(2, 2);
    WaitVm<4 * G::IPW>();  // K(0), K(1), V(0)
    __builtin_amdgcn_s_barrier();
    floatx16 s0[G::RT], s1[G::RT];
    read_k.template operator()<0>();
    WaitLgkmTied<0>(kf[0]);
#pragma unroll
    for (int ks = 1; ks < G::KS; ++ks) WaitLgkmTied<0>(kf[ks]);
#pragma unroll
    for (int r = 0; r < G::RT; ++r) {
        A::first_v(s0[r], kf[0], qf[r][0]);
#pragma unroll
        for (int ks = 1; ks < G::KS; ++ks) A::acc_v(s0[r], kf[ks], qf[r][ks]);
    }
    asm volatile("s_nop 15\n\ts_nop 15");  // the QK results are complete; kf has been read
    {
        const float lm0 = mask_max(s0[0], 0, 0, n_plain == 0);
        const float lm1 = mask_max(s0[1], 1, 0, n_plain == 0);
        rescale_if_grown(lm0, lm1);
    }
    read_k.template operator()<1>();
#pragma unroll
    for (int i = 0; i < 4 * G::DT; ++i) read_v1.template operator()<0, 0>(i);
    WaitVm<2 * G::IPW>();  // K(2), V(1)
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();

    // One step for key tile j (S = j & 3, VB = j & 1). On entry S(j) is masked and the rescale
    // for tile j is done, kf holds K(j+1)'s fragments and va[VB] V(j)'s. Four regions, each one
    // MFMA stream with VALU and LDS work placed between its MFMAs:
    //   A  QK(j+1) of subtile 0          | the 8 exponential pairs of S(j) subtile 0
    //   B  PV(j) of subtile 0            | exponential pairs 0-3 of subtile 1, V(j+1)'s reads
    //   C  QK(j+1) of subtile 1          | exponential pairs 4-7 of subtile 1, S(j+1) subtile 0's
    //                                      masking and maximum
    //   D  PV(j) of subtile 1            | S(j+1) subtile 1's masking and maximum, K(j+2)'s
    //                                      fragment reads, the DMAs of K(j+4) and V(j+3)
    // then the rare rescale for tile j+1, the DMA wait (K(j+3) and V(j+2) must land: only the
    // two groups issued in this step stay in flight) and the barrier. Hazards the compiler
    // does not see (inline-asm MFMAs): a QK result is read by VALU only after at least two
    // later MFMAs and 5 wait states; kf is rewritten only after two later MFMAs; the O
    // accumulators are read by VALU only through SettleO; P operands are written by VALU at
    // least a region before their MFMAs.
    auto step = [&]<bool kMaskable, int S>(int j, floatx16 (&s_in)[G::RT],
                                           floatx16 (&s_out)[G::RT]) __attribute__((always_inline)) {
        constexpr int VB = S & 1;
        constexpr int NPV = 2 * G::DT;  // PV MFMAs per subtile
        const bool next_ok = !kMaskable || j + 1 < n_tiles;   // S(j+1) is a real tile
        const bool next_masked = kMaskable && j + 1 >= n_plain;
        uint32_t pw[G::RT][8];
        // The 56 VALU operations that turn S(j) subtile r into P: 16 exponent arguments
        // s * scale2 - m (codes 0-15), 16 exponentials (16-31), 8 packs to the input dtype
        // (32-39) and 16 additions of the fp32 weights into the two denominator halves (40-55),
        // all in place; op(r, n) runs the n-th in the order of kOps, which keeps each result at
        // least two operations from its first use. (The sums use v_add: a v_dot2 issued between
        // MFMAs does not overlap with them.)
        auto op = [&](int r, int n) __attribute__((always_inline)) {
            constexpr int kOps[56] = {0,  1,  2,  3,  16, 17, 4,  5,  18, 19, 6,  7,  20, 21,
                                      32, 33, 8,  9,  22, 23, 34, 10, 11, 24, 25, 35, 40, 41,
                                      12, 13, 26, 27, 36, 42, 43, 14, 15, 28, 29, 37, 44, 45,
                                      30, 31, 46, 47, 38, 39, 48, 49, 50, 51, 52, 53, 54, 55};
            const int c = kOps[n];
            if (c < 16) {
                s_in[r][c] = fmaf(s_in[r][c], scale2, rs[r].neg_mu);
            } else if (c < 32) {
                s_in[r][c - 16] = fast_exp2(s_in[r][c - 16]);
            } else if (c < 40) {
                pw[r][c - 32] = M::pack(s_in[r][2 * (c - 32)], s_in[r][2 * (c - 32) + 1]);
            } else if (c % 2 == 0) {
                rs[r].l += s_in[r][c - 40];
            } else {
                l2[r] += s_in[r][c - 40];
            }
        };
        auto qk = [&](int r, int ks) __attribute__((always_inline)) {
            if (!next_ok) return;  // the last tile has no S(j+1)
            if (ks == 0) {
                A::first_v(s_out[r], kf[0], qf[r][0]);
            } else {
                A::acc_v(s_out[r], kf[ks], qf[r][ks]);
            }
        };
        vec8 pb[G::RT][2];
        auto pack_p = [&](int r) __attribute__((always_inline)) {
            pb[r][0] = __builtin_bit_cast(vec8, make_uint4(pw[r][0], pw[r][1], pw[r][2], pw[r][3]));
            pb[r][1] = __builtin_bit_cast(vec8, make_uint4(pw[r][4], pw[r][5], pw[r][6], pw[r][7]));
        };
        auto pv = [&](int r, int i) __attribute__((always_inline)) {
            A::acc_a(o[r][i / 2], va[VB][i], pb[r][i % 2]);
        };
        // The step's 2*IPW DMA instructions (K(j+4) into K slot S, V(j+3) into V slot S-1),
        // spread over the four regions: in region g, after MFMA i, instruction number
        // g*kDmaPerRegion + i / kDmaSpacing when i is a multiple of kDmaSpacing.
        constexpr int kDmaPerRegion = (2 * G::IPW + 3) / 4;
        auto dma = [&](int g, int i) __attribute__((always_inline)) {
            constexpr int kSpacing = 8 / kDmaPerRegion > 0 ? 8 / kDmaPerRegion : 1;
            if (i % kSpacing != 0) return;
            const int n = g * kDmaPerRegion + i / kSpacing;
            if (n >= 2 * G::IPW || i / kSpacing >= kDmaPerRegion) return;
            const bool is_k = n < G::IPW;
            if (kMaskable && (is_k ? j + 4 >= n_tiles : j + 3 >= n_tiles)) return;
            issue_one(n, S, (S + 3) & 3, j + 4, j + 3);
        };

        // ---- A ----
        constexpr int kOpsA = 56 / G::KS;  // VALU operations per QK MFMA
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            qk(0, ks);
            Fence();
#pragma unroll
            for (int q = 0; q < kOpsA; ++q) op(0, ks * kOpsA + q);
            dma(0, ks);
            Fence();
        }
        pack_p(0);
        // P operands: 2 wait states after their VALU writes (the compiler does not see the
        // inline-asm MFMA that reads them).
        asm volatile("s_nop 1" : "+v"(pb[0][0]), "+v"(pb[0][1]));
        // ---- B ----
        constexpr int kVReadsB = 4 * G::DT / NPV;  // V reads per PV MFMA
        constexpr int kOpsB = (28 + NPV - 1) / NPV;  // subtile 1's operations 0-27
#pragma unroll
        for (int i = 0; i < NPV; ++i) {
            pv(0, i);
            Fence();
#pragma unroll
            for (int q = 0; q < kOpsB; ++q) {
                if (i * kOpsB + q < 28) op(1, i * kOpsB + q);
            }
            dma(1, i);
#pragma unroll
            for (int q = 0; q < kVReadsB; ++q) {
                read_v1.template operator()<(S + 1) & 3, VB ^ 1>(i * kVReadsB + q);
            }
            Fence();
        }
        // ---- C ----
        float lm0 = neg_inf(), lm1 = neg_inf();
        constexpr int kOpsC = (28 + G::KS - 1) / G::KS;  // subtile 1's operations 28-55
#pragma unroll
        for (int ks = 0; ks < G::KS; ++ks) {
            qk(1, ks);
            Fence();
#pragma unroll
            for (int q = 0; q < kOpsC; ++q) {
                if (ks * kOpsC + q < 28) op(1, 28 + ks * kOpsC + q);
            }
            dma(2, ks);
            if (ks == G::KS / 2) {
                if (next_ok) lm0 = mask_max(s_out[0], 0, j + 1, next_masked);
            }
            Fence();
        }
        pack_p(1);
        // P operands: 2 wait states after their VALU writes.
        asm volatile("s_nop 1" : "+v"(pb[1][0]), "+v"(pb[1][1]));
        // ---- D ----
#pragma unroll
        for (int i = 0; i < NPV; ++i) {
            pv(1, i);
            Fence();
            if (i == 1) {
                asm volatile("s_nop 4");
                if (next_ok) lm1 = mask_max(s_out[1], 1, j + 1, next_masked);
            }
            if (i >= 1) {
                // KS K reads over the MFMAs 1 .. NPV-1 (kf was last read two MFMAs ago).
                constexpr int kPer = (G::KS + NPV - 2) / (NPV - 1);
#pragma unroll
                for (int q = 0; q < kPer; ++q) {
                    const int ks = (i - 1) * kPer + q;
                    if (ks < G::KS) {
                        switch (ks) {
                            case 0: ReadB128Asm<((S + 2) & 3) * G::TILE_BYTES>(kf[0], k_addr[0]); break;
                            case 1: ReadB128Asm<((S + 2) & 3) * G::TILE_BYTES>(kf[1], k_addr[1]); break;
                            case 2: ReadB128Asm<((S + 2) & 3) * G::TILE_BYTES>(kf[2], k_addr[2]); break;
                            case 3: ReadB128Asm<((S + 2) & 3) * G::TILE_BYTES>(kf[3], k_addr[3]); break;
                            case 4: ReadB128Asm<((S + 2) & 3) * G::TILE_BYTES>(kf[4 % G::KS], k_addr[4 % G::KS]); break;
                            case 5: ReadB128Asm<((S + 2) & 3) * G::TILE_BYTES>(kf[5 % G::KS], k_addr[5 % G::KS]); break;
                            case 6: ReadB128Asm<((S + 2) & 3) * G::TILE_BYTES>(kf[6 % G::KS], k_addr[6 % G::KS]); break;
                            default: ReadB128Asm<((S + 2) & 3) * G::TILE_BYTES>(kf[7 % G::KS], k_addr[7 % G::KS]); break;
                        }
                    }
                }
            }
            dma(3, i);
            Fence();
        }
        // ---- rare rescale for tile j+1 ----
        if (next_ok) rescale_if_grown(lm0, lm1);
        Fence();
        // ---- K(j+3) and V(j+2) landed (at the tail, everything); fragment reads retired ----
        if (!kMaskable || j + 4 < n_tiles) {
            WaitVm<2 * G::IPW>();
        } else {
            WaitVm<0>();
        }
        WaitLgkmTied<0>(kf[G::KS - 1]);
        __builtin_amdgcn_s_barrier();
    };

    int j = 0;
    // Steady state: plain tiles with the full ring ahead, four steps per trip.
    for (; j + 5 <= n_plain && j + 8 <= n_tiles; j += 4) {
        step.template operator()<false, 0>(j, s0, s1);
        step.template operator()<false, 1>(j + 1, s1, s0);
        step.template operator()<false, 2>(j + 2, s0, s1);
        step.template operator()<false, 3>(j + 3, s1, s0);
    }
    // Tail (j is a multiple of 4 here): masked steps, same slot rotation.
    for (; j < n_tiles; j += 4) {
        step.template operator()<true, 0>(j, s0, s1);
        if (j + 1 >= n_tiles) break;
        step.template operator()<true, 1>(j + 1, s1, s0);
        if (j + 2 >= n_tiles) break;
        step.template operator()<true, 2>(j + 2, s0, s1);
        if (j + 3 >= n_tiles) break;
        step.template operator()<true, 3>(j + 3, s1, s0);
    }

    // ---- epilogue: merge the key halves of each row group, normalise, store ----
    WaitVm<0>();
    SettleO(o);
    __builtin_amdgcn_s_barrier();
    float* const mbuf = reinterpret_cast<float*>(lds8) + rg * kWave * G::MERGE_FLOATS;
    if (kq == 1) {
        // O as quads, quad k of lane L at k*64 + L (conflict-free 16-byte accesses).
        float4* q4 = reinterpret_cast<float4*>(mbuf) + lane;
#pragma unroll
        for (int r = 0; r < G::RT; ++r) {
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    q4[((r * G::DT + dt) * 4 + g) * kWave] =
                        make_float4(o[r][dt][4 * g], o[r][dt][4 * g + 1], o[r][dt][4 * g + 2],
                                    o[r][dt][4 * g + 3]);
                }
            }
        }
        float2* st = reinterpret_cast<float2*>(mbuf + G::RT * G::DT * 16 * kWave) + lane;
#pragma unroll
        for (int r = 0; r < G::RT; ++r) st[r * kWave] = make_float2(rs[r].m, rs[r].l + l2[r]);
    }
    __syncthreads();
    if (kq == 1) return;

    const float4* q4 = reinterpret_cast<const float4*>(mbuf) + lane;
    const float2* st = reinterpret_cast<const float2*>(mbuf + G::RT * G::DT * 16 * kWave) + lane;
#pragma unroll
    for (int r = 0; r < G::RT; ++r) {
        const float2 other = st[r * kWave];
        const float mm = fmaxf(rs[r].m, other.x);
        const float w0 = (rs[r].m == neg_inf()) ? 0.0f : fast_exp2(rs[r].m - mm);
        const float w1 = (other.x == neg_inf()) ? 0.0f : fast_exp2(other.x - mm);
        const float l_tot = HalfSum((rs[r].l + l2[r]) * w0) + HalfSum(other.y * w1);
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        const int row = row0 + 32 * r;
        const bool row_ok = row < seq_q;
        uint16_t* out_row = static_cast<uint16_t*>(p.out) + b * p.o_sb + h * p.o_sh +
                            (tok_q + row) * p.o_ss;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const float4 v = q4[((r * G::DT + dt) * 4 + g) * kWave];
                const float a0 = (o[r][dt][4 * g] * w0 + v.x * w1) * inv;
                const float a1 = (o[r][dt][4 * g + 1] * w0 + v.y * w1) * inv;
                const float a2 = (o[r][dt][4 * g + 2] * w0 + v.z * w1) * inv;
                const float a3 = (o[r][dt][4 * g + 3] * w0 + v.w * w1) * inv;
                if (row_ok) {
                    const int d0 = 32 * dt + 8 * g + 4 * hh;
                    *reinterpret_cast<uint2*>(out_row + d0) =
                        make_uint2(M::pack(a0, a1), M::pack(a2, a3));
                }
            }
        }
        if (row_ok && p.lse != nullptr && hh == 0) {
            p.lse[(b * p.num_heads + h) * p.seq_q + row] =
                l_tot > 0.0f ? (mm + __log2f(l_tot)) * kLn2 : neg_inf();
        }
    }
}

template <typename E, int D, bool kCausal>
int LaunchFlash(const sca_flash_params& p, hipStream_t s);

template <typename E, int D, bool kCausal>
int LaunchFlashWide(const sca_flash_params& p, hipStream_t s) {
    using G = WideGeom<D>;
    // Buffer offsets are 32-bit: rows up to seq_kv plus the ring's overrun must fit.
    const int64_t extent_k = (p.seq_kv + 8 * G::BN) * p.k_ss * 2;
    const int64_t extent_v = (p.seq_kv + 8 * G::BN) * p.v_ss * 2;
    if (extent_k >= (1LL << 31) || extent_v >= (1LL << 31)) return LaunchFlash<E, D, kCausal>(p, s);
    const int64_t num_q_tiles = (p.seq_q + G::BM - 1) / G::BM;
    const int64_t blocks = num_q_tiles * p.batch * p.num_heads;
    if (blocks <= 0) return 0;
    if (blocks > 0x7fffffffLL) {
        return SetError(SCA_E_SEQ_TOO_LONG, "flash: grid of " + std::to_string(blocks) +
                                                " workgroups exceeds the launch limit");
    }
    if (const int rc =
            EnsureLdsLimit<&flash_fwd_wide_kernel<E, D, kCausal, false>>(G::LDS_BYTES, "flash LDS limit")) {
        return rc;
    }
    hipLaunchKernelGGL((flash_fwd_wide_kernel<E, D, kCausal, false>),
                       dim3(static_cast<unsigned>(blocks)), dim3(G::THREADS), G::LDS_BYTES, s, p,
                       static_cast<int>(num_q_tiles), VarlenArgs{nullptr, nullptr, nullptr});
    return CheckLaunch("flash_fwd_wide_kernel", s);
}

template <typename E, int D, bool kCausal>
int LaunchFlash(const sca_flash_params& p, hipStream_t s);

template <typename E, int D, bool kCausal>
int LaunchFlash(const sca_flash_params& p, hipStream_t s) {
    using G = FlashGeom<D>;
    const int64_t num_q_tiles = (p.seq_q + kBlockM - 1) / kBlockM;
    const int64_t blocks = num_q_tiles * p.batch * p.num_heads;
    if (blocks <= 0) return 0;
    if (blocks > 0x7fffffffLL) {
        return SetError(SCA_E_SEQ_TOO_LONG, "flash: grid of " + std::to_string(blocks) +
                                                " workgroups exceeds the launch limit");
    }
    if (const int rc =
            EnsureLdsLimit<&flash_fwd_kernel<E, D, kCausal>>(G::LDS_BYTES, "flash LDS limit")) {
        return rc;
    }
    hipLaunchKernelGGL((flash_fwd_kernel<E, D, kCausal>), dim3(static_cast<unsigned>(blocks)),
                       dim3(G::THREADS), G::LDS_BYTES, s, p, static_cast<int>(num_q_tiles));
    return CheckLaunch("flash_fwd_kernel", s);
}

template <typename E, int D>
int LaunchFlashPair(const sca_flash_params& p, hipStream_t s) {
    using G = PairGeom<D>;
    const int64_t extent_k = (p.seq_kv + 4 * G::BN) * p.k_ss * 2;
    const int64_t extent_v = (p.seq_kv + 4 * G::BN) * p.v_ss * 2;
    if (extent_k >= (1LL << 31) || extent_v >= (1LL << 31)) return LaunchFlash<E, D, true>(p, s);
    const int64_t num_q_tiles = (p.seq_q + G::BM - 1) / G::BM;
    const int64_t blocks = (num_q_tiles + 1) / 2 * p.batch * p.num_heads;
    if (blocks <= 0) return 0;
    if (blocks > 0x7fffffffLL) {
        return SetError(SCA_E_SEQ_TOO_LONG, "flash: grid of " + std::to_string(blocks) +
                                                " workgroups exceeds the launch limit");
    }
    if (const int rc =
            EnsureLdsLimit<&flash_fwd_pair_kernel<E, D>>(G::LDS_BYTES, "flash LDS limit")) {
        return rc;
    }
    hipLaunchKernelGGL((flash_fwd_pair_kernel<E, D>), dim3(static_cast<unsigned>(blocks)),
                       dim3(G::THREADS), G::LDS_BYTES, s, p, static_cast<int>(num_q_tiles));
    return CheckLaunch("flash_fwd_pair_kernel", s);
}

// Causal grids with at most one 128-row tile per CU run the pair kernel (64-row tiles in
// complementary pairs, so every workgroup holds the same share of the triangle); larger causal
// grids and every non-causal grid run the wide kernel (longest tiles first when causal). Measured
// warm: at 320-448 tiles on 256 CUs the longest-first 128-row grid is 20-30% faster than a
// second partial wave of pairs; at 256 tiles the pairs are 30% faster.
bool UsePairs(const sca_flash_params& p) {
    static int cu_count = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
            (void)hipGetLastError();
            n = 256;
        }
        return n > 0 ? n : 256;
    }();
    const int64_t tiles128 = (p.seq_q + 127) / 128 * p.batch * p.num_heads;
    return tiles128 <= static_cast<int64_t>(cu_count);
}

template <typename E, bool kCausal>
int LaunchForDim(const sca_flash_params& p, hipStream_t s) {
    switch (p.head_dim) {
        case 32: return LaunchFlash<E, 32, kCausal>(p, s);
        case 64:
            if (kCausal && UsePairs(p)) return LaunchFlashPair<E, 64>(p, s);
            return LaunchFlashWide<E, 64, kCausal>(p, s);
        case 96: return LaunchFlash<E, 96, kCausal>(p, s);
        case 128:
            if (kCausal && UsePairs(p)) return LaunchFlashPair<E, 128>(p, s);
            return LaunchFlashWide<E, 128, kCausal>(p, s);
        case 160: return LaunchFlash<E, 160, kCausal>(p, s);
        case 192: return LaunchFlash<E, 192, kCausal>(p, s);
        case 256: return LaunchFlash<E, 256, kCausal>(p, s);
        default: break;
    }
    return SetError(SCA_E_UNSUPPORTED_HEAD_DIM,
                    "flash: head_dim=" + std::to_string(p.head_dim) + " is not instantiated");
}

bool Aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

// One launch over a packed batch: the wide kernel, one workgroup per (work entry, head).
template <typename E, int D, bool kCausal>
int LaunchFlashVarlen(const sca_flash_varlen_params& v, hipStream_t s) {
    using G = WideGeom<D>;
    static_assert(G::BM == 128, "the work list's row tiles are 128 rows");
    // 32-bit buffer offsets: a sequence's rows plus the wide kernel's ring overrun must fit.
    const int64_t rows_k = v.max_seq_kv + 8 * G::BN;
    if (rows_k * v.k_ss * 2 >= (1LL << 31) || rows_k * v.v_ss * 2 >= (1LL << 31)) {
        return SetError(SCA_E_SEQ_TOO_LONG, "flash varlen: a sequence of " +
                                                std::to_string(v.max_seq_kv) +
                                                " keys exceeds the 32-bit tile offsets");
    }
    const int64_t blocks = v.num_tiles * v.num_heads;
    if (blocks <= 0) return 0;
    if (blocks > 0x7fffffffLL) {
        return SetError(SCA_E_SEQ_TOO_LONG, "flash varlen: grid too large");
    }
    sca_flash_params p{};
    p.q = v.q;
    p.k = v.k;
    p.v = v.v;
    p.out = v.out;
    p.lse = nullptr;
    p.batch = 1;
    p.num_heads = v.num_heads;
    p.num_kv_heads = v.num_kv_heads;
    p.head_dim = v.head_dim;
    p.q_sh = v.q_sh, p.q_ss = v.q_ss;
    p.k_sh = v.k_sh, p.k_ss = v.k_ss;
    p.v_sh = v.v_sh, p.v_ss = v.v_ss;
    p.o_sh = v.o_sh, p.o_ss = v.o_ss;
    p.scale = v.scale;
    p.causal = v.causal;
    p.dtype = v.dtype;
    if (const int rc = EnsureLdsLimit<&flash_fwd_wide_kernel<E, D, kCausal, true>>(
            G::LDS_BYTES, "flash LDS limit")) {
        return rc;
    }
    hipLaunchKernelGGL((flash_fwd_wide_kernel<E, D, kCausal, true>),
                       dim3(static_cast<unsigned>(blocks)), dim3(G::THREADS), G::LDS_BYTES, s, p,
                       0, VarlenArgs{v.cu_seqlens_q, v.cu_seqlens_kv, v.tiles});
    return CheckLaunch("flash_fwd_wide_kernel (varlen)", s);
}

template <typename E>
int LaunchVarlenTyped(const sca_flash_varlen_params& v, hipStream_t s) {
    if (v.head_dim == 64) {
        return v.causal ? LaunchFlashVarlen<E, 64, true>(v, s) : LaunchFlashVarlen<E, 64, false>(v, s);
    }
    return v.causal ? LaunchFlashVarlen<E, 128, true>(v, s) : LaunchFlashVarlen<E, 128, false>(v, s);
}



int LdsBytesFor(int64_t head_dim) {
    switch (head_dim) {
        case 32: return FlashGeom<32>::LDS_BYTES;
        case 64: return std::max(WideGeom<64>::LDS_BYTES, PairGeom<64>::LDS_BYTES);
        case 96: return FlashGeom<96>::LDS_BYTES;
        case 128: return std::max(WideGeom<128>::LDS_BYTES, PairGeom<128>::LDS_BYTES);
        case 160: return FlashGeom<160>::LDS_BYTES;
        case 192: return FlashGeom<192>::LDS_BYTES;
        case 256: return FlashGeom<256>::LDS_BYTES;
        default: return -1;
    }
}

}  // namespace
}  // namespace sca_hip

using sca_hip::SetError;

extern "C" {

int64_t sca_hip_flash_lds_bytes(int32_t head_dim, int64_t elem_bytes) {
    if (elem_bytes != 2) return -1;
    return sca_hip::LdsBytesFor(head_dim);
}

int sca_hip_flash_tile(int32_t head_dim, int32_t* block_m, int32_t* block_n, int32_t* waves,
                       int32_t* stages) {
    if (sca_hip::LdsBytesFor(head_dim) < 0) {
        return SetError(SCA_E_UNSUPPORTED_HEAD_DIM,
                        "flash: no tile for head_dim=" + std::to_string(head_dim));
    }
    // D = 64 / 128 report the wide kernel (every non-causal and every large causal grid); the
    // other head dims the register-staged one.
    const bool wide = head_dim == 64 || head_dim == 128;
    int32_t bn = 0, nw = 0, ns = 0;
    switch (head_dim) {
        case 32: bn = sca_hip::FlashGeom<32>::BN; nw = sca_hip::FlashGeom<32>::WAVES;
                 ns = sca_hip::FlashGeom<32>::STAGES; break;
        case 96: bn = sca_hip::FlashGeom<96>::BN; nw = sca_hip::FlashGeom<96>::WAVES;
                 ns = sca_hip::FlashGeom<96>::STAGES; break;
        case 160: bn = sca_hip::FlashGeom<160>::BN; nw = sca_hip::FlashGeom<160>::WAVES;
                  ns = sca_hip::FlashGeom<160>::STAGES; break;
        case 192: bn = sca_hip::FlashGeom<192>::BN; nw = sca_hip::FlashGeom<192>::WAVES;
                  ns = sca_hip::FlashGeom<192>::STAGES; break;
        case 256: bn = sca_hip::FlashGeom<256>::BN; nw = sca_hip::FlashGeom<256>::WAVES;
                  ns = sca_hip::FlashGeom<256>::STAGES; break;
        default: break;
    }
    if (wide) {
        bn = sca_hip::WideGeom<64>::BN;
        nw = sca_hip::WideGeom<64>::WAVES;
        ns = sca_hip::WideGeom<64>::SLOTS;
    }
    if (block_m != nullptr) *block_m = sca_hip::kBlockM;
    if (block_n != nullptr) *block_n = bn;
    if (waves != nullptr) *waves = nw;
    if (stages != nullptr) *stages = ns;
    return 0;
}

int sca_hip_flash_varlen_supported(int32_t head_dim) { return head_dim == 64 || head_dim == 128; }

int64_t sca_hip_flash_varlen_tiles(const int32_t* cu_q, const int32_t* cu_kv, int64_t num_seqs,
                                   int32_t causal, int32_t* tiles_out) {
    if (cu_q == nullptr || cu_kv == nullptr || num_seqs < 1) {
        return -SetError(SCA_E_SHAPE_MISMATCH, "flash varlen: null cu_seqlens or no sequences");
    }
    constexpr int64_t kRows = 128;  // rows per workgroup of the varlen launch
    struct Tile {
        int64_t keys;
        int32_t seq;
        int32_t tile;
    };
    std::vector<Tile> tiles;
    for (int64_t s = 0; s < num_seqs; ++s) {
        const int64_t sq = static_cast<int64_t>(cu_q[s + 1]) - cu_q[s];
        const int64_t skv = static_cast<int64_t>(cu_kv[s + 1]) - cu_kv[s];
        if (sq < 0 || skv < 0 || (causal && skv < sq) || (sq > 0 && skv == 0)) {
            return -SetError(SCA_E_SHAPE_MISMATCH,
                             "flash varlen: sequence " + std::to_string(s) + " has S_q=" +
                                 std::to_string(sq) + ", S_kv=" + std::to_string(skv));
        }
        for (int64_t t = 0; t * kRows < sq; ++t) {
            const int64_t last = std::min(sq, (t + 1) * kRows) - 1 + (skv - sq);
            const int64_t keys = causal ? std::min(skv, last + 1) : skv;
            tiles.push_back({keys, static_cast<int32_t>(s), static_cast<int32_t>(t)});
        }
    }
    std::stable_sort(tiles.begin(), tiles.end(),
                     [](const Tile& a, const Tile& b) { return a.keys > b.keys; });
    if (tiles_out != nullptr) {
        for (size_t i = 0; i < tiles.size(); ++i) {
            tiles_out[2 * i] = tiles[i].seq;
            tiles_out[2 * i + 1] = tiles[i].tile;
        }
    }
    return static_cast<int64_t>(tiles.size());
}

int sca_hip_flash_fwd_varlen(const sca_flash_varlen_params* v, void* stream) {
    if (v == nullptr || v->q == nullptr || v->k == nullptr || v->v == nullptr ||
        v->out == nullptr || v->cu_seqlens_q == nullptr || v->cu_seqlens_kv == nullptr ||
        (v->num_tiles > 0 && v->tiles == nullptr)) {
        return SetError(SCA_E_SHAPE_MISMATCH, "flash varlen: null pointer");
    }
    if (!sca_hip_flash_varlen_supported(static_cast<int32_t>(v->head_dim))) {
        return SetError(SCA_E_UNSUPPORTED_HEAD_DIM,
                        "flash varlen: head_dim=" + std::to_string(v->head_dim) +
                            " has no one-launch kernel (64 and 128 do)");
    }
    if (v->dtype != SCA_DTYPE_F16 && v->dtype != SCA_DTYPE_BF16) {
        return SetError(SCA_E_UNSUPPORTED_DTYPE, "flash varlen: fp16/bf16 only");
    }
    if (v->num_heads < 1 || v->num_kv_heads < 1 || v->num_heads % v->num_kv_heads != 0 ||
        v->num_tiles < 0 || v->max_seq_kv < 0 || v->num_seqs < 1) {
        return SetError(SCA_E_SHAPE_MISMATCH, "flash varlen: invalid heads or counts");
    }
    if (!sca_hip::Aligned16(v->q) || !sca_hip::Aligned16(v->k) || !sca_hip::Aligned16(v->v) ||
        !sca_hip::Aligned16(v->out) || v->q_ss % 8 || v->q_sh % 8 || v->k_ss % 8 ||
        v->k_sh % 8 || v->v_ss % 8 || v->v_sh % 8 || v->o_ss % 8 || v->o_sh % 8) {
        return SetError(SCA_E_LAYOUT_MISMATCH,
                        "flash varlen: pointers must be 16 B aligned and strides multiples of 8");
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    return v->dtype == SCA_DTYPE_F16 ? sca_hip::LaunchVarlenTyped<sca_hip::F16>(*v, s)
                                     : sca_hip::LaunchVarlenTyped<sca_hip::BF16>(*v, s);
}

int sca_hip_flash_fwd(const sca_flash_params* p, void* stream) {
    if (p == nullptr) return SetError(SCA_E_SHAPE_MISMATCH, "flash: null params");
    if (p->q == nullptr || p->k == nullptr || p->v == nullptr || p->out == nullptr) {
        return SetError(SCA_E_SHAPE_MISMATCH, "flash: null pointer");
    }
    if (p->dtype != SCA_DTYPE_F16 && p->dtype != SCA_DTYPE_BF16) {
        return SetError(SCA_E_UNSUPPORTED_DTYPE,
                        "flash: dtype id " + std::to_string(p->dtype) +
                            " (the MFMA kernel computes in fp16/bf16 only)");
    }
    if (p->batch < 1 || p->num_heads < 1 || p->num_kv_heads < 1 || p->seq_q < 1 ||
        p->seq_kv < 1 || p->num_heads % p->num_kv_heads != 0) {
        return SetError(SCA_E_SHAPE_MISMATCH,
                        "flash: invalid geometry B=" + std::to_string(p->batch) +
                            " Hq=" + std::to_string(p->num_heads) +
                            " Hkv=" + std::to_string(p->num_kv_heads) +
                            " Sq=" + std::to_string(p->seq_q) + " Skv=" + std::to_string(p->seq_kv));
    }
    if (p->seq_q > (1LL << 30) || p->seq_kv > (1LL << 30) || p->k_ss > (1LL << 24) ||
        p->v_ss > (1LL << 24)) {
        return SetError(SCA_E_SEQ_TOO_LONG,
                        "flash: seq_q/seq_kv must be <= 2^30 and K/V row strides <= 2^24 elements");
    }
    if (p->causal && p->diagonal < 0) {
        return SetError(SCA_E_SHAPE_MISMATCH,
                        "flash: causal needs diagonal >= 0 (seq_kv >= seq_q); diagonal=" +
                            std::to_string(p->diagonal));
    }
    if (!(p->scale > 0.0f)) {
        return SetError(SCA_E_SHAPE_MISMATCH, "flash: scale must be > 0");
    }
    if (!sca_hip::Aligned16(p->q) || !sca_hip::Aligned16(p->k) || !sca_hip::Aligned16(p->v) ||
        !sca_hip::Aligned16(p->out) || p->q_ss % 8 || p->q_sh % 8 || p->q_sb % 8 ||
        p->k_ss % 8 || p->k_sh % 8 || p->k_sb % 8 || p->v_ss % 8 || p->v_sh % 8 ||
        p->v_sb % 8 || p->o_ss % 4 || p->o_sh % 4 || p->o_sb % 4) {
        return SetError(SCA_E_LAYOUT_MISMATCH,
                        "flash: q/k/v/out must be 16 B aligned with 16 B-multiple row strides");
    }
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (p->dtype == SCA_DTYPE_F16) {
        return p->causal ? sca_hip::LaunchForDim<sca_hip::F16, true>(*p, s)
                         : sca_hip::LaunchForDim<sca_hip::F16, false>(*p, s);
    }
    return p->causal ? sca_hip::LaunchForDim<sca_hip::BF16, true>(*p, s)
                     : sca_hip::LaunchForDim<sca_hip::BF16, false>(*p, s);
}

}  // extern "C"

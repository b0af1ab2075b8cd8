// Flash prefill forward for gfx950: O = softmax(scale * Q K^T + mask) V, fp16/bf16 in, fp32
// accumulation, optional natural-log LSE. No score matrix is ever written to memory.
//
// Semantics follow the reference kernel (src/backends/flash/flash_fwd_impl.cuh:45-279,
// flash_online_softmax.cuh:34-99, flash_causal_mask.cuh:14-28): bottom-right causal mask
// (key j visible from row i iff j <= i + diagonal), masked logits are exactly -inf, GQA maps
// q head h to kv head h / (H_q / H_kv), P is rounded to the input dtype before the PV product,
// out = O / l (0 when l == 0), LSE = m + ln(l) (-inf when l == 0).
//
// MI355X design
//   * workgroup = 4 waves = 128 query rows of one (batch, head); each wave owns 32 rows;
//   * S^T = K Q^T with v_mfma_f32_32x32x16_{f16,bf16}: A = K rows from LDS (one 16 B read per
//     lane), B = Q^T held in registers for the whole kernel. In the S^T accumulator every lane
//     holds 16 keys of ONE query row, so the row max/sum need a single exchange between the two
//     32-lane halves and the online-softmax state (m, l) is one register per lane;
//   * the P^T accumulator registers, converted to fp16/bf16, are directly the B operand of
//     O^T = V^T P^T (the key order inside an MFMA k-step is chosen to match the accumulator
//     layout), so P never leaves registers;
//   * V is transposed once per tile while it is staged into LDS (V^T rows = head-dim), so the
//     A operand of the PV MFMA is two 8-byte LDS reads per lane;
//   * K/V tiles are double-buffered in LDS with a register prefetch of the next tile issued
//     before the current tile's MFMAs; one barrier per tile;
//   * causal grids are issued longest-row-tile first (LPT order) and waves skip tiles that are
//     fully masked for their 32 rows.

#include <hip/hip_runtime.h>

#include <string>

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
    static constexpr int STAGE_BYTES = 2 * (K_STAGE + V_STAGE) * 2;
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

template <typename E, int D, bool kCausal>
__global__ __launch_bounds__(FlashGeom<D>::THREADS, 1) void flash_fwd_kernel(
    const sca_flash_params p, int num_q_tiles) {
    using G = FlashGeom<D>;
    using M = Mfma<E>;
    using vec8 = typename E::vec8;
    constexpr int BN = G::BN;

    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t* sK = lds;                    // [2][BN][KSTR]
    uint16_t* sV = lds + 2 * G::K_STAGE;   // [2][D][VSTR]  (V^T)

    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid % kWave;
    const int lr = lane & 31;
    const int hh = lane >> 5;
    const int rg = wave % kRowGroups;  // row group
    const int kh = wave / kRowGroups;  // which 32 keys of every tile this wave owns

    // Block -> (tile, batch*head). Causal: longest row tiles are dispatched first.
    const int64_t bh_count = p.batch * p.num_heads;
    const int64_t tile_linear = static_cast<int64_t>(blockIdx.x) / bh_count;
    const int64_t bh = static_cast<int64_t>(blockIdx.x) % bh_count;
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
    if (kCausal) {
        const int last_key = q0 + kBlockM - 1 + diag;
        const int causal_tiles = last_key < 0 ? 0 : last_key / BN + 1;
        if (causal_tiles < n_tiles) n_tiles = causal_tiles;
    }

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

    if (n_tiles > 0) {
        load_tile(0);
        store_tile(0);
    }

    const int wkey_base = 32 * kh;  // this wave's first key inside a tile
    for (int j = 0; j < n_tiles; ++j) {
        __syncthreads();
        const int stage = j & 1;
        const bool more = (j + 1) < n_tiles;
        if (more) load_tile(j + 1);

        const int wkey0 = j * BN + wkey_base;
        // Skip the tile when none of this wave's 32 keys exists or is visible to its rows.
        const bool wave_active = wkey0 < seq_kv &&
                                 (!kCausal || wkey0 <= wave_q0 + kRowsPerWave - 1 + diag);
        if (wave_active) {
            const uint16_t* k_tile = sK + stage * G::K_STAGE + (wkey_base + lr) * G::KSTR + 8 * hh;
            // S^T[key][q] for this wave's 32 keys x 32 rows.
            floatx16 s;
#pragma unroll
            for (int i = 0; i < 16; ++i) s[i] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < G::KS; ++ks) {
                const vec8 a = *reinterpret_cast<const vec8*>(k_tile + 16 * ks);
                s = M::mma(a, qf[ks], s);
            }

            // Mask only where some key is beyond seq_kv or above the causal diagonal.
            const bool tail = wkey0 + 32 > seq_kv;
            const bool on_diag = kCausal && (wkey0 + 31 > wave_q0 + diag);
            if (tail || on_diag) {
                const int lim = kCausal ? min(seq_kv - 1, my_q + diag) : seq_kv - 1;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int key = wkey0 + 8 * (i / 4) + 4 * hh + (i % 4);
                    if (key > lim) s[i] = neg_inf();
                }
            }

            // Row max over the lane's 16 keys and the partner half (lane ^ 32).
            float tmax = fmaxf(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])),
                               fmaxf(fmaxf(s[4], s[5]), fmaxf(s[6], s[7])));
            tmax = fmaxf(tmax, fmaxf(fmaxf(fmaxf(s[8], s[9]), fmaxf(s[10], s[11])),
                                     fmaxf(fmaxf(s[12], s[13]), fmaxf(s[14], s[15]))));
            tmax = fmaxf(tmax, xor32(tmax)) * scale2;
            // Lazy rescale: the max used for the exponentials only moves when the row max grew by
            // more than kRescaleSlack (weights stay <= 2^slack), and the O/l rescale runs only
            // when some lane of the wave moved.
            const bool grow = tmax > m_used + kRescaleSlack;
            if (__builtin_amdgcn_ballot_w64(grow) != 0) {
                const float m_new = grow ? tmax : m_used;
                const float alpha = grow ? fast_exp2(m_used - m_new) : 1.0f;
                m_used = m_new;
                l_run *= alpha;
#pragma unroll
                for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
                    for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
                }
            }
            const float mu = (m_used == neg_inf()) ? 0.0f : m_used;

            // P^T = 2^(s*scale2 - m), rounded to the input dtype: directly the PV B operand.
            uint32_t pw[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float p0 = fast_exp2(fmaf(s[2 * i], scale2, -mu));
                const float p1 = fast_exp2(fmaf(s[2 * i + 1], scale2, -mu));
                pw[i] = M::pack(p0, p1);
                l_run = M::sum2(pw[i], l_run);
            }
            const vec8 pb0 = __builtin_bit_cast(vec8, make_uint4(pw[0], pw[1], pw[2], pw[3]));
            const vec8 pb1 = __builtin_bit_cast(vec8, make_uint4(pw[4], pw[5], pw[6], pw[7]));

            // O^T[d][q] += V^T[d][key] P^T[key][q]; k-step ps covers keys
            // 16*ps + {0..3, 8..11} (hh = 0) or 16*ps + {4..7, 12..15} (hh = 1).
            const uint16_t* v_tile =
                sV + stage * G::V_STAGE + lr * G::VSTR + wkey_base + 4 * hh;
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
                for (int ps = 0; ps < 2; ++ps) {
                    const uint16_t* vrow = v_tile + 32 * dt * G::VSTR + 16 * ps;
                    const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                    const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 8);
                    const vec8 a = __builtin_bit_cast(vec8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                    o[dt] = M::mma(a, ps == 0 ? pb0 : pb1, o[dt]);
                }
            }
        }

        if (more) store_tile((j + 1) & 1);
    }

    // Merge the KSPLIT partial states of each row group through LDS.
    if constexpr (G::KSPLIT > 1) {
        __syncthreads();  // every wave is done reading the K/V stages
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
    static bool attr_set = false;  // benign race: the attribute call is idempotent
    if (!attr_set) {
        const hipError_t err = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&flash_fwd_kernel<E, D, kCausal>),
            hipFuncAttributeMaxDynamicSharedMemorySize, G::LDS_BYTES);
        // A refusal here is not fatal: the launch itself reports an LDS request the device
        // cannot serve.
        if (err != hipSuccess) (void)hipGetLastError();
        attr_set = true;
    }
    hipLaunchKernelGGL((flash_fwd_kernel<E, D, kCausal>), dim3(static_cast<unsigned>(blocks)),
                       dim3(G::THREADS), G::LDS_BYTES, s, p, static_cast<int>(num_q_tiles));
    return CheckLaunch("flash_fwd_kernel", s);
}

template <typename E, bool kCausal>
int LaunchForDim(const sca_flash_params& p, hipStream_t s) {
    switch (p.head_dim) {
        case 32: return LaunchFlash<E, 32, kCausal>(p, s);
        case 64: return LaunchFlash<E, 64, kCausal>(p, s);
        case 96: return LaunchFlash<E, 96, kCausal>(p, s);
        case 128: return LaunchFlash<E, 128, kCausal>(p, s);
        case 160: return LaunchFlash<E, 160, kCausal>(p, s);
        case 192: return LaunchFlash<E, 192, kCausal>(p, s);
        case 256: return LaunchFlash<E, 256, kCausal>(p, s);
        default: break;
    }
    return SetError(SCA_E_UNSUPPORTED_HEAD_DIM,
                    "flash: head_dim=" + std::to_string(p.head_dim) + " is not instantiated");
}

bool Aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

int LdsBytesFor(int64_t head_dim) {
    switch (head_dim) {
        case 32: return FlashGeom<32>::LDS_BYTES;
        case 64: return FlashGeom<64>::LDS_BYTES;
        case 96: return FlashGeom<96>::LDS_BYTES;
        case 128: return FlashGeom<128>::LDS_BYTES;
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
    if (block_m != nullptr) *block_m = sca_hip::kBlockM;
    if (block_n != nullptr) *block_n = head_dim <= 128 ? 64 : 32;
    if (waves != nullptr) *waves = head_dim <= 128 ? 8 : 4;
    if (stages != nullptr) *stages = 2;
    return 0;
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

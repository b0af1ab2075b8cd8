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

constexpr int kFlashThreads = 256;
constexpr int kFlashWaves = kFlashThreads / kWave;
constexpr int kRowsPerWave = 32;
constexpr int kBlockM = kFlashWaves * kRowsPerWave;  // 128
constexpr int kKPad = 8;  // K rows padded by 16 B
constexpr int kVPad = 4;  // V^T rows padded by 8 B

template <int D>
struct FlashGeom {
    static constexpr int BN = D <= 128 ? 64 : 32;        // keys per tile
    static constexpr int KS = D / 16;                    // QK k-steps
    static constexpr int NT = BN / 32;                   // 32-key sub-tiles of S^T
    static constexpr int DT = D / 32;                    // 32-row tiles of O^T
    static constexpr int PS = BN / 16;                   // PV k-steps
    static constexpr int KSTR = D + kKPad;               // K row stride (elements)
    static constexpr int VSTR = BN + kVPad;              // V^T row stride (elements)
    static constexpr int K_CHUNKS = BN * D / 8;          // 16 B chunks per K tile
    static constexpr int K_PER_THREAD = (K_CHUNKS + kFlashThreads - 1) / kFlashThreads;
    static constexpr int V_UNITS = (BN / 4) * (D / 8);   // 4 keys x 8 dims per unit
    static constexpr int V_PER_THREAD = (V_UNITS + kFlashThreads - 1) / kFlashThreads;
    static constexpr int K_STAGE = BN * KSTR;            // elements per K stage
    static constexpr int V_STAGE = D * VSTR;             // elements per V^T stage
    static constexpr int LDS_BYTES = 2 * (K_STAGE + V_STAGE) * 2;
};

template <typename E>
struct Mfma;

template <>
struct Mfma<F16> {
    static __device__ __forceinline__ floatx16 mma(const half8& a, const half8& b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Mfma<BF16> {
    static __device__ __forceinline__ floatx16 mma(const bf16x8& a, const bf16x8& b, floatx16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

__device__ __forceinline__ uint16_t Half16(const uint4& v, int t) {
    const uint32_t w = (t < 2) ? v.x : (t < 4) ? v.y : (t < 6) ? v.z : v.w;
    return static_cast<uint16_t>((t & 1) ? (w >> 16) : (w & 0xffffu));
}

template <typename E, int D, bool kCausal>
__global__ __launch_bounds__(kFlashThreads, 1) void flash_fwd_kernel(const sca_flash_params p,
                                                                     int num_q_tiles) {
    using G = FlashGeom<D>;
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

    // Block -> (tile, batch*head). Causal: longest row tiles are dispatched first.
    const int64_t bh_count = p.batch * p.num_heads;
    const int64_t tile_linear = static_cast<int64_t>(blockIdx.x) / bh_count;
    const int64_t bh = static_cast<int64_t>(blockIdx.x) % bh_count;
    const int64_t qt = kCausal ? (num_q_tiles - 1 - tile_linear) : tile_linear;
    const int64_t b = bh / p.num_heads;
    const int64_t h = bh % p.num_heads;
    const int64_t h_kv = h / (p.num_heads / p.num_kv_heads);
    const int64_t q0 = qt * kBlockM;
    const int64_t wave_q0 = q0 + wave * kRowsPerWave;
    const int64_t my_q = wave_q0 + lr;

    const uint16_t* q_ptr = static_cast<const uint16_t*>(p.q) + b * p.q_sb + h * p.q_sh;
    const uint16_t* k_ptr = static_cast<const uint16_t*>(p.k) + b * p.k_sb + h_kv * p.k_sh;
    const uint16_t* v_ptr = static_cast<const uint16_t*>(p.v) + b * p.v_sb + h_kv * p.v_sh;

    // Q^T fragments (B operand of S^T = K Q^T): lane holds Q[my_q][16*ks + 8*hh + 0..7].
    vec8 qf[G::KS];
#pragma unroll
    for (int ks = 0; ks < G::KS; ++ks) {
        uint4 raw = make_uint4(0, 0, 0, 0);
        if (my_q < p.seq_q) {
            raw = *reinterpret_cast<const uint4*>(q_ptr + my_q * p.q_ss + 16 * ks + 8 * hh);
        }
        qf[ks] = __builtin_bit_cast(vec8, raw);
    }

    // Number of KV tiles this workgroup needs.
    int64_t n_tiles = (p.seq_kv + BN - 1) / BN;
    if (kCausal) {
        const int64_t last_key = q0 + kBlockM - 1 + p.diagonal;
        const int64_t causal_tiles = last_key < 0 ? 0 : last_key / BN + 1;
        if (causal_tiles < n_tiles) n_tiles = causal_tiles;
    }

    floatx16 o[G::DT];
#pragma unroll
    for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
        for (int i = 0; i < 16; ++i) o[dt][i] = 0.0f;
    }
    float m_run = neg_inf();  // running max, log2 domain (scale * log2e folded in)
    float l_run = 0.0f;       // running sum over this lane's keys (halves merged at the end)
    const float scale2 = p.scale * kLog2e;

    // ---- staging: global -> registers -> LDS ------------------------------------------------
    uint4 k_stage[G::K_PER_THREAD];
    uint4 v_stage[G::V_PER_THREAD][4];

    auto load_tile = [&](int64_t t) {
        const int64_t key0 = t * BN;
#pragma unroll
        for (int i = 0; i < G::K_PER_THREAD; ++i) {
            const int c = tid + i * kFlashThreads;
            k_stage[i] = make_uint4(0, 0, 0, 0);
            if (c < G::K_CHUNKS) {
                const int row = c / (D / 8);
                const int col = (c % (D / 8)) * 8;
                const int64_t key = key0 + row;
                if (key < p.seq_kv) {
                    k_stage[i] = *reinterpret_cast<const uint4*>(k_ptr + key * p.k_ss + col);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < G::V_PER_THREAD; ++i) {
            const int u = tid + i * kFlashThreads;
#pragma unroll
            for (int j = 0; j < 4; ++j) v_stage[i][j] = make_uint4(0, 0, 0, 0);
            if (u < G::V_UNITS) {
                const int kg = u / (D / 8);
                const int dc = u % (D / 8);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const int64_t key = key0 + 4 * kg + j;
                    if (key < p.seq_kv) {
                        v_stage[i][j] =
                            *reinterpret_cast<const uint4*>(v_ptr + key * p.v_ss + 8 * dc);
                    }
                }
            }
        }
    };

    auto store_tile = [&](int stage) {
        uint16_t* k_dst = sK + stage * G::K_STAGE;
        uint16_t* v_dst = sV + stage * G::V_STAGE;
#pragma unroll
        for (int i = 0; i < G::K_PER_THREAD; ++i) {
            const int c = tid + i * kFlashThreads;
            if (c < G::K_CHUNKS) {
                const int row = c / (D / 8);
                const int col = (c % (D / 8)) * 8;
                *reinterpret_cast<uint4*>(k_dst + row * G::KSTR + col) = k_stage[i];
            }
        }
#pragma unroll
        for (int i = 0; i < G::V_PER_THREAD; ++i) {
            const int u = tid + i * kFlashThreads;
            if (u < G::V_UNITS) {
                const int kg = u / (D / 8);
                const int dc = u % (D / 8);
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const uint32_t lo = static_cast<uint32_t>(Half16(v_stage[i][0], t)) |
                                        (static_cast<uint32_t>(Half16(v_stage[i][1], t)) << 16);
                    const uint32_t hi = static_cast<uint32_t>(Half16(v_stage[i][2], t)) |
                                        (static_cast<uint32_t>(Half16(v_stage[i][3], t)) << 16);
                    *reinterpret_cast<uint2*>(v_dst + (8 * dc + t) * G::VSTR + 4 * kg) =
                        make_uint2(lo, hi);
                }
            }
        }
    };

    if (n_tiles > 0) {
        load_tile(0);
        store_tile(0);
    }

    for (int64_t j = 0; j < n_tiles; ++j) {
        __syncthreads();
        const int stage = static_cast<int>(j & 1);
        const bool more = (j + 1) < n_tiles;
        if (more) load_tile(j + 1);

        const int64_t key0 = j * BN;
        // A wave whose 32 rows cannot see any key of this tile skips it entirely.
        const bool wave_active = !kCausal || key0 <= wave_q0 + kRowsPerWave - 1 + p.diagonal;
        if (wave_active) {
            const uint16_t* k_tile = sK + stage * G::K_STAGE;
            const uint16_t* v_tile = sV + stage * G::V_STAGE;

            // S^T[key][q] for this wave's 32 rows.
            floatx16 s[G::NT];
#pragma unroll
            for (int nt = 0; nt < G::NT; ++nt) {
#pragma unroll
                for (int i = 0; i < 16; ++i) s[nt][i] = 0.0f;
#pragma unroll
                for (int ks = 0; ks < G::KS; ++ks) {
                    const vec8 a = *reinterpret_cast<const vec8*>(
                        k_tile + (32 * nt + lr) * G::KSTR + 16 * ks + 8 * hh);
                    s[nt] = Mfma<E>::mma(a, qf[ks], s[nt]);
                }
            }

            // Scale to the log2 domain, mask, tile row max.
            const bool tail = key0 + BN > p.seq_kv;
            const bool diag = kCausal && (key0 + BN - 1 > wave_q0 + p.diagonal);
            float tile_max = neg_inf();
#pragma unroll
            for (int nt = 0; nt < G::NT; ++nt) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    float x = s[nt][i] * scale2;
                    if (tail || diag) {
                        const int64_t key = key0 + 32 * nt + 8 * (i / 4) + 4 * hh + (i % 4);
                        const bool visible =
                            key < p.seq_kv && (!kCausal || key <= my_q + p.diagonal);
                        x = visible ? x : neg_inf();
                    }
                    s[nt][i] = x;
                    tile_max = fmaxf(tile_max, x);
                }
            }
            tile_max = fmaxf(tile_max, xor32(tile_max));
            const float m_new = fmaxf(m_run, tile_max);
            const float m_use = (m_new == neg_inf()) ? 0.0f : m_new;
            const float alpha = fast_exp2(m_run - m_use);
            m_run = m_new;
            l_run *= alpha;
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
                for (int i = 0; i < 16; ++i) o[dt][i] *= alpha;
            }

            // P^T = 2^(s - m), rounded to the input dtype: directly the PV B operand.
            vec8 pb[G::PS];
#pragma unroll
            for (int ps = 0; ps < G::PS; ++ps) {
                u16x8 bits;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const float pv = fast_exp2(s[ps / 2][8 * (ps % 2) + t] - m_use);
                    bits[t] = E::from_float(pv);
                    // l sums the rounded weights, so the normaliser matches the PV weights.
                    l_run += E::to_float(bits[t]);
                }
                pb[ps] = __builtin_bit_cast(vec8, bits);
            }

            // O^T[d][q] += V^T[d][key] P^T[key][q]
#pragma unroll
            for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
                for (int ps = 0; ps < G::PS; ++ps) {
                    const uint16_t* vrow = v_tile + (32 * dt + lr) * G::VSTR + 16 * ps + 4 * hh;
                    const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                    const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 8);
                    const vec8 a = __builtin_bit_cast(vec8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                    o[dt] = Mfma<E>::mma(a, pb[ps], o[dt]);
                }
            }
        }

        if (more) store_tile(static_cast<int>((j + 1) & 1));
    }

    // Epilogue: merge the two halves' partial sums, normalise, store.
    const float l_tot = l_run + xor32(l_run);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (my_q < p.seq_q) {
        uint16_t* out_row =
            static_cast<uint16_t*>(p.out) + b * p.o_sb + h * p.o_sh + my_q * p.o_ss;
#pragma unroll
        for (int dt = 0; dt < G::DT; ++dt) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int d0 = 32 * dt + 8 * g + 4 * hh;
                const uint32_t lo = static_cast<uint32_t>(E::from_float(o[dt][4 * g + 0] * inv)) |
                                    (static_cast<uint32_t>(E::from_float(o[dt][4 * g + 1] * inv))
                                     << 16);
                const uint32_t hi = static_cast<uint32_t>(E::from_float(o[dt][4 * g + 2] * inv)) |
                                    (static_cast<uint32_t>(E::from_float(o[dt][4 * g + 3] * inv))
                                     << 16);
                *reinterpret_cast<uint2*>(out_row + d0) = make_uint2(lo, hi);
            }
        }
        if (p.lse != nullptr && hh == 0) {
            p.lse[(b * p.num_heads + h) * p.seq_q + my_q] =
                l_tot > 0.0f ? (m_run + __log2f(l_tot)) * kLn2 : neg_inf();
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
                       dim3(kFlashThreads), G::LDS_BYTES, s, p, static_cast<int>(num_q_tiles));
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
    if (waves != nullptr) *waves = sca_hip::kFlashWaves;
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

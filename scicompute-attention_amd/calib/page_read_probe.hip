// Calibration kernel for the paged decode roofline: reads exactly the K/V bytes the paged decode
// kernel reads, in its order, and does nothing else. A block-major pool of pages
// [num_blocks, block_size, num_kv_heads, head_dim] is addressed through a permuted page table,
// so every (page, kv head) is a 4 KB slice of 16 rows x 256 B at a 2 KB row stride. Each wave
// streams one (sequence, kv head, split) of K and V as the decode kernel's waves do, with DEPTH
// 32-token tiles (16 KB per wave) in flight, and folds the data into one XOR per lane so the
// loads cannot be dropped. Variants (mode bits): V through LDS with global_load_lds as the decode
// kernel stages it (1); K loaded as the decode kernel's MFMA fragments, 16 rows x 64 B per
// instruction, instead of 4 rows x 256 B (2); 8 waves per workgroup, every kv head of a row,
// instead of 4 (4). The rates they reach are the practical ceilings for these access patterns,
// measured rather than assumed.
//
// Built into lib/libsca_calib.so for bench.py's calibration leg only; it is not part of the
// attention library or its C ABI.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kWave = 64;
constexpr int kWaves = 4;       // waves per workgroup: neighbouring kv heads of one sequence
constexpr int kTile = 32;       // tokens per tile
constexpr int kLoads = 8;       // 16-byte loads per lane per tile and tensor (32 rows x 256 B)

template <int N>
__device__ __forceinline__ void WaitVm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

struct ProbeArgs {
    const uint8_t* k;
    const uint8_t* v;
    const int32_t* page_table;
    const int32_t* seq_lens;
    uint32_t* sink;
    int num_kv_heads;
    int max_blocks;
    int splits;
};

// head_dim 128, bf16/fp16 (256 B per row and head), block size 16. kLdsV: V goes global -> LDS
// through global_load_lds (a DEPTH-stage ring of 8 KB per wave, one LDS object per stage), as the
// decode kernel stages it; otherwise both tensors go to registers.
template <int DEPTH, bool kLdsV, bool kKFrag, int WAVES>
__global__ __launch_bounds__(kWave * WAVES) void page_read_probe(const ProbeArgs a) {
    __shared__ __align__(16) uint8_t s0[kLdsV ? WAVES * 8192 : 16];
    __shared__ __align__(16) uint8_t s1[kLdsV && DEPTH > 1 ? WAVES * 8192 : 16];
    __shared__ __align__(16) uint8_t s2[kLdsV && DEPTH > 2 ? WAVES * 8192 : 16];
    __shared__ __align__(16) uint8_t s3[kLdsV && DEPTH > 3 ? WAVES * 8192 : 16];
    uint8_t* const stage[4] = {s0, s1, s2, s3};
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int head = blockIdx.y * WAVES + wave;
    const int b = blockIdx.z;
    const int split = blockIdx.x;
    if (head >= a.num_kv_heads) return;
    const int len = a.seq_lens[b];
    const int chunk = (len + a.splits - 1) / a.splits;
    const int t_begin = split * chunk;
    const int t_end = min(t_begin + chunk, len);
    const int n_tiles = t_end > t_begin ? (t_end - t_begin + kTile - 1) / kTile : 0;
    const int64_t row_bytes = static_cast<int64_t>(a.num_kv_heads) * 256;
    const int32_t* table = a.page_table + static_cast<int64_t>(b) * a.max_blocks;

    uint4 kr[DEPTH][kLoads], vr[DEPTH][kLoads];
    auto issue = [&](int tile, int st) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            int t = t_begin + tile * kTile + 4 * i + lane / 16;
            t = t < t_end ? t : t_begin;
            const int64_t row = static_cast<int64_t>(table[t >> 4]) * 16 + (t & 15);
            const int64_t off = row * row_bytes + head * 256 + (lane % 16) * 16;
            if constexpr (kKFrag) {
                // The decode kernel's K fragments: load (rt, j) = i gives lane l the 16 bytes
                // (4j + l/16)*16 of token 16 rt + l%16 (16 rows x 64 B per instruction).
                int tk = t_begin + tile * kTile + 16 * (i / 4) + lane % 16;
                tk = tk < t_end ? tk : t_begin;
                const int64_t rk = static_cast<int64_t>(table[tk >> 4]) * 16 + (tk & 15);
                kr[st][i] = *reinterpret_cast<const uint4*>(
                    a.k + rk * row_bytes + head * 256 + (4 * (i % 4) + lane / 16) * 16);
            } else {
                kr[st][i] = *reinterpret_cast<const uint4*>(a.k + off);
            }
            if constexpr (kLdsV) {
                __builtin_amdgcn_global_load_lds(
                    a.v + off,
                    (__attribute__((address_space(3))) void*)(stage[st] + wave * 8192 + i * 1024),
                    16, 0, 0);
            } else {
                vr[st][i] = *reinterpret_cast<const uint4*>(a.v + off);
            }
        }
    };
    uint32_t acc = 0;
    auto fold = [&](int st) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            uint4 v;
            if constexpr (kLdsV) {
                v = *reinterpret_cast<const uint4*>(stage[st] + wave * 8192 + i * 1024 + lane * 16);
            } else {
                v = vr[st][i];
            }
            acc ^= kr[st][i].x ^ kr[st][i].w ^ v.y ^ v.z;
        }
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        if (d < n_tiles) issue(d, d);
    }
    for (int tile = 0; tile < n_tiles; tile += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            if (tile + d < n_tiles) {
                // The DEPTH - 1 tiles after this one are in flight unless the split ends first.
                if (tile + d + DEPTH - 1 < n_tiles) {
                    WaitVm<2 * kLoads * (DEPTH - 1)>();
                } else {
                    WaitVm<0>();
                }
                fold(d);
                if (tile + d + DEPTH < n_tiles) issue(tile + d + DEPTH, d);
            }
        }
    }
    if (acc == 0x9e3779b9u) a.sink[0] = acc;  // keeps the loads; practically never taken
}

template <int DEPTH, int WAVES>
void LaunchW(const ProbeArgs& a, int batch, int mode, hipStream_t s) {
    const unsigned gy = static_cast<unsigned>((a.num_kv_heads + WAVES - 1) / WAVES);
    const dim3 grid(static_cast<unsigned>(a.splits), gy, static_cast<unsigned>(batch));
    const dim3 block(kWave * WAVES);
    constexpr bool kLdsFits = DEPTH * WAVES * 8192 <= 131072;
    switch (mode & 3) {
        case 0: hipLaunchKernelGGL((page_read_probe<DEPTH, false, false, WAVES>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((page_read_probe<DEPTH, false, true, WAVES>), grid, block, 0, s, a); break;
        case 1:
            if constexpr (kLdsFits) {
                hipLaunchKernelGGL((page_read_probe<DEPTH, true, false, WAVES>), grid, block, 0, s, a);
            }
            break;
        default:
            if constexpr (kLdsFits) {
                hipLaunchKernelGGL((page_read_probe<DEPTH, true, true, WAVES>), grid, block, 0, s, a);
            }
            break;
    }
}

// mode bit 0: V through LDS; bit 1: K in the decode kernel's fragment pattern; bit 2: 8 waves
// (every kv head of a row) per workgroup instead of 4.
template <int DEPTH>
int Launch(const ProbeArgs& a, int batch, int mode, hipStream_t s) {
    if (mode & 4) {
        if (DEPTH > 2 && (mode & 1)) return static_cast<int>(hipErrorInvalidValue);  // LDS
        LaunchW<DEPTH, 8>(a, batch, mode, s);
    } else {
        LaunchW<DEPTH, kWaves>(a, batch, mode, s);
    }
    return static_cast<int>(hipGetLastError());
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int sca_calib_page_read(
    const void* k_pool, const void* v_pool, const int32_t* page_table, const int32_t* seq_lens,
    int batch, int num_kv_heads, int max_blocks, int splits, int depth, int mode,
    uint32_t* sink, void* stream) {
    if (k_pool == nullptr || v_pool == nullptr || page_table == nullptr || seq_lens == nullptr ||
        sink == nullptr || batch < 1 || batch > 65535 || num_kv_heads < 1 || max_blocks < 1 ||
        splits < 1 || splits > 65535 || mode < 0 || mode > 7) {
        return static_cast<int>(hipErrorInvalidValue);
    }
    const ProbeArgs a{static_cast<const uint8_t*>(k_pool), static_cast<const uint8_t*>(v_pool),
                      page_table, seq_lens, sink, num_kv_heads, max_blocks, splits};
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (depth) {
        case 1: return Launch<1>(a, batch, mode, s);
        case 2: return Launch<2>(a, batch, mode, s);
        case 3: return Launch<3>(a, batch, mode, s);
        case 4: return Launch<4>(a, batch, mode, s);
        default: return static_cast<int>(hipErrorInvalidValue);
    }
}

#pragma once

#include <cstdint>
#include <string>

#include "scicompute_attention/export.hpp"

namespace sca {

// Tile geometry of a tiled/MMA backend, as reported by the dispatcher and in the run stats.
//   block_m : query rows per workgroup
//   block_n : keys per pipeline step
//   warps   : wavefronts per workgroup (64 lanes each on CDNA; the field keeps the reference's
//             name so caller code compiles unchanged)
//   stages  : K/V buffering depth in LDS
//   use_tma : always false on this hardware
struct TileConfig {
    int32_t block_m{0};
    int32_t block_n{0};
    int32_t warps{0};
    int32_t stages{0};
    bool use_tma{false};

    static constexpr int32_t kLanesPerWave = 64;

    constexpr int Threads() const noexcept { return warps * kLanesPerWave; }
    constexpr bool Empty() const noexcept { return block_m == 0 || block_n == 0 || warps == 0; }

    // The reference's padded-row footprint formula for a flash tile (Q tile + `stages` K tiles +
    // `stages` V tiles, each row padded by kSmemPadElems elements); -1 for an invalid tile. Kept
    // because it is public arithmetic callers use for budgeting; the MI355X kernel's own LDS use
    // is reported by FlashLdsBytes().
    static constexpr int64_t SmemBytesFlash(int32_t head_dim, int64_t elem_bytes, int32_t block_m,
                                            int32_t block_n, int32_t warps, int32_t stages) {
        if (head_dim <= 0 || block_m <= 0 || block_n <= 0 || warps <= 0 || stages <= 0) return -1;
        const int64_t row = static_cast<int64_t>(head_dim + kSmemPadElems) * elem_bytes;
        return static_cast<int64_t>(block_m) * row +
               2 * static_cast<int64_t>(stages) * static_cast<int64_t>(block_n) * row;
    }

    int64_t SmemBytesFlash(int32_t head_dim, int64_t elem_bytes) const {
        return SmemBytesFlash(head_dim, elem_bytes, block_m, block_n, warps, stages);
    }

    static constexpr int32_t kSmemPadElems = 8;

    std::string ToString() const {
        return "bm=" + std::to_string(block_m) + ",bn=" + std::to_string(block_n) +
               ",warps=" + std::to_string(warps) + ",stages=" + std::to_string(stages) +
               (use_tma ? ",tma=on" : ",tma=off");
    }
};

}  // namespace sca

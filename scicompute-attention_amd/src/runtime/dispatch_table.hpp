// Compiled-in dispatch thresholds of the MI355X build.
//
// The routing rules are the reference's (src/runtime/dispatch_table.inc:30-37, r0) except one:
// short sequences (seq_kv <= 128) go to the flash kernel, which serves every length without a
// score workspace, instead of the reference's score-materialising tiled kernel (not built here).
// Split counts are derived from the compute-unit count: enough workgroups for every CU to hold
// several, each split still covering at least `min_tokens_per_split` keys.
#pragma once

#include <cstdint>

namespace sca {
namespace detail {

struct DispatchThresholds {
    int64_t decode_max_seq_q;      // seq_q <= this and seq_kv >= decode_min_seq_kv => decode
    int64_t decode_min_seq_kv;
    int64_t short_max_seq_kv;      // seq_kv <= this => "short sequence" rule (flash here)
    int64_t min_tokens_per_split;  // lower bound on keys per split
    int64_t workgroups_per_cu;     // split-K target occupancy
    int64_t max_splits;            // cap on the split count (explicit and automatic)
    const char* revision;          // reported by Explain()
};

inline constexpr DispatchThresholds kDispatchThresholds{
    /* decode_max_seq_q     */ 1,
    /* decode_min_seq_kv    */ 256,
    /* short_max_seq_kv     */ 128,
    /* min_tokens_per_split */ 512,
    /* workgroups_per_cu    */ 6,
    /* max_splits           */ 64,
    /* revision             */ "r0-mi355x",
};

// Split count of the decode kernels for `batch` sequences of up to `seq_kv` keys. A head slot is
// one KV head and up to 16 of its query heads; the MFMA kernel runs a workgroup per (sequence,
// split, slot) with four waves per slot (slot_waves = 4, the contiguous default) or per (sequence,
// split, four slots) with one wave per slot (slot_waves = 1, the paged default).
//  - Four waves per slot: a batch with at least one slot per CU runs unsplit, which also skips
//    the combine kernel (measured on MI355X, fp16, H_q 32, H_kv 8, D 128: 64 x 4096 keys 6.07 TB/s
//    against 5.65 at 8 splits; 128 x 2048 6.02 against 5.64; 32 x 4096 5.74 against 5.42);
//    smaller batches take splits until every CU holds 4 workgroups, but no more than 8 unless
//    fewer would leave CUs without a workgroup (C4, 16 x 4096: 8 splits, 5.97 TB/s; 8 x 32768:
//    8 splits, 5.95 against 5.47 at 64; 4 x 16384: 8, 5.84 against 5.66 at 32; 1 x 65536: 32,
//    5.60 against 5.22 at 64).
//  - One wave per slot: splits are added until every CU holds `workgroups_per_cu` workgroups.
//  - head_dim outside {64, 128} (the VALU kernel, a workgroup per (sequence, split, 1-8 heads)):
//    unsplit once the batch gives every CU a workgroup, else splits until every CU holds four,
//    with no cap at 8 (fp16, H_q 32, H_kv 8, D 96: 4 x 16384 keys 32 splits, 4.34 TB/s against
//    3.37 at 8; 16 x 4096 8 splits, 4.63, the best of 1..32; 64 x 4096 unsplit 5.05 against
//    5.10 at 4). fp32 with D 64 or 128 runs the VALU kernel under the MFMA rule (16 x 4096,
//    D 128: 5.21 TB/s at 8 splits against 5.52 at 4).
// Each split keeps at least `min_tokens_per_split` keys.
inline int64_t DecodeSplits(int64_t batch, int64_t num_heads, int64_t num_kv_heads,
                            int64_t seq_kv, int64_t cu_count, int slot_waves = 4,
                            int64_t head_dim = 128) {
    const auto& th = kDispatchThresholds;
    if (batch < 1 || num_kv_heads < 1 || seq_kv < 1) return 1;
    const int64_t group = num_heads / num_kv_heads;
    const int64_t slots = num_kv_heads * ((group + 15) / 16);
    const int64_t cus = cu_count > 0 ? cu_count : 256;
    int64_t splits;
    const bool mfma = head_dim == 64 || head_dim == 128;
    if (!mfma) {
        const int64_t jobs = batch * slots;
        splits = jobs >= cus ? 1 : (4 * cus + jobs - 1) / jobs;
    } else if (slot_waves == 1) {
        const int64_t wgs_per_split = batch * ((slots + 3) / 4);
        splits = (th.workgroups_per_cu * cus + wgs_per_split - 1) / wgs_per_split;
    } else {
        const int64_t jobs = batch * slots;
        if (jobs >= cus) {
            splits = 1;
        } else {
            const int64_t fill = (cus + jobs - 1) / jobs;  // one workgroup per CU
            const int64_t four = (4 * cus + jobs - 1) / jobs;
            splits = four < 8 ? four : (fill > 8 ? fill : 8);
        }
    }
    const int64_t by_length = (seq_kv + th.min_tokens_per_split - 1) / th.min_tokens_per_split;
    if (splits > by_length) splits = by_length;
    if (splits > th.max_splits) splits = th.max_splits;
    return splits < 1 ? 1 : splits;
}

// Work split of the paged MFMA decode kernel for a batch whose host-side lengths are known.
// slot_waves = 1: one wave per head slot, a workgroup serves four slots; 4: four waves share one
// slot's key tiles. Measured on MI355X over 48-step decode loops (bf16, H_q 32, H_kv 8, D 128):
//  - near-uniform batches (longest <= 11/10 of the mean) that leave some CUs free with one split:
//    one wave per slot, one workgroup per CU (uniform 64 x 8448 keys: 5.89 TB/s vs 5.58);
//  - ragged batches with at most two slots per CU: four waves per slot, `workgroups_per_cu`
//    workgroups per CU (C5, 64 x 512..16384: 5.74 TB/s vs 5.61; 16 sequences: 4.98 vs 4.26;
//    64 x 6000..10000: 5.55 vs 5.41 for one wave per slot at one workgroup per CU);
//  - otherwise (many sequences): one wave per slot, `workgroups_per_cu` workgroups per CU
//    (256 x 512..4096: 5.56 TB/s vs 5.54).
// Each split keeps at least `min_tokens_per_split` keys of the longest sequence.
struct PagedDecodePlanResult {
    int64_t splits;
    int32_t slot_waves;
};

inline PagedDecodePlanResult PagedDecodePlan(const int64_t* lengths, int64_t batch,
                                             int64_t num_heads, int64_t num_kv_heads,
                                             int64_t cu_count) {
    const auto& th = kDispatchThresholds;
    if (lengths == nullptr || batch < 1 || num_kv_heads < 1 || num_heads < num_kv_heads) {
        return {1, 0};
    }
    int64_t longest = 0;
    int64_t total = 0;
    for (int64_t b = 0; b < batch; ++b) {
        const int64_t len = lengths[b] > 0 ? lengths[b] : 0;
        longest = len > longest ? len : longest;
        total += len;
    }
    if (longest < 1) return {1, 0};
    const int64_t group = num_heads / num_kv_heads;
    const int64_t slots = num_kv_heads * ((group + 15) / 16);
    const int64_t quads = (slots + 3) / 4;
    const int64_t cus = cu_count > 0 ? cu_count : 256;
    const bool uniform = 10 * longest * batch <= 11 * total;
    int64_t splits;
    int32_t slot_waves;
    if (uniform && batch * quads <= cus) {
        slot_waves = 1;
        splits = cus / (batch * quads);
    } else if (batch * slots <= 2 * cus) {
        slot_waves = 4;
        splits = (th.workgroups_per_cu * cus + batch * slots - 1) / (batch * slots);
    } else {
        slot_waves = 1;
        splits = (th.workgroups_per_cu * cus + batch * quads - 1) / (batch * quads);
    }
    const int64_t by_length = (longest + th.min_tokens_per_split - 1) / th.min_tokens_per_split;
    if (splits > by_length) splits = by_length;
    if (splits > th.max_splits) splits = th.max_splits;
    return {splits < 1 ? 1 : splits, slot_waves};
}

}  // namespace detail
}  // namespace sca

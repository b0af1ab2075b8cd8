#pragma once

#include <cstdint>
#include <vector>

#include "core/status.hpp"
#include "tensor/tensor.hpp"

#include "scicompute_attention/attention_types.hpp"
#include "scicompute_attention/export.hpp"

namespace sci {
class Stream;
}  // namespace sci

namespace sca {

// Interface of the reference's KVCache (include/scicompute_attention/kv_cache.hpp:15-95).

struct KVCacheConfig {
    int64_t num_layers{0};
    int64_t num_kv_heads{0};
    int64_t head_dim{0};
    int64_t block_size{16};  // tokens per page; one of 1, 8, 16, 32, 64
    int64_t num_blocks{0};   // physical pages per layer
    int64_t max_num_seqs{1};
    sci::DType dtype{sci::DType::kFloat16};
    KvLayout layout{KvLayout::kBlockMajor};
    bool enable_stats{true};
};

struct KVCacheStats {
    int64_t num_blocks{0};
    int64_t used_blocks{0};
    int64_t free_blocks{0};
    int64_t num_appends{0};
    int64_t num_resets{0};
    size_t peak_bytes{0};
    size_t bytes{0};
};

// Page storage in HBM, one K and one V tensor per layer, each
//   [num_blocks][block_size][num_kv_heads][head_dim]
// so a page is block_size * num_kv_heads * head_dim contiguous elements and one token row of a
// page (all KV heads) is contiguous: the paged decode kernel reads it with 16-byte vector loads.
class SCI_ATTENTION_API KVCache {
public:
    KVCache() = default;

    // Refuses a cache larger than 80% of the free device memory, naming the largest num_blocks
    // that would fit.
    static sci::Result<KVCache> Create(const KVCacheConfig& cfg, sci::Device& device);

    // Scatters k_new/v_new [num_tokens, num_kv_heads, head_dim] (device) into the slots of
    // `slot_mapping` (device int32, slot = page * block_size + offset; slot < 0 skips the token).
    sci::Status Append(int64_t layer, const sci::Tensor& k_new, const sci::Tensor& v_new,
                       const int32_t* slot_mapping, int64_t num_tokens, sci::Stream* stream);

    // Copies the listed pages (device int32 ids) into a new [num_blocks, block_size, H_kv, D]
    // tensor; ids outside the pool give zero pages. For tests and debugging.
    sci::Result<sci::Tensor> GatherK(int64_t layer, const int32_t* block_ids, int64_t num_blocks,
                                     sci::Stream* stream) const;
    sci::Result<sci::Tensor> GatherV(int64_t layer, const int32_t* block_ids, int64_t num_blocks,
                                     sci::Stream* stream) const;

    // Zeroes the listed pages (device int32 ids) in every layer.
    sci::Status Reset(const int32_t* block_ids, int64_t num_blocks, sci::Stream* stream);

    const sci::Tensor& K(int64_t layer) const;
    const sci::Tensor& V(int64_t layer) const;
    KVCacheStats Stats() const;
    size_t MemoryBytes() const noexcept;
    int64_t LayerElements() const noexcept { return layer_elements_; }
    const KVCacheConfig& Config() const noexcept { return cfg_; }

private:
    sci::Result<sci::Tensor> GatherInternal(int64_t layer, const int32_t* block_ids,
                                            int64_t num_blocks, bool is_key,
                                            sci::Stream* stream) const;

    KVCacheConfig cfg_{};
    int64_t layer_elements_{0};
    std::vector<sci::Tensor> k_layers_;
    std::vector<sci::Tensor> v_layers_;
    KVCacheStats stats_{};
};

// Slots of tokens [seq_start, seq_start + num_tokens) of one sequence whose page list is
// block_table_row (max_blocks entries, -1 = unmapped).
SCI_ATTENTION_API sci::Result<std::vector<int32_t>> ComputeSlotMapping(
    const int32_t* block_table_row, int64_t seq_start, int64_t num_tokens, int64_t block_size,
    int64_t max_blocks);

// 2 * num_layers * num_blocks * block_size * num_kv_heads * head_dim * sizeof(dtype).
SCI_ATTENTION_API sci::Result<size_t> KvCacheBytes(const KVCacheConfig& cfg);

// floor(budget_bytes / bytes per page across K, V and all layers); 0 when a page does not fit.
SCI_ATTENTION_API int64_t MaxBlocksForBudget(const KVCacheConfig& cfg, size_t budget_bytes);

}  // namespace sca

#pragma once

#include <cstdint>
#include <vector>

#include "core/status.hpp"
#include "tensor/tensor.hpp"

#include "scicompute_attention/export.hpp"

namespace sci {
class Stream;
}  // namespace sci

namespace sca {

// Interface of the reference's BlockManager (include/scicompute_attention/block_manager.hpp:17-61).

// Per-sequence page lists: host [max_num_seqs, max_blocks_per_seq] int32 (-1 = empty) and its
// device copy, which is refreshed only when `revision` has moved past `synced_revision`.
struct BlockTable {
    std::vector<int32_t> host;
    sci::Tensor device;
    uint64_t revision{0};
    uint64_t synced_revision{0};
    int64_t max_num_seqs{0};
    int64_t max_blocks_per_seq{0};
};

// Exclusive page allocator (no sharing, no reference counts). Free pages sit on a LIFO stack
// seeded so that a fresh manager hands out 0, 1, 2, ...; allocation is all-or-nothing.
class SCI_ATTENTION_API BlockManager {
public:
    BlockManager() = default;

    static sci::Result<BlockManager> Create(int64_t num_blocks, int64_t max_num_seqs,
                                            int64_t max_blocks_per_seq, sci::Device& device);

    // `count` pages, or kKVCapacityExceeded with the state unchanged (failure counter aside).
    sci::Result<std::vector<int32_t>> Allocate(int64_t count);

    // Returns pages to the free stack in argument order; ids that are out of range or not in use
    // are skipped and counted as double frees.
    void Free(const int32_t* block_ids, int64_t count);

    int64_t NumFreeBlocks() const noexcept { return static_cast<int64_t>(free_list_.size()); }
    int64_t NumTotalBlocks() const noexcept { return num_blocks_; }
    int64_t AllocationFailures() const noexcept { return allocation_failures_; }
    int64_t DoubleFreeEvents() const noexcept { return double_free_events_; }

    // Writes `count` ids after the last used entry of the sequence's row.
    sci::Status AppendToTable(int64_t seq_id, const int32_t* block_ids, int64_t count);
    // Frees every page of the row (in row order) and clears it.
    sci::Status ResetSeq(int64_t seq_id);
    // Uploads the host table when it changed since the last upload.
    sci::Status SyncTableToDevice(sci::Stream* stream);

    const BlockTable& Table() const noexcept { return table_; }

private:
    int64_t num_blocks_{0};
    std::vector<int32_t> free_list_;
    std::vector<uint8_t> in_use_;
    BlockTable table_;
    int64_t allocation_failures_{0};
    int64_t double_free_events_{0};
};

}  // namespace sca

#pragma once

#include <cstdint>
#include <vector>

#include "core/status.hpp"
#include "tensor/tensor.hpp"

#include "scicompute_attention/block_manager.hpp"
#include "scicompute_attention/export.hpp"
#include "scicompute_attention/kv_cache.hpp"

namespace sci {
class Stream;
}  // namespace sci

namespace sca {

// Interface of the reference's PagedKVCache (include/scicompute_attention/paged_kv_cache.hpp:20-68).
//
// KVCache pages + a BlockManager + the page table the paged decode kernel reads
// ([max_num_seqs, max_blocks_per_seq] int32 in HBM, max_blocks_per_seq = num_blocks).
//
// Host state follows the reference exactly (which pages a sequence receives, in which order, the
// lengths, the revision counter). Two mechanics differ, without changing any observable value:
//   * SyncPageTable writes only the table entries that changed since the last sync (a sparse
//     update on the device; ForceSyncPageTable uploads the whole table);
//   * slot mappings (and the page ids ResetSeq clears) are staged in pinned host memory and copied
//     on the caller's stream.
// As in the reference, AppendTokens advances the sequence length on every call whatever the
// layer, so one call per token (layer 0) is its supported usage; multi-layer callers reserve the
// tokens once and write each layer (ReserveTokens / WriteReservedLayer).
class SCI_ATTENTION_API PagedKVCache {
public:
    PagedKVCache() = default;
    PagedKVCache(PagedKVCache&& other) noexcept;
    PagedKVCache& operator=(PagedKVCache&& other) noexcept;
    PagedKVCache(const PagedKVCache&) = delete;
    PagedKVCache& operator=(const PagedKVCache&) = delete;
    ~PagedKVCache();

    static sci::Result<PagedKVCache> Create(const KVCacheConfig& cfg, sci::Device& device);

    // Appends k_new/v_new [num_tokens, num_kv_heads, head_dim] (device) to sequence seq_id:
    // allocates the pages the new length needs, extends the page-table row, computes the slots
    // and scatters the tokens. Fails with kKVCapacityExceeded (state unchanged) when the pool
    // cannot supply the pages.
    sci::Status AppendTokens(int64_t seq_id, int64_t layer, const sci::Tensor& k_new,
                             const sci::Tensor& v_new, sci::Stream* stream);

    // One decode step for a batch: token i of k_new/v_new ([num_entries, num_kv_heads, head_dim],
    // device) is appended to sequence seq_ids[i], in order (an id may repeat). No counterpart in
    // the reference, which appends one sequence per call; the resulting state (pages, their order,
    // table rows, lengths, revision) equals that of one AppendTokens call per entry in order, but
    // the slots go up in one copy and the tokens in one scatter launch. All or nothing: when the
    // pool cannot supply every page the batch needs, nothing changes (kKVCapacityExceeded).
    sci::Status AppendTokensBatch(const int64_t* seq_ids, int64_t num_entries, int64_t layer,
                                  const sci::Tensor& k_new, const sci::Tensor& v_new,
                                  sci::Stream* stream);

    // Multi-layer appends (no counterpart in the reference, whose AppendTokens advances the
    // length on every call whatever the layer, so a model with several layers cannot store one
    // token per layer through it). A reservation allocates the pages, extends the rows, uploads
    // the slots and advances the lengths once: the host state afterwards (pages, their order,
    // rows, lengths, revision, append count) equals that of AppendTokens / AppendTokensBatch for
    // the same tokens, but no K/V is written. WriteReservedLayer then scatters one layer's K/V
    // rows ([reserved, num_kv_heads, head_dim], in reservation order) into the reserved slots;
    // a model calls it once per layer as its layers produce K and V. The reservation holds until
    // the next Reserve*, AppendTokens*, or ResetSeq call (they reuse the slot buffer).
    sci::Status ReserveTokens(int64_t seq_id, int64_t num_tokens, sci::Stream* stream);
    sci::Status ReserveTokensBatch(const int64_t* seq_ids, int64_t num_entries,
                                   sci::Stream* stream);
    sci::Status WriteReservedLayer(int64_t layer, const sci::Tensor& k_new,
                                   const sci::Tensor& v_new, sci::Stream* stream);
    int64_t ReservedTokens() const noexcept { return reserved_tokens_; }
    // One call for all layers: k_layers / v_layers are [num_layers, num_entries, num_kv_heads,
    // head_dim]; reserves one token per entry (ids may repeat, as in AppendTokensBatch) and writes
    // every layer's rows. Shapes are checked before anything changes.
    sci::Status AppendTokensBatchAllLayers(const int64_t* seq_ids, int64_t num_entries,
                                           const sci::Tensor& k_layers,
                                           const sci::Tensor& v_layers, sci::Stream* stream);

    // Zeroes the sequence's pages, returns them to the pool and clears its row.
    sci::Status ResetSeq(int64_t seq_id, sci::Stream* stream);

    const int32_t* PageTableDevicePtr() const noexcept;
    int64_t LogicalBlockCount(int64_t seq_id) const noexcept;
    int64_t SeqLength(int64_t seq_id) const noexcept;
    int64_t BlockSize() const noexcept { return cfg_.block_size; }
    int64_t MaxBlocksPerSeq() const noexcept { return max_blocks_per_seq_; }
    int64_t MaxNumSeqs() const noexcept { return cfg_.max_num_seqs; }
    const KVCache& Storage() const noexcept { return storage_; }
    KVCache& MutableStorage() noexcept { return storage_; }
    const BlockManager& Blocks() const noexcept { return blocks_; }

    // Brings the device page table up to date (no-op when nothing changed).
    sci::Status SyncPageTable(sci::Stream* stream);
    KVCacheStats Stats() const;
    // Uploads the whole host table regardless of the revision.
    sci::Status ForceSyncPageTable(sci::Stream* stream);

    // Host copy of the page table (row-major [max_num_seqs, max_blocks_per_seq]).
    const std::vector<int32_t>& PageTableHost() const noexcept { return page_table_host_; }
    uint64_t Revision() const noexcept { return revision_; }
    uint64_t SyncedRevision() const noexcept { return synced_revision_; }

private:
    sci::Status ReserveSlots(int64_t seq_id, int64_t num_new, const char* who, sci::Stream* stream);
    sci::Status ReserveBatchSlots(const int64_t* seq_ids, int64_t num_entries, const char* who,
                                  sci::Stream* stream);
    sci::Status CheckTokenRows(const sci::Tensor& k_new, const sci::Tensor& v_new, int64_t rows,
                               const char* who) const;
    sci::Result<int32_t*> Staging(int64_t entries);
    sci::Status StagingSubmitted(void* stream, bool blocking);
    void ReleaseStaging() noexcept;

    KVCacheConfig cfg_{};
    int64_t max_blocks_per_seq_{0};
    KVCache storage_{};
    BlockManager blocks_{};
    std::vector<int64_t> seq_lengths_;
    std::vector<std::vector<int32_t>> seq_blocks_;
    std::vector<int32_t> page_table_host_;
    std::vector<int64_t> pending_entries_;  // flat table indices changed since the last sync
    sci::Tensor page_table_device_;
    sci::Tensor slot_mapping_device_;       // slots of the last append / ids of the last reset
    int64_t slot_mapping_capacity_{0};
    int64_t reserved_tokens_{0};            // slots of the last reservation (0: none)
    sci::Tensor pairs_device_;              // (index, value) pairs of the last sparse sync
    int64_t pairs_capacity_{0};
    int32_t* staging_host_{nullptr};        // pinned host staging for both uploads
    int64_t staging_capacity_{0};
    void* staging_event_{nullptr};          // completes when the staging memory is free again
    uint64_t revision_{0};
    uint64_t synced_revision_{0};
    int64_t num_appends_{0};
    int64_t num_resets_{0};
};

}  // namespace sca

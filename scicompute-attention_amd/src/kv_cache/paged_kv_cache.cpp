// Multi-sequence paged KV cache: pages (KVCache) + allocator (BlockManager) + the page table the
// paged decode kernel reads.
//
// Host-visible state follows the reference's src/kv_cache/paged_kv_cache.cpp:13-211 exactly: which
// pages a sequence gets and in which order, lengths, revision, counters, error texts, the
// "no partial update when the pool is exhausted" rule and the clear-then-free-then-unmap order of
// ResetSeq. The device side is MI355X-specific:
//   * the page table is refreshed by a sparse update of the entries that changed since the last
//     sync (one pinned-memory copy + one scatter kernel) instead of re-uploading
//     max_num_seqs x num_blocks entries; ForceSyncPageTable still uploads everything;
//   * slot mappings are staged in pinned memory and copied on the caller's stream, so an append is
//     two asynchronous operations on that stream. An event guards reuse of the staging memory.
//   With stream == nullptr both paths wait for their copy before returning, as the reference's
//   synchronous copies do.

#include <algorithm>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "device/device.hpp"
#include "device/stream.hpp"
#include "runtime/internal.hpp"
#include "scicompute_attention/paged_kv_cache.hpp"

namespace sca {
namespace {

constexpr int64_t kMinStagingEntries = 1024;

}  // namespace

// ---- lifetime ----------------------------------------------------------------------------------

PagedKVCache::PagedKVCache(PagedKVCache&& o) noexcept
    : cfg_(o.cfg_),
      max_blocks_per_seq_(o.max_blocks_per_seq_),
      storage_(std::move(o.storage_)),
      blocks_(std::move(o.blocks_)),
      seq_lengths_(std::move(o.seq_lengths_)),
      seq_blocks_(std::move(o.seq_blocks_)),
      page_table_host_(std::move(o.page_table_host_)),
      pending_entries_(std::move(o.pending_entries_)),
      page_table_device_(std::move(o.page_table_device_)),
      slot_mapping_device_(std::move(o.slot_mapping_device_)),
      slot_mapping_capacity_(o.slot_mapping_capacity_),
      reserved_tokens_(o.reserved_tokens_),
      pairs_device_(std::move(o.pairs_device_)),
      pairs_capacity_(o.pairs_capacity_),
      staging_host_(o.staging_host_),
      staging_capacity_(o.staging_capacity_),
      staging_event_(o.staging_event_),
      revision_(o.revision_),
      synced_revision_(o.synced_revision_),
      num_appends_(o.num_appends_),
      num_resets_(o.num_resets_) {
    o.staging_host_ = nullptr;
    o.staging_capacity_ = 0;
    o.staging_event_ = nullptr;
}

PagedKVCache& PagedKVCache::operator=(PagedKVCache&& o) noexcept {
    if (this != &o) {
        ReleaseStaging();
        cfg_ = o.cfg_;
        max_blocks_per_seq_ = o.max_blocks_per_seq_;
        storage_ = std::move(o.storage_);
        blocks_ = std::move(o.blocks_);
        seq_lengths_ = std::move(o.seq_lengths_);
        seq_blocks_ = std::move(o.seq_blocks_);
        page_table_host_ = std::move(o.page_table_host_);
        pending_entries_ = std::move(o.pending_entries_);
        page_table_device_ = std::move(o.page_table_device_);
        slot_mapping_device_ = std::move(o.slot_mapping_device_);
        slot_mapping_capacity_ = o.slot_mapping_capacity_;
        reserved_tokens_ = o.reserved_tokens_;
        pairs_device_ = std::move(o.pairs_device_);
        pairs_capacity_ = o.pairs_capacity_;
        staging_host_ = o.staging_host_;
        staging_capacity_ = o.staging_capacity_;
        staging_event_ = o.staging_event_;
        revision_ = o.revision_;
        synced_revision_ = o.synced_revision_;
        num_appends_ = o.num_appends_;
        num_resets_ = o.num_resets_;
        o.staging_host_ = nullptr;
        o.staging_capacity_ = 0;
        o.staging_event_ = nullptr;
    }
    return *this;
}

PagedKVCache::~PagedKVCache() { ReleaseStaging(); }

void PagedKVCache::ReleaseStaging() noexcept {
    if (staging_event_ != nullptr) {
        sca_hip_event_synchronize(staging_event_);
        sca_hip_event_destroy(staging_event_);
        staging_event_ = nullptr;
    }
    if (staging_host_ != nullptr) {
        sca_hip_host_free(staging_host_);
        staging_host_ = nullptr;
    }
    staging_capacity_ = 0;
}

// Pinned staging of at least `entries` int32 values, free to overwrite (its last copy finished).
sci::Result<int32_t*> PagedKVCache::Staging(int64_t entries) {
    if (staging_event_ == nullptr) {
        const sci::Status st =
            runtime::StatusFromHip(sca_hip_event_create(&staging_event_), "staging event");
        if (!st.ok()) return sci::MakeUnexpected<int32_t*>(st);
    } else {
        const sci::Status st =
            runtime::StatusFromHip(sca_hip_event_synchronize(staging_event_), "staging wait");
        if (!st.ok()) return sci::MakeUnexpected<int32_t*>(st);
    }
    if (staging_capacity_ < entries) {
        if (staging_host_ != nullptr) sca_hip_host_free(staging_host_);
        staging_host_ = nullptr;
        staging_capacity_ = 0;
        const int64_t capacity = std::max<int64_t>(entries, kMinStagingEntries);
        void* p = nullptr;
        if (sca_hip_host_malloc(&p, static_cast<size_t>(capacity) * sizeof(int32_t)) != 0) {
            return sci::MakeUnexpected<int32_t*>(MakeStatus(
                AttnStatusCode::kKVCapacityExceeded, "PagedKVCache: pinned staging allocation failed"));
        }
        staging_host_ = static_cast<int32_t*>(p);
        staging_capacity_ = capacity;
    }
    return sci::Ok(staging_host_);
}

// Marks the staging memory busy until the work queued so far on `stream` has run; with
// `blocking` the call waits for it.
sci::Status PagedKVCache::StagingSubmitted(void* stream, bool blocking) {
    sci::Status st =
        runtime::StatusFromHip(sca_hip_event_record(staging_event_, stream), "staging record");
    if (st.ok() && blocking) {
        st = runtime::StatusFromHip(sca_hip_event_synchronize(staging_event_), "staging wait");
    }
    return st;
}

sci::Result<PagedKVCache> PagedKVCache::Create(const KVCacheConfig& cfg, sci::Device& device) {
    if (cfg.max_num_seqs <= 0) {
        return sci::MakeUnexpected<PagedKVCache>(MakeStatus(
            AttnStatusCode::kShapeMismatch,
            "PagedKVCacheConfig invalid: max_num_seqs=" + std::to_string(cfg.max_num_seqs)));
    }
    sci::Result<KVCache> storage = KVCache::Create(cfg, device);
    if (!storage.ok()) return sci::MakeUnexpected<PagedKVCache>(storage.error());
    // Pages are exclusive, so one row can hold every page of the pool.
    const int64_t row_len = cfg.num_blocks;
    sci::Result<BlockManager> blocks =
        BlockManager::Create(cfg.num_blocks, cfg.max_num_seqs, row_len, device);
    if (!blocks.ok()) return sci::MakeUnexpected<PagedKVCache>(blocks.error());

    PagedKVCache cache;
    cache.cfg_ = cfg;
    cache.max_blocks_per_seq_ = row_len;
    cache.storage_ = std::move(*storage);
    cache.blocks_ = std::move(*blocks);
    cache.seq_lengths_.assign(static_cast<size_t>(cfg.max_num_seqs), 0);
    cache.seq_blocks_.assign(static_cast<size_t>(cfg.max_num_seqs), {});
    cache.page_table_host_.assign(static_cast<size_t>(cfg.max_num_seqs * row_len), -1);
    cache.page_table_device_ = sci::Tensor(sci::TensorShape({cfg.max_num_seqs, row_len}),
                                           sci::DType::kInt32, device);
    if (cache.page_table_device_.data() == nullptr) {
        return sci::MakeUnexpected<PagedKVCache>(MakeStatus(
            AttnStatusCode::kKVCapacityExceeded, "PagedKVCache: page table allocation failed"));
    }
    cache.page_table_device_.copy_from(cache.page_table_host_.data(),
                                       cache.page_table_host_.size() * sizeof(int32_t));
    device.synchronize();
    cache.revision_ = 1;
    cache.synced_revision_ = 1;
    return sci::Ok(std::move(cache));
}

// ---- appends and resets ------------------------------------------------------------------------

sci::Status PagedKVCache::AppendTokens(int64_t seq_id, int64_t layer, const sci::Tensor& k_new,
                                       const sci::Tensor& v_new, sci::Stream* stream) {
    if (seq_id < 0 || seq_id >= cfg_.max_num_seqs) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::AppendTokens seq_id=" + std::to_string(seq_id) +
                              " out of range [0," + std::to_string(cfg_.max_num_seqs) + ")");
    }
    if (layer < 0 || layer >= cfg_.num_layers) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::AppendTokens layer=" + std::to_string(layer) +
                              " out of range [0," + std::to_string(cfg_.num_layers) + ")");
    }
    if (k_new.ndims() != 3 || v_new.ndims() != 3 || k_new.dim(0) != v_new.dim(0)) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::AppendTokens expects [num_tokens, n_kv_heads, head_dim] "
                          "tensors");
    }
    const int64_t num_new = k_new.dim(0);
    if (num_new <= 0) {
        return MakeStatus(AttnStatusCode::kShapeMismatch, "PagedKVCache::AppendTokens: 0 tokens");
    }
    const int64_t current_len = seq_lengths_[static_cast<size_t>(seq_id)];
    sci::Status st = ReserveSlots(seq_id, num_new, "PagedKVCache::AppendTokens", stream);
    if (!st.ok()) return st;
    st = storage_.Append(layer, k_new, v_new,
                         static_cast<const int32_t*>(slot_mapping_device_.data()), num_new, stream);
    if (!st.ok()) return st;  // pages stay attached; ResetSeq recovers
    seq_lengths_[static_cast<size_t>(seq_id)] = current_len + num_new;
    ++revision_;
    ++num_appends_;
    return sci::Status::Ok();
}

// Pages for num_new more tokens of seq_id (all or nothing), the row's new tail, and the slots of
// the tokens uploaded to slot_mapping_device_ on the stream. Lengths and the revision are left to
// the caller. `who` names the entry point in the capacity message.
sci::Status PagedKVCache::ReserveSlots(int64_t seq_id, int64_t num_new, const char* who,
                                       sci::Stream* stream) {
    reserved_tokens_ = 0;  // the slot buffer is about to hold this call's slots
    const size_t sid = static_cast<size_t>(seq_id);
    std::vector<int32_t>& owned = seq_blocks_[sid];
    const int64_t current_len = seq_lengths_[sid];
    const int64_t needed = (current_len + num_new + cfg_.block_size - 1) / cfg_.block_size;
    const int64_t missing = needed - static_cast<int64_t>(owned.size());

    std::vector<int32_t> fresh;
    if (missing > 0) {
        sci::Result<std::vector<int32_t>> got = blocks_.Allocate(missing);
        if (!got.ok()) {
            return MakeStatus(AttnStatusCode::kKVCapacityExceeded,
                              std::string(who) + " seq=" + std::to_string(seq_id) + " needs " +
                                  std::to_string(missing) + " more blocks but only " +
                                  std::to_string(blocks_.NumFreeBlocks()) + " are free");
        }
        fresh = std::move(*got);
        const sci::Status st =
            blocks_.AppendToTable(seq_id, fresh.data(), static_cast<int64_t>(fresh.size()));
        if (!st.ok()) {
            blocks_.Free(fresh.data(), static_cast<int64_t>(fresh.size()));
            return st;
        }
    }
    // The row always equals the owned page list followed by -1, so only the new tail changes.
    int32_t* row = page_table_host_.data() + seq_id * max_blocks_per_seq_;
    for (int32_t page : fresh) {
        const int64_t pos = static_cast<int64_t>(owned.size());
        owned.push_back(page);
        row[pos] = page;
        pending_entries_.push_back(seq_id * max_blocks_per_seq_ + pos);
    }

    const sci::Result<std::vector<int32_t>> slots =
        ComputeSlotMapping(row, current_len, num_new, cfg_.block_size, max_blocks_per_seq_);
    if (!slots.ok()) return slots.error();

    if (slot_mapping_capacity_ < num_new) {
        const int64_t capacity = std::max<int64_t>(num_new, kMinStagingEntries);
        slot_mapping_device_ = sci::Tensor(sci::TensorShape({capacity}), sci::DType::kInt32,
                                           page_table_device_.device());
        if (slot_mapping_device_.data() == nullptr) {
            slot_mapping_capacity_ = 0;
            return MakeStatus(AttnStatusCode::kKVCapacityExceeded,
                              "PagedKVCache: slot-mapping buffer allocation failed");
        }
        slot_mapping_capacity_ = capacity;
    }
    sci::Result<int32_t*> staging = Staging(num_new);
    if (!staging.ok()) return staging.error();
    std::memcpy(*staging, slots->data(), static_cast<size_t>(num_new) * sizeof(int32_t));
    void* s = runtime::StreamHandle(stream);
    sci::Status st = runtime::StatusFromHip(
        sca_hip_memcpy_async(slot_mapping_device_.data(), *staging,
                             static_cast<size_t>(num_new) * sizeof(int32_t), SCA_COPY_H2D, s),
        "PagedKVCache slot upload");
    if (st.ok()) st = StagingSubmitted(s, stream == nullptr);
    return st;
}

sci::Status PagedKVCache::AppendTokensBatch(const int64_t* seq_ids, int64_t num_entries,
                                            int64_t layer, const sci::Tensor& k_new,
                                            const sci::Tensor& v_new, sci::Stream* stream) {
    if (seq_ids == nullptr || num_entries <= 0) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::AppendTokensBatch needs at least one sequence id");
    }
    if (layer < 0 || layer >= cfg_.num_layers) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::AppendTokensBatch layer=" + std::to_string(layer) +
                              " out of range [0," + std::to_string(cfg_.num_layers) + ")");
    }
    const sci::Status shape = CheckTokenRows(k_new, v_new, num_entries,
                                             "PagedKVCache::AppendTokensBatch");
    if (!shape.ok()) return shape;
    const sci::Status st = ReserveBatchSlots(seq_ids, num_entries,
                                             "PagedKVCache::AppendTokensBatch", stream);
    if (!st.ok()) return st;
    reserved_tokens_ = 0;
    return storage_.Append(layer, k_new, v_new,
                           static_cast<const int32_t*>(slot_mapping_device_.data()), num_entries,
                           stream);
}

// k_new / v_new are [rows, num_kv_heads, head_dim] tensors of the cache's dtype.
sci::Status PagedKVCache::CheckTokenRows(const sci::Tensor& k_new, const sci::Tensor& v_new,
                                         int64_t rows, const char* who) const {
    if (k_new.ndims() != 3 || v_new.ndims() != 3 || k_new.dim(0) != rows ||
        v_new.dim(0) != rows) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          std::string(who) + " expects [num_entries, n_kv_heads, head_dim] "
                                             "tensors with one token per sequence id");
    }
    if (k_new.dim(1) != cfg_.num_kv_heads || k_new.dim(2) != cfg_.head_dim ||
        v_new.dim(1) != cfg_.num_kv_heads || v_new.dim(2) != cfg_.head_dim ||
        k_new.dtype() != cfg_.dtype || v_new.dtype() != cfg_.dtype) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          std::string(who) + " token shape differs from the cache's [" +
                              std::to_string(cfg_.num_kv_heads) + ", " +
                              std::to_string(cfg_.head_dim) + "]");
    }
    return sci::Status::Ok();
}

// Pages, rows, slots (uploaded), lengths and revision for one token per entry of seq_ids, in
// order, exactly as one AppendTokens call per entry would leave them; all or nothing.
sci::Status PagedKVCache::ReserveBatchSlots(const int64_t* seq_ids, int64_t num_entries,
                                            const char* who, sci::Stream* stream) {
    reserved_tokens_ = 0;
    // Pages the whole batch needs, before anything changes.
    std::vector<int64_t> lens;   // running lengths of the sequences touched, by first appearance
    std::vector<int64_t> owned;  // their page counts
    std::vector<int64_t> first(static_cast<size_t>(cfg_.max_num_seqs), -1);  // by sequence id
    int64_t missing = 0;
    for (int64_t i = 0; i < num_entries; ++i) {
        const int64_t id = seq_ids[i];
        if (id < 0 || id >= cfg_.max_num_seqs) {
            return MakeStatus(AttnStatusCode::kShapeMismatch,
                              std::string(who) + " seq_id=" + std::to_string(id) +
                                  " out of range [0," + std::to_string(cfg_.max_num_seqs) + ")");
        }
        int64_t& slot = first[static_cast<size_t>(id)];
        if (slot < 0) {
            slot = static_cast<int64_t>(lens.size());
            lens.push_back(seq_lengths_[static_cast<size_t>(id)]);
            owned.push_back(static_cast<int64_t>(seq_blocks_[static_cast<size_t>(id)].size()));
        }
        const size_t u = static_cast<size_t>(slot);
        const int64_t needed = (lens[u] + 1 + cfg_.block_size - 1) / cfg_.block_size;
        if (needed > owned[u]) {
            missing += needed - owned[u];
            owned[u] = needed;
        }
        if (needed > max_blocks_per_seq_) {
            return MakeStatus(AttnStatusCode::kKVCapacityExceeded,
                              std::string(who) + " seq=" + std::to_string(id) +
                                  " would exceed " + std::to_string(max_blocks_per_seq_) +
                                  " pages");
        }
        ++lens[u];
    }
    if (missing > blocks_.NumFreeBlocks()) {
        return MakeStatus(AttnStatusCode::kKVCapacityExceeded,
                          std::string(who) + " needs " + std::to_string(missing) +
                              " more blocks but only " + std::to_string(blocks_.NumFreeBlocks()) +
                              " are free");
    }
    if (slot_mapping_capacity_ < num_entries) {
        const int64_t capacity = std::max<int64_t>(num_entries, kMinStagingEntries);
        slot_mapping_device_ = sci::Tensor(sci::TensorShape({capacity}), sci::DType::kInt32,
                                           page_table_device_.device());
        if (slot_mapping_device_.data() == nullptr) {
            slot_mapping_capacity_ = 0;
            return MakeStatus(AttnStatusCode::kKVCapacityExceeded,
                              "PagedKVCache: slot-mapping buffer allocation failed");
        }
        slot_mapping_capacity_ = capacity;
    }
    sci::Result<int32_t*> staging = Staging(num_entries);
    if (!staging.ok()) return staging.error();

    // Entry by entry, exactly as AppendTokens would: page (if the token opens one), table tail,
    // slot; lengths and the revision advance per entry.
    int32_t* slots = *staging;
    for (int64_t i = 0; i < num_entries; ++i) {
        const int64_t id = seq_ids[i];
        const size_t sid = static_cast<size_t>(id);
        std::vector<int32_t>& pages = seq_blocks_[sid];
        const int64_t len = seq_lengths_[sid];
        int32_t* row = page_table_host_.data() + id * max_blocks_per_seq_;
        if (len / cfg_.block_size >= static_cast<int64_t>(pages.size())) {
            sci::Result<std::vector<int32_t>> got = blocks_.Allocate(1);
            if (!got.ok()) return got.error();  // cannot happen: counted above
            const sci::Status st = blocks_.AppendToTable(id, got->data(), 1);
            if (!st.ok()) {
                blocks_.Free(got->data(), 1);
                return st;
            }
            const int64_t pos = static_cast<int64_t>(pages.size());
            pages.push_back((*got)[0]);
            row[pos] = (*got)[0];
            pending_entries_.push_back(id * max_blocks_per_seq_ + pos);
        }
        slots[i] = static_cast<int32_t>(static_cast<int64_t>(row[len / cfg_.block_size]) *
                                            cfg_.block_size +
                                        len % cfg_.block_size);
        seq_lengths_[sid] = len + 1;
        ++revision_;
        ++num_appends_;
    }
    void* s = runtime::StreamHandle(stream);
    sci::Status st = runtime::StatusFromHip(
        sca_hip_memcpy_async(slot_mapping_device_.data(), slots,
                             static_cast<size_t>(num_entries) * sizeof(int32_t), SCA_COPY_H2D, s),
        "PagedKVCache batch slot upload");
    if (st.ok()) st = StagingSubmitted(s, stream == nullptr);
    return st;
}

// ---- multi-layer appends -----------------------------------------------------------------------

sci::Status PagedKVCache::ReserveTokens(int64_t seq_id, int64_t num_tokens, sci::Stream* stream) {
    reserved_tokens_ = 0;
    if (seq_id < 0 || seq_id >= cfg_.max_num_seqs) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::ReserveTokens seq_id=" + std::to_string(seq_id) +
                              " out of range [0," + std::to_string(cfg_.max_num_seqs) + ")");
    }
    if (num_tokens <= 0) {
        return MakeStatus(AttnStatusCode::kShapeMismatch, "PagedKVCache::ReserveTokens: 0 tokens");
    }
    const sci::Status st = ReserveSlots(seq_id, num_tokens, "PagedKVCache::ReserveTokens", stream);
    if (!st.ok()) return st;
    seq_lengths_[static_cast<size_t>(seq_id)] += num_tokens;
    ++revision_;
    ++num_appends_;
    reserved_tokens_ = num_tokens;
    return sci::Status::Ok();
}

sci::Status PagedKVCache::ReserveTokensBatch(const int64_t* seq_ids, int64_t num_entries,
                                             sci::Stream* stream) {
    reserved_tokens_ = 0;
    if (seq_ids == nullptr || num_entries <= 0) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::ReserveTokensBatch needs at least one sequence id");
    }
    const sci::Status st =
        ReserveBatchSlots(seq_ids, num_entries, "PagedKVCache::ReserveTokensBatch", stream);
    if (!st.ok()) return st;
    reserved_tokens_ = num_entries;
    return sci::Status::Ok();
}

sci::Status PagedKVCache::WriteReservedLayer(int64_t layer, const sci::Tensor& k_new,
                                             const sci::Tensor& v_new, sci::Stream* stream) {
    if (reserved_tokens_ <= 0) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::WriteReservedLayer: no reservation (call ReserveTokens or "
                          "ReserveTokensBatch first)");
    }
    if (layer < 0 || layer >= cfg_.num_layers) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::WriteReservedLayer layer=" + std::to_string(layer) +
                              " out of range [0," + std::to_string(cfg_.num_layers) + ")");
    }
    const sci::Status shape =
        CheckTokenRows(k_new, v_new, reserved_tokens_, "PagedKVCache::WriteReservedLayer");
    if (!shape.ok()) return shape;
    return storage_.Append(layer, k_new, v_new,
                           static_cast<const int32_t*>(slot_mapping_device_.data()),
                           reserved_tokens_, stream);
}


sci::Status PagedKVCache::AppendTokensBatchAllLayers(const int64_t* seq_ids, int64_t num_entries,
                                                     const sci::Tensor& k_layers,
                                                     const sci::Tensor& v_layers,
                                                     sci::Stream* stream) {
    const char* who = "PagedKVCache::AppendTokensBatchAllLayers";
    if (seq_ids == nullptr || num_entries <= 0) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          std::string(who) + " needs at least one sequence id");
    }
    for (const sci::Tensor* t : {&k_layers, &v_layers}) {
        if (t->ndims() != 4 || t->dim(0) != cfg_.num_layers || t->dim(1) != num_entries ||
            t->dim(2) != cfg_.num_kv_heads || t->dim(3) != cfg_.head_dim ||
            t->dtype() != cfg_.dtype) {
            return MakeStatus(AttnStatusCode::kShapeMismatch,
                              std::string(who) + " expects [num_layers, num_entries, n_kv_heads, "
                                                 "head_dim] = [" +
                                  std::to_string(cfg_.num_layers) + ", " +
                                  std::to_string(num_entries) + ", " +
                                  std::to_string(cfg_.num_kv_heads) + ", " +
                                  std::to_string(cfg_.head_dim) + "] tensors of the cache's dtype");
        }
    }
    sci::Status st = ReserveBatchSlots(seq_ids, num_entries, who, stream);
    if (!st.ok()) return st;
    reserved_tokens_ = num_entries;
    const int64_t layer_bytes = num_entries * cfg_.num_kv_heads * cfg_.head_dim *
                                static_cast<int64_t>(sci::kDTypeSize(cfg_.dtype));
    const sci::TensorShape rows({num_entries, cfg_.num_kv_heads, cfg_.head_dim});
    for (int64_t layer = 0; layer < cfg_.num_layers; ++layer) {
        const sci::Tensor k(rows, cfg_.dtype, k_layers.device(),
                            static_cast<char*>(const_cast<void*>(k_layers.data())) + layer * layer_bytes);
        const sci::Tensor v(rows, cfg_.dtype, v_layers.device(),
                            static_cast<char*>(const_cast<void*>(v_layers.data())) + layer * layer_bytes);
        st = WriteReservedLayer(layer, k, v, stream);
        if (!st.ok()) return st;
    }
    return sci::Status::Ok();
}

sci::Status PagedKVCache::ResetSeq(int64_t seq_id, sci::Stream* stream) {
    reserved_tokens_ = 0;  // the slot buffer carries the page ids below
    if (seq_id < 0 || seq_id >= cfg_.max_num_seqs) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "PagedKVCache::ResetSeq seq_id=" + std::to_string(seq_id) +
                              " out of range");
    }
    std::vector<int32_t>& owned = seq_blocks_[static_cast<size_t>(seq_id)];
    if (!owned.empty()) {
        // Clear the pages first (their ids must be device-resident for the kernel), then release
        // them, then unmap the row.
        const int64_t n = static_cast<int64_t>(owned.size());
        if (slot_mapping_capacity_ < n) {
            const int64_t capacity = std::max<int64_t>(n, kMinStagingEntries);
            slot_mapping_device_ = sci::Tensor(sci::TensorShape({capacity}), sci::DType::kInt32,
                                               page_table_device_.device());
            if (slot_mapping_device_.data() == nullptr) {
                slot_mapping_capacity_ = 0;
                return MakeStatus(AttnStatusCode::kKVCapacityExceeded,
                                  "PagedKVCache: block-id buffer allocation failed");
            }
            slot_mapping_capacity_ = capacity;
        }
        sci::Result<int32_t*> staging = Staging(n);
        if (!staging.ok()) return staging.error();
        std::memcpy(*staging, owned.data(), static_cast<size_t>(n) * sizeof(int32_t));
        void* s = runtime::StreamHandle(stream);
        sci::Status st = runtime::StatusFromHip(
            sca_hip_memcpy_async(slot_mapping_device_.data(), *staging,
                                 static_cast<size_t>(n) * sizeof(int32_t), SCA_COPY_H2D, s),
            "PagedKVCache block-id upload");
        if (st.ok()) st = StagingSubmitted(s, stream == nullptr);
        if (st.ok()) {
            st = storage_.Reset(static_cast<const int32_t*>(slot_mapping_device_.data()), n,
                                stream);
        }
        if (!st.ok()) return st;
        for (int64_t i = 0; i < n; ++i) pending_entries_.push_back(seq_id * max_blocks_per_seq_ + i);
    }
    blocks_.ResetSeq(seq_id);
    owned.clear();
    seq_lengths_[static_cast<size_t>(seq_id)] = 0;
    int32_t* row = page_table_host_.data() + seq_id * max_blocks_per_seq_;
    std::fill(row, row + max_blocks_per_seq_, -1);
    ++revision_;
    ++num_resets_;
    return sci::Status::Ok();
}

// ---- page table --------------------------------------------------------------------------------

const int32_t* PagedKVCache::PageTableDevicePtr() const noexcept {
    return static_cast<const int32_t*>(page_table_device_.data());
}

int64_t PagedKVCache::LogicalBlockCount(int64_t seq_id) const noexcept {
    if (seq_id < 0 || seq_id >= cfg_.max_num_seqs) return 0;
    return static_cast<int64_t>(seq_blocks_[static_cast<size_t>(seq_id)].size());
}

int64_t PagedKVCache::SeqLength(int64_t seq_id) const noexcept {
    if (seq_id < 0 || seq_id >= cfg_.max_num_seqs) return 0;
    return seq_lengths_[static_cast<size_t>(seq_id)];
}

sci::Status PagedKVCache::SyncPageTable(sci::Stream* stream) {
    if (revision_ == synced_revision_) return sci::Status::Ok();
    if (page_table_device_.data() == nullptr) {
        return MakeStatus(AttnStatusCode::kShapeMismatch, "PagedKVCache: page table missing");
    }
    const int64_t table_entries = static_cast<int64_t>(page_table_host_.size());
    const int64_t n = static_cast<int64_t>(pending_entries_.size());
    // A sparse update moves 8 B per changed entry; past half the table a full copy is cheaper.
    if (n * 2 * 2 > table_entries || table_entries > (int64_t{1} << 31)) {
        return ForceSyncPageTable(stream);
    }
    if (n > 0) {
        if (pairs_capacity_ < n) {
            const int64_t capacity = std::max<int64_t>(n, kMinStagingEntries);
            pairs_device_ = sci::Tensor(sci::TensorShape({2 * capacity}), sci::DType::kInt32,
                                        page_table_device_.device());
            if (pairs_device_.data() == nullptr) {
                pairs_capacity_ = 0;
                return ForceSyncPageTable(stream);
            }
            pairs_capacity_ = capacity;
        }
        sci::Result<int32_t*> staging = Staging(2 * n);
        if (!staging.ok()) return staging.error();
        int32_t* pairs = *staging;
        for (int64_t i = 0; i < n; ++i) {
            const int64_t flat = pending_entries_[static_cast<size_t>(i)];
            pairs[2 * i] = static_cast<int32_t>(flat);
            pairs[2 * i + 1] = page_table_host_[static_cast<size_t>(flat)];
        }
        void* s = runtime::StreamHandle(stream);
        sci::Status st = runtime::StatusFromHip(
            sca_hip_memcpy_async(pairs_device_.data(), pairs,
                                 static_cast<size_t>(2 * n) * sizeof(int32_t), SCA_COPY_H2D, s),
            "PagedKVCache page-table update upload");
        if (st.ok()) {
            st = runtime::StatusFromHip(
                sca_hip_i32_scatter(static_cast<int32_t*>(page_table_device_.data()),
                                    table_entries, static_cast<const int32_t*>(pairs_device_.data()),
                                    n, s),
                "PagedKVCache page-table update");
        }
        if (st.ok()) st = StagingSubmitted(s, stream == nullptr);
        if (!st.ok()) return st;
    }
    pending_entries_.clear();
    synced_revision_ = revision_;
    return sci::Status::Ok();
}

sci::Status PagedKVCache::ForceSyncPageTable(sci::Stream* stream) {
    if (page_table_device_.data() == nullptr) {
        return MakeStatus(AttnStatusCode::kShapeMismatch, "PagedKVCache: page table missing");
    }
    const size_t bytes = page_table_host_.size() * sizeof(int32_t);
    if (stream != nullptr) {
        page_table_device_.device().copy_async(page_table_device_.data(), page_table_host_.data(),
                                               bytes, *stream);
    } else {
        page_table_device_.copy_from(page_table_host_.data(), bytes);
    }
    pending_entries_.clear();
    synced_revision_ = revision_;
    return sci::Status::Ok();
}

KVCacheStats PagedKVCache::Stats() const {
    KVCacheStats stats = storage_.Stats();
    stats.num_blocks = blocks_.NumTotalBlocks();
    stats.free_blocks = blocks_.NumFreeBlocks();
    stats.used_blocks = stats.num_blocks - stats.free_blocks;
    stats.num_appends = num_appends_;
    stats.num_resets = num_resets_;
    return stats;
}

}  // namespace sca

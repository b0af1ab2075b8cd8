// Exclusive page allocator and per-sequence page table.
// State transitions follow the reference's src/kv_cache/block_manager.cpp:11-144 exactly (the
// free stack order, all-or-nothing allocation, double-free accounting, revision counting), since
// the page ids a sequence receives are observable through the page table.

#include <string>

#include "device/device.hpp"
#include "device/stream.hpp"
#include "runtime/internal.hpp"
#include "scicompute_attention/block_manager.hpp"

namespace sca {

sci::Result<BlockManager> BlockManager::Create(int64_t num_blocks, int64_t max_num_seqs,
                                               int64_t max_blocks_per_seq, sci::Device& device) {
    if (num_blocks <= 0 || max_num_seqs <= 0 || max_blocks_per_seq <= 0) {
        return sci::MakeUnexpected<BlockManager>(MakeStatus(
            AttnStatusCode::kShapeMismatch,
            "BlockManager::Create invalid arguments: num_blocks=" + std::to_string(num_blocks) +
                ", max_num_seqs=" + std::to_string(max_num_seqs) +
                ", max_blocks_per_seq=" + std::to_string(max_blocks_per_seq)));
    }
    BlockManager bm;
    bm.num_blocks_ = num_blocks;
    bm.in_use_.assign(static_cast<size_t>(num_blocks), 0);
    // Top of the stack is the back: seeding N-1 .. 0 makes a fresh manager hand out 0, 1, 2, ...
    bm.free_list_.resize(static_cast<size_t>(num_blocks));
    for (int64_t i = 0; i < num_blocks; ++i) {
        bm.free_list_[static_cast<size_t>(i)] = static_cast<int32_t>(num_blocks - 1 - i);
    }
    bm.table_.max_num_seqs = max_num_seqs;
    bm.table_.max_blocks_per_seq = max_blocks_per_seq;
    bm.table_.host.assign(static_cast<size_t>(max_num_seqs * max_blocks_per_seq), -1);
    bm.table_.device = sci::Tensor(sci::TensorShape({max_num_seqs, max_blocks_per_seq}),
                                   sci::DType::kInt32, device);
    if (bm.table_.device.data() == nullptr) {
        return sci::MakeUnexpected<BlockManager>(MakeStatus(
            AttnStatusCode::kKVCapacityExceeded,
            "BlockManager: page table allocation of " +
                std::to_string(max_num_seqs * max_blocks_per_seq * 4) + " B failed"));
    }
    // The device copy starts as the host table (all -1).
    bm.table_.device.copy_from(bm.table_.host.data(), bm.table_.host.size() * sizeof(int32_t));
    device.synchronize();
    return sci::Ok(std::move(bm));
}

sci::Result<std::vector<int32_t>> BlockManager::Allocate(int64_t count) {
    using Ids = std::vector<int32_t>;
    if (count <= 0) {
        return sci::MakeUnexpected<Ids>(MakeStatus(
            AttnStatusCode::kShapeMismatch, "BlockManager::Allocate count=" + std::to_string(count)));
    }
    const int64_t available = static_cast<int64_t>(free_list_.size());
    if (count > available) {
        ++allocation_failures_;
        return sci::MakeUnexpected<Ids>(MakeStatus(
            AttnStatusCode::kKVCapacityExceeded,
            "BlockManager::Allocate requested " + std::to_string(count) + " blocks but only " +
                std::to_string(available) + " of " + std::to_string(num_blocks_) + " are free"));
    }
    Ids ids(static_cast<size_t>(count));
    for (auto& id : ids) {
        id = free_list_.back();
        free_list_.pop_back();
        in_use_[static_cast<size_t>(id)] = 1;
    }
    return sci::Ok(std::move(ids));
}

void BlockManager::Free(const int32_t* block_ids, int64_t count) {
    if (block_ids == nullptr || count <= 0) return;
    for (int64_t i = 0; i < count; ++i) {
        const int32_t id = block_ids[i];
        const bool valid = id >= 0 && id < num_blocks_ && in_use_[static_cast<size_t>(id)] != 0;
        if (!valid) {
            ++double_free_events_;
            continue;
        }
        in_use_[static_cast<size_t>(id)] = 0;
        free_list_.push_back(id);
    }
}

sci::Status BlockManager::AppendToTable(int64_t seq_id, const int32_t* block_ids, int64_t count) {
    if (seq_id < 0 || seq_id >= table_.max_num_seqs) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "BlockManager::AppendToTable seq_id=" + std::to_string(seq_id) +
                              " out of range [0," + std::to_string(table_.max_num_seqs) + ")");
    }
    if (block_ids == nullptr || count <= 0) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "BlockManager::AppendToTable requires block_ids and count > 0");
    }
    int32_t* row = table_.host.data() + seq_id * table_.max_blocks_per_seq;
    int64_t used = 0;
    while (used < table_.max_blocks_per_seq && row[used] >= 0) ++used;
    if (used + count > table_.max_blocks_per_seq) {
        return MakeStatus(AttnStatusCode::kKVCapacityExceeded,
                          "BlockManager::AppendToTable sequence " + std::to_string(seq_id) +
                              " would need " + std::to_string(used + count) +
                              " blocks > max_blocks_per_seq=" +
                              std::to_string(table_.max_blocks_per_seq));
    }
    for (int64_t i = 0; i < count; ++i) row[used + i] = block_ids[i];
    ++table_.revision;
    return sci::Status::Ok();
}

sci::Status BlockManager::ResetSeq(int64_t seq_id) {
    if (seq_id < 0 || seq_id >= table_.max_num_seqs) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "BlockManager::ResetSeq seq_id=" + std::to_string(seq_id) +
                              " out of range");
    }
    int32_t* row = table_.host.data() + seq_id * table_.max_blocks_per_seq;
    // The first `mapped` entries are freed in row order. AppendToTable fills rows front to back,
    // so the mapped entries are exactly that prefix.
    int64_t mapped = 0;
    for (int64_t i = 0; i < table_.max_blocks_per_seq; ++i) mapped += row[i] >= 0 ? 1 : 0;
    if (mapped > 0) Free(row, mapped);
    for (int64_t i = 0; i < table_.max_blocks_per_seq; ++i) row[i] = -1;
    ++table_.revision;
    return sci::Status::Ok();
}

sci::Status BlockManager::SyncTableToDevice(sci::Stream* stream) {
    if (table_.synced_revision == table_.revision && table_.device.data() != nullptr) {
        return sci::Status::Ok();
    }
    if (table_.device.data() == nullptr) {
        return MakeStatus(AttnStatusCode::kShapeMismatch, "BlockManager: page table not allocated");
    }
    const size_t bytes = table_.host.size() * sizeof(int32_t);
    if (stream != nullptr) {
        table_.device.device().copy_async(table_.device.data(), table_.host.data(), bytes, *stream);
    } else {
        table_.device.copy_from(table_.host.data(), bytes);
    }
    table_.synced_revision = table_.revision;
    return sci::Status::Ok();
}

}  // namespace sca

// Paged KV storage over HBM plus the slot / budget helpers.
// Config checks, the 80%-of-free-memory budget rule with its advice text, the slot formula and
// the error texts follow the reference's src/kv_cache/kv_cache.cpp:16-268; the data movement is
// the kernel library's (sca_hip_kv_append / _reset_blocks / _gather).

#include <algorithm>
#include <string>
#include <vector>

#include "device/device.hpp"
#include "runtime/internal.hpp"
#include "scicompute_attention/kv_cache.hpp"

namespace sca {
namespace {

constexpr double kKvBudgetRatio = 0.8;  // share of the free device memory a cache may claim

bool SupportedBlockSize(int64_t bs) {
    return bs == 1 || bs == 8 || bs == 16 || bs == 32 || bs == 64;
}

sci::Status CheckConfig(const KVCacheConfig& cfg) {
    auto bad = [](AttnStatusCode code, const std::string& what) {
        return MakeStatus(code, "KVCacheConfig invalid: " + what);
    };
    if (cfg.num_layers <= 0) {
        return bad(AttnStatusCode::kShapeMismatch, "num_layers=" + std::to_string(cfg.num_layers));
    }
    if (cfg.num_kv_heads <= 0) {
        return bad(AttnStatusCode::kShapeMismatch,
                   "num_kv_heads=" + std::to_string(cfg.num_kv_heads));
    }
    if (SupportedHeadDimIndex(cfg.head_dim) < 0) {
        return bad(AttnStatusCode::kUnsupportedHeadDim, "head_dim=" + std::to_string(cfg.head_dim));
    }
    if (!SupportedBlockSize(cfg.block_size)) {
        return bad(AttnStatusCode::kShapeMismatch, "block_size=" + std::to_string(cfg.block_size) +
                                                       " (supported: 1, 8, 16, 32, 64)");
    }
    if (cfg.num_blocks <= 0) {
        return bad(AttnStatusCode::kShapeMismatch, "num_blocks=" + std::to_string(cfg.num_blocks));
    }
    if (cfg.max_num_seqs <= 0) {
        return bad(AttnStatusCode::kShapeMismatch,
                   "max_num_seqs=" + std::to_string(cfg.max_num_seqs));
    }
    if (!IsSupportedComputeDtype(cfg.dtype)) {
        return bad(AttnStatusCode::kUnsupportedDtype,
                   std::string("dtype=") + sci::kDTypeName(cfg.dtype));
    }
    if (cfg.layout != KvLayout::kBlockMajor) {
        return bad(AttnStatusCode::kUnsupportedLayout,
                   std::string("layout=") + KvLayoutName(cfg.layout) +
                       " (v1 implements block-major only)");
    }
    return sci::Status::Ok();
}

sca_kv_shape KernelShape(const KVCacheConfig& cfg) {
    sca_kv_shape s{};
    s.num_blocks = cfg.num_blocks;
    s.block_size = cfg.block_size;
    s.num_kv_heads = cfg.num_kv_heads;
    s.head_dim = cfg.head_dim;
    return s;
}

std::string Mib(size_t bytes) { return std::to_string(bytes / (1024 * 1024)); }

}  // namespace

sci::Result<size_t> KvCacheBytes(const KVCacheConfig& cfg) {
    const sci::Status valid = CheckConfig(cfg);
    if (!valid.ok()) return sci::MakeUnexpected<size_t>(valid);
    const int64_t per_layer = cfg.num_blocks * cfg.block_size * cfg.num_kv_heads * cfg.head_dim;
    const int64_t total = 2 * cfg.num_layers * per_layer * DtypeSize(cfg.dtype);
    if (total <= 0) {
        return sci::MakeUnexpected<size_t>(
            MakeStatus(AttnStatusCode::kShapeMismatch, "KVCacheConfig overflow"));
    }
    return sci::Ok(static_cast<size_t>(total));
}

int64_t MaxBlocksForBudget(const KVCacheConfig& cfg, size_t budget_bytes) {
    const int64_t per_block = 2 * cfg.num_layers * cfg.block_size * cfg.num_kv_heads *
                              cfg.head_dim * DtypeSize(cfg.dtype);
    if (per_block <= 0) return 0;
    return static_cast<int64_t>(budget_bytes / static_cast<size_t>(per_block));
}

sci::Result<std::vector<int32_t>> ComputeSlotMapping(const int32_t* block_table_row,
                                                     int64_t seq_start, int64_t num_tokens,
                                                     int64_t block_size, int64_t max_blocks) {
    using Slots = std::vector<int32_t>;
    if (block_table_row == nullptr) {
        return sci::MakeUnexpected<Slots>(
            MakeStatus(AttnStatusCode::kShapeMismatch, "ComputeSlotMapping: null block table row"));
    }
    if (block_size <= 0 || num_tokens <= 0) {
        return sci::MakeUnexpected<Slots>(MakeStatus(
            AttnStatusCode::kShapeMismatch, "ComputeSlotMapping: block_size/num_tokens <= 0"));
    }
    Slots slots(static_cast<size_t>(num_tokens), -1);
    for (int64_t t = 0; t < num_tokens; ++t) {
        const int64_t pos = seq_start + t;
        const int64_t logical = pos / block_size;
        if (logical >= max_blocks) {
            return sci::MakeUnexpected<Slots>(MakeStatus(
                AttnStatusCode::kKVCapacityExceeded,
                "ComputeSlotMapping: logical block " + std::to_string(logical) +
                    " >= max_blocks=" + std::to_string(max_blocks)));
        }
        const int32_t page = block_table_row[logical];
        if (page < 0) {
            return sci::MakeUnexpected<Slots>(MakeStatus(
                AttnStatusCode::kShapeMismatch,
                "ComputeSlotMapping: block table slot " + std::to_string(logical) +
                    " is empty (-1) for position " + std::to_string(pos)));
        }
        slots[static_cast<size_t>(t)] = static_cast<int32_t>(page * block_size + pos % block_size);
    }
    return sci::Ok(std::move(slots));
}

sci::Result<KVCache> KVCache::Create(const KVCacheConfig& cfg, sci::Device& device) {
    const sci::Result<size_t> bytes = KvCacheBytes(cfg);
    if (!bytes.ok()) return sci::MakeUnexpected<KVCache>(bytes.error());

    if (device.type() == sci::DeviceType::kGPU) {
        unsigned long long free_bytes = 0, total_bytes = 0;
        if (sca_hip_mem_get_info(&free_bytes, &total_bytes) == 0) {
            const double budget = static_cast<double>(free_bytes) * kKvBudgetRatio;
            if (static_cast<double>(*bytes) > budget) {
                const int64_t suggested =
                    MaxBlocksForBudget(cfg, static_cast<size_t>(budget / (2 * cfg.num_layers)));
                return sci::MakeUnexpected<KVCache>(MakeStatus(
                    AttnStatusCode::kKVCapacityExceeded,
                    "KV cache needs " + Mib(*bytes) + " MiB but only " +
                        Mib(static_cast<size_t>(free_bytes)) + " MiB is free (budget " +
                        std::to_string(budget / (1024 * 1024)) + " MiB); suggest num_blocks <= " +
                        std::to_string(std::max<int64_t>(1, suggested))));
            }
        }
    }

    KVCache cache;
    cache.cfg_ = cfg;
    cache.layer_elements_ = cfg.num_blocks * cfg.block_size * cfg.num_kv_heads * cfg.head_dim;
    const sci::TensorShape layer_shape({cfg.num_blocks, cfg.block_size, cfg.num_kv_heads,
                                        cfg.head_dim});
    cache.k_layers_.reserve(static_cast<size_t>(cfg.num_layers));
    cache.v_layers_.reserve(static_cast<size_t>(cfg.num_layers));
    const size_t layer_bytes = static_cast<size_t>(cache.layer_elements_) *
                               static_cast<size_t>(DtypeSize(cfg.dtype));
    for (int64_t layer = 0; layer < cfg.num_layers; ++layer) {
        cache.k_layers_.emplace_back(layer_shape, cfg.dtype, device);
        cache.v_layers_.emplace_back(layer_shape, cfg.dtype, device);
        if (cache.k_layers_.back().data() == nullptr || cache.v_layers_.back().data() == nullptr) {
            return sci::MakeUnexpected<KVCache>(MakeStatus(
                AttnStatusCode::kKVCapacityExceeded,
                "KV cache allocation failed at layer " + std::to_string(layer) + " (" +
                    Mib(*bytes) + " MiB requested)"));
        }
        // Pages start zeroed, as after a Reset().
        device.memset(cache.k_layers_.back().data(), 0, layer_bytes);
        device.memset(cache.v_layers_.back().data(), 0, layer_bytes);
    }
    cache.stats_.num_blocks = cfg.num_blocks;
    cache.stats_.free_blocks = cfg.num_blocks;
    cache.stats_.bytes = *bytes;
    cache.stats_.peak_bytes = *bytes;
    return sci::Ok(std::move(cache));
}

sci::Status KVCache::Append(int64_t layer, const sci::Tensor& k_new, const sci::Tensor& v_new,
                            const int32_t* slot_mapping, int64_t num_tokens, sci::Stream* stream) {
    if (layer < 0 || layer >= cfg_.num_layers) {
        return MakeStatus(AttnStatusCode::kShapeMismatch,
                          "KVCache::Append layer=" + std::to_string(layer) + " out of range [0," +
                              std::to_string(cfg_.num_layers) + ")");
    }
    if (k_new.dtype() != cfg_.dtype || v_new.dtype() != cfg_.dtype) {
        return MakeStatus(AttnStatusCode::kUnsupportedDtype,
                          std::string("KVCache::Append dtype mismatch: cache=") +
                              sci::kDTypeName(cfg_.dtype) + ", k=" + sci::kDTypeName(k_new.dtype()));
    }
    for (const sci::Tensor* t : {&k_new, &v_new}) {
        if (t->ndims() != 3 || t->dim(0) != num_tokens || t->dim(1) != cfg_.num_kv_heads ||
            t->dim(2) != cfg_.head_dim) {
            return MakeStatus(AttnStatusCode::kShapeMismatch,
                              "KVCache::Append expects k_new [num_tokens, num_kv_heads, head_dim]=" +
                                  std::to_string(num_tokens) + "x" +
                                  std::to_string(cfg_.num_kv_heads) + "x" +
                                  std::to_string(cfg_.head_dim));
        }
    }
    if (slot_mapping == nullptr) {
        return MakeStatus(AttnStatusCode::kShapeMismatch, "KVCache::Append null slot_mapping");
    }
    const sca_kv_shape shape = KernelShape(cfg_);
    const size_t l = static_cast<size_t>(layer);
    const sci::Status status = runtime::StatusFromHip(
        sca_hip_kv_append(k_layers_[l].data(), v_layers_[l].data(), k_new.data(), v_new.data(),
                          slot_mapping, num_tokens, &shape, DtypeSize(cfg_.dtype),
                          runtime::StreamHandle(stream)),
        "KVCache::Append");
    if (!status.ok()) return status;
    ++stats_.num_appends;
    return sci::Status::Ok();
}

sci::Result<sci::Tensor> KVCache::GatherK(int64_t layer, const int32_t* block_ids,
                                           int64_t num_blocks, sci::Stream* stream) const {
    return GatherInternal(layer, block_ids, num_blocks, true, stream);
}

sci::Result<sci::Tensor> KVCache::GatherV(int64_t layer, const int32_t* block_ids,
                                           int64_t num_blocks, sci::Stream* stream) const {
    return GatherInternal(layer, block_ids, num_blocks, false, stream);
}

sci::Result<sci::Tensor> KVCache::GatherInternal(int64_t layer, const int32_t* block_ids,
                                                 int64_t num_blocks, bool is_key,
                                                 sci::Stream* stream) const {
    if (layer < 0 || layer >= cfg_.num_layers) {
        return sci::MakeUnexpected<sci::Tensor>(
            MakeStatus(AttnStatusCode::kShapeMismatch,
                       "KVCache::Gather layer=" + std::to_string(layer) + " out of range"));
    }
    if (block_ids == nullptr || num_blocks <= 0) {
        return sci::MakeUnexpected<sci::Tensor>(MakeStatus(
            AttnStatusCode::kShapeMismatch, "KVCache::Gather requires block_ids and num_blocks>0"));
    }
    const sci::Tensor& src = is_key ? k_layers_[static_cast<size_t>(layer)]
                                    : v_layers_[static_cast<size_t>(layer)];
    sci::Tensor out(sci::TensorShape({num_blocks, cfg_.block_size, cfg_.num_kv_heads,
                                      cfg_.head_dim}),
                    cfg_.dtype, src.device());
    if (out.data() == nullptr) {
        return sci::MakeUnexpected<sci::Tensor>(
            MakeStatus(AttnStatusCode::kWorkspaceExceeded, "KVCache::Gather allocation failed"));
    }
    const sca_kv_shape shape = KernelShape(cfg_);
    const sci::Status status = runtime::StatusFromHip(
        sca_hip_kv_gather(src.data(), block_ids, num_blocks, out.data(), &shape,
                          DtypeSize(cfg_.dtype), runtime::StreamHandle(stream)),
        "KVCache::Gather");
    if (!status.ok()) return sci::MakeUnexpected<sci::Tensor>(status);
    return sci::Ok(std::move(out));
}

sci::Status KVCache::Reset(const int32_t* block_ids, int64_t num_blocks, sci::Stream* stream) {
    if (block_ids == nullptr) {
        return MakeStatus(AttnStatusCode::kShapeMismatch, "KVCache::Reset null block_ids");
    }
    if (num_blocks <= 0) return sci::Status::Ok();
    const sca_kv_shape shape = KernelShape(cfg_);
    for (int64_t layer = 0; layer < cfg_.num_layers; ++layer) {
        const size_t l = static_cast<size_t>(layer);
        const sci::Status status = runtime::StatusFromHip(
            sca_hip_kv_reset_blocks(k_layers_[l].data(), v_layers_[l].data(), block_ids,
                                    num_blocks, &shape, DtypeSize(cfg_.dtype),
                                    runtime::StreamHandle(stream)),
            "KVCache::Reset");
        if (!status.ok()) return status;
    }
    ++stats_.num_resets;
    return sci::Status::Ok();
}

const sci::Tensor& KVCache::K(int64_t layer) const {
    static const sci::Tensor kNone;
    return layer >= 0 && layer < cfg_.num_layers ? k_layers_[static_cast<size_t>(layer)] : kNone;
}

const sci::Tensor& KVCache::V(int64_t layer) const {
    static const sci::Tensor kNone;
    return layer >= 0 && layer < cfg_.num_layers ? v_layers_[static_cast<size_t>(layer)] : kNone;
}

KVCacheStats KVCache::Stats() const { return stats_; }

size_t KVCache::MemoryBytes() const noexcept { return stats_.bytes; }

}  // namespace sca

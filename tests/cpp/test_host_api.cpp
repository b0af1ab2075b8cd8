// C++ tests of the public sca:: API, written against include/ exactly as a user of the
// reference's C++ API would (the cases follow the reference's tests/unit/*.cpp and tests/kv/*.cpp).
// Built by scicompute-attention_amd/build.py into lib/test_host_api and run by
// tests/test_cpp_api.py:  test_host_api cpu   (no GPU needed)
//                         test_host_api gpu   (needs the MI355X)
// Prints one line per case and exits non-zero when any check failed.

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "device/device.hpp"
#include "scicompute_attention/attention.hpp"

namespace {

int g_failures = 0;
int g_checks = 0;

#define CHECK(cond)                                                                      \
    do {                                                                                 \
        ++g_checks;                                                                      \
        if (!(cond)) {                                                                   \
            ++g_failures;                                                                \
            std::printf("    CHECK failed %s:%d: %s\n", __FILE__, __LINE__, #cond);       \
        }                                                                                \
    } while (0)

bool Has(const std::string& text, const char* needle) {
    return text.find(needle) != std::string::npos;
}

sca::AttentionShape Shape(int64_t sq, int64_t skv, int64_t d = 128, int64_t b = 1,
                          int64_t hq = 8, int64_t hkv = 8) {
    sca::AttentionShape s;
    s.batch = b;
    s.seq_q = sq;
    s.seq_kv = skv;
    s.num_heads = hq;
    s.num_kv_heads = hkv;
    s.head_dim = d;
    return s;
}

// ---- host-side data helpers -------------------------------------------------------------------

uint32_t g_state = 1;
float Uniform() {
    g_state ^= g_state << 13;
    g_state ^= g_state >> 17;
    g_state ^= g_state << 5;
    return -1.0f + 2.0f * static_cast<float>(g_state) / 4294967295.0f;
}

// IEEE binary16 round-to-nearest-even of normal values (test inputs stay in [-1, 1]).
uint16_t ToHalf(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((x >> 23) & 0xff) - 127 + 15;
    if (e <= 0) return static_cast<uint16_t>(sign);
    uint32_t m = x & 0x7fffffu;
    uint32_t h = sign | (static_cast<uint32_t>(e) << 10) | (m >> 13);
    const uint32_t rest = m & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
    return static_cast<uint16_t>(h);
}
float FromHalf(uint16_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1f;
    const uint32_t m = h & 0x3ff;
    uint32_t x = sign;
    if (e != 0) x |= ((e - 15 + 127) << 23) | (m << 13);
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

struct HostHalf {
    std::vector<uint16_t> bits;
    std::vector<double> values;
};

HostHalf RandomHalf(size_t n) {
    HostHalf h;
    h.bits.resize(n);
    h.values.resize(n);
    for (size_t i = 0; i < n; ++i) {
        h.bits[i] = ToHalf(Uniform());
        h.values[i] = FromHalf(h.bits[i]);
    }
    return h;
}

sci::Tensor Upload(const HostHalf& h, std::initializer_list<sci::index_t> dims) {
    sci::Tensor t(sci::TensorShape(dims), sci::DType::kFloat16, sci::GpuDevice(0));
    t.copy_from(h.bits.data(), h.bits.size() * 2);
    return t;
}

std::vector<double> Download(const sci::Tensor& t) {
    std::vector<uint16_t> bits(static_cast<size_t>(t.num_elements()));
    sci::GpuDevice(0).synchronize();
    t.copy_to_host(bits.data(), bits.size() * 2);
    std::vector<double> out(bits.size());
    for (size_t i = 0; i < bits.size(); ++i) out[i] = FromHalf(bits[i]);
    return out;
}

// Double-precision attention over BHSD host values (bottom-right causal, GQA by h / group).
std::vector<double> Reference(const std::vector<double>& q, const std::vector<double>& k,
                              const std::vector<double>& v, const sca::AttentionShape& s,
                              bool causal) {
    const int64_t D = s.head_dim, g = s.num_heads / s.num_kv_heads;
    const double scale = 1.0 / std::sqrt(static_cast<double>(D));
    std::vector<double> out(static_cast<size_t>(s.batch * s.num_heads * s.seq_q * D), 0.0);
    std::vector<double> p(static_cast<size_t>(s.seq_kv));
    for (int64_t b = 0; b < s.batch; ++b)
        for (int64_t h = 0; h < s.num_heads; ++h)
            for (int64_t i = 0; i < s.seq_q; ++i) {
                const double* qi = &q[static_cast<size_t>(((b * s.num_heads + h) * s.seq_q + i) * D)];
                const int64_t hk = h / g;
                double m = -INFINITY;
                for (int64_t j = 0; j < s.seq_kv; ++j) {
                    if (causal && j > i + s.seq_kv - s.seq_q) {
                        p[static_cast<size_t>(j)] = -INFINITY;
                        continue;
                    }
                    const double* kj =
                        &k[static_cast<size_t>(((b * s.num_kv_heads + hk) * s.seq_kv + j) * D)];
                    double dot = 0;
                    for (int64_t d = 0; d < D; ++d) dot += qi[d] * kj[d];
                    p[static_cast<size_t>(j)] = dot * scale;
                    m = std::max(m, dot * scale);
                }
                double l = 0;
                for (auto& x : p) {
                    x = std::isinf(x) ? 0.0 : std::exp(x - m);
                    l += x;
                }
                double* o = &out[static_cast<size_t>(((b * s.num_heads + h) * s.seq_q + i) * D)];
                for (int64_t j = 0; j < s.seq_kv; ++j) {
                    const double* vj =
                        &v[static_cast<size_t>(((b * s.num_kv_heads + hk) * s.seq_kv + j) * D)];
                    for (int64_t d = 0; d < D; ++d) o[d] += p[static_cast<size_t>(j)] / l * vj[d];
                }
            }
    return out;
}

double RelErr(const std::vector<double>& got, const std::vector<double>& ref) {
    double err = 0, scale = 0;
    for (size_t i = 0; i < ref.size(); ++i) {
        err = std::max(err, std::fabs(got[i] - ref[i]));
        scale = std::max(scale, std::fabs(ref[i]));
    }
    return scale > 0 ? err / scale : err;
}

// ---- CPU cases ----------------------------------------------------------------------------------

void DispatchRules() {
    const sca::AttentionDispatcher dispatcher;
    sca::DispatchDecision d = dispatcher.Select(sca::AttentionConfig{}, Shape(1, 2048));
    CHECK(d.backend == sca::BackendKind::kDecode);
    CHECK(Has(d.reason, "auto") && Has(d.reason, "decode") && Has(d.reason, "table=r0"));
    d = dispatcher.Select(sca::AttentionConfig{}, Shape(16, 4096));
    CHECK(d.backend == sca::BackendKind::kFlash && Has(d.reason, "grouped small-q"));
    d = dispatcher.Select(sca::AttentionConfig{}, Shape(1024, 1024));
    CHECK(d.backend == sca::BackendKind::kFlash && Has(d.reason, "online softmax"));
    // Short sequences: the reference's rule, served by flash on this hardware.
    d = dispatcher.Select(sca::AttentionConfig{}, Shape(64, 64));
    CHECK(d.backend == sca::BackendKind::kFlash && Has(d.reason, "short sequence"));
    sca::AttentionConfig naive;
    naive.backend = sca::BackendKind::kNaive;
    d = dispatcher.Select(naive, Shape(1024, 1024));
    CHECK(d.backend == sca::BackendKind::kNaive && Has(d.reason, "explicit"));
    CHECK(Has(d.reason, "unsupported(naive)"));
    d = dispatcher.Select(sca::AttentionConfig{}, Shape(1024, 64, 48));
    CHECK(d.backend == sca::BackendKind::kAuto && Has(d.reason, "invalid") &&
          Has(d.reason, "head_dim=48"));
    const std::string text = dispatcher.Explain(sca::AttentionConfig{}, Shape(1024, 1024));
    CHECK(Has(text, "backend=") && Has(text, "tile={bm=") && Has(text, "workspace=") &&
          Has(text, "reason="));
    // MI355X tiles: 128 query rows per workgroup, 4 waves (the wide kernel up to D=128).
    CHECK(dispatcher.Select(sca::AttentionConfig{}, Shape(1024, 1024, 128)).tile.block_m == 128);
    CHECK(dispatcher.Select(sca::AttentionConfig{}, Shape(1024, 1024, 128)).tile.warps == 4);
    CHECK(dispatcher.Select(sca::AttentionConfig{}, Shape(1024, 1024, 256)).tile.warps == 4);
    CHECK(sca::AttentionDispatcher::ReloadDispatchTable(nullptr).ok());
    CHECK(!sca::AttentionDispatcher::ReloadDispatchTable("table.json").ok());
    sca::BackendKind kind = sca::BackendKind::kAuto;
    CHECK(sca::ParseBackendName("paged", &kind) && kind == sca::BackendKind::kPaged);
    CHECK(!sca::ParseBackendName("fa3", &kind));
    CHECK(sca::GetBackend(sca::BackendKind::kAuto) != nullptr);
}

void ConfigValidation() {
    sca::AttentionConfig cfg;
    for (int64_t d : sca::kSupportedHeadDims) CHECK(sca::Validate(cfg, Shape(128, 128, d)).ok());
    std::string detail;
    sci::Status st = sca::Validate(cfg, Shape(128, 128, 48), &detail);
    CHECK(!st.ok() && sca::ExtractCode(st) == sca::AttnStatusCode::kUnsupportedHeadDim);
    CHECK(Has(detail, "head_dim=48") && Has(detail, "128"));
    cfg.causal = true;
    st = sca::Validate(cfg, Shape(256, 128), &detail);
    CHECK(!st.ok() && Has(detail, "causal=true") && Has(detail, "seq_kv(128)") &&
          Has(detail, "seq_q(256)"));
    cfg = sca::AttentionConfig{};
    st = sca::Validate(cfg, Shape(128, 128, 128, 1, 32, 6));
    CHECK(sca::ExtractCode(st) == sca::AttnStatusCode::kShapeMismatch);
    CHECK(Has(st.message(), "num_heads=32") && Has(st.message(), "num_kv_heads=6"));
    cfg.sliding_window = 512;
    st = sca::Validate(cfg, Shape(128, 128));
    CHECK(sca::ExtractCode(st) == sca::AttnStatusCode::kUnsupportedFeature &&
          Has(st.message(), "sliding_window=512"));
    cfg = sca::AttentionConfig{};
    cfg.softcap = 50.0f;
    cfg.backend = sca::BackendKind::kNaive;
    CHECK(!sca::Validate(cfg, Shape(128, 128)).ok());
    cfg.backend = sca::BackendKind::kFlash;
    CHECK(sca::Validate(cfg, Shape(128, 128)).ok());
    cfg = sca::AttentionConfig{};
    CHECK(std::fabs(sca::EffectiveScale(cfg, Shape(1, 1, 128)) - 1.0f / std::sqrt(128.0f)) < 1e-7f);
    cfg.scale = 0.5f;
    CHECK(sca::EffectiveScale(cfg, Shape(1, 1, 128)) == 0.5f);
    cfg.scale = 0.0f;
    CHECK(std::fabs(sca::EffectiveScale(cfg, Shape(1, 1, 64)) - 0.125f) < 1e-7f);
    const int32_t good[] = {0, 3, 10, 11};
    int64_t max_seq = 0;
    CHECK(sca::ValidateVarlenHost(good, 3, &max_seq).ok() && max_seq == 7);
    const int32_t bad_start[] = {1, 3, 4};
    const int32_t not_monotonic[] = {0, 3, 3};
    CHECK(!sca::ValidateVarlenHost(bad_start, 2).ok());
    CHECK(sca::ExtractCode(sca::ValidateVarlenHost(not_monotonic, 2)) ==
          sca::AttnStatusCode::kShapeMismatch);
    CHECK(!sca::ValidateVarlenHost(nullptr, 2).ok());
}

void StatusAndNames() {
    for (int c = 2001; c <= 2010; ++c) {
        const char* text = sca::ToString(static_cast<sca::AttnStatusCode>(c));
        CHECK(text != nullptr && std::strlen(text) > 0);
    }
    CHECK(std::string(sca::ToString(sca::AttnStatusCode::kKVCapacityExceeded)) ==
          "KVCapacityExceeded");
    const sci::Status st =
        sca::MakeStatus(sca::AttnStatusCode::kKVCapacityExceeded, "requested 40 blocks");
    CHECK(!st.ok() && st.code() == sci::StatusCode::kResourceExhausted);
    CHECK(sca::ExtractCode(st) == sca::AttnStatusCode::kKVCapacityExceeded);
    CHECK(Has(st.message(), "[SCA-2007]") && Has(st.message(), "requested 40 blocks"));
    CHECK(sca::ToSciCode(sca::AttnStatusCode::kUnsupportedHeadDim) ==
          sci::StatusCode::kInvalidArgument);
    CHECK(sca::ToSciCode(sca::AttnStatusCode::kWorkspaceExceeded) ==
          sci::StatusCode::kResourceExhausted);
    CHECK(sca::ToSciCode(sca::AttnStatusCode::kUnsupportedFeature) ==
          sci::StatusCode::kNotImplemented);
    CHECK(sca::ExtractCode(sci::Status::Ok()) == sca::AttnStatusCode::kOk);
    CHECK(std::string(sca::BackendName(sca::BackendKind::kFlash)) == "flash");
    CHECK(std::string(sca::LayoutName(sca::AttnLayout::kBSHD)) == "bshd");
    CHECK(std::string(sca::VersionString()) == SCI_ATTENTION_VERSION_STRING);
    CHECK(sca::DtypeSize(sci::DType::kBFloat16) == 2);
    CHECK(sca::IsSupportedComputeDtype(sci::DType::kFloat32));
    CHECK(!sca::IsSupportedComputeDtype(sci::DType::kInt8));
    CHECK(sca::SupportedHeadDimIndex(128) == 3 && sca::SupportedHeadDimIndex(48) == -1);
    CHECK(sca::TileConfig::SmemBytesFlash(128, 2, 64, 64, 4, 2) == 87040);
}

void BlockManagerOn(sci::Device& device) {
    auto made = sca::BlockManager::Create(16, 2, 8, device);
    CHECK(made.ok());
    sca::BlockManager bm = std::move(*made);
    CHECK(bm.NumFreeBlocks() == 16);
    auto first = bm.Allocate(5);
    CHECK(first.ok() && first->size() == 5 && bm.NumFreeBlocks() == 11);
    std::vector<int32_t> sorted = *first;
    std::sort(sorted.begin(), sorted.end());
    CHECK(std::adjacent_find(sorted.begin(), sorted.end()) == sorted.end());
    CHECK(sorted.front() >= 0 && sorted.back() < 16);
    bm.Free(first->data(), 5);
    CHECK(bm.NumFreeBlocks() == 16);

    auto small = sca::BlockManager::Create(8, 2, 8, device);
    sca::BlockManager b8 = std::move(*small);
    CHECK(b8.Allocate(8).ok());
    auto overflow = b8.Allocate(1);
    CHECK(!overflow.ok() && sca::ExtractCode(overflow.error()) ==
                                sca::AttnStatusCode::kKVCapacityExceeded);
    CHECK(b8.NumFreeBlocks() == 0 && b8.AllocationFailures() == 1);
    CHECK(Has(overflow.error().message(), "only 0 of 8"));

    auto tiny = sca::BlockManager::Create(4, 1, 4, device);
    sca::BlockManager b4 = std::move(*tiny);
    auto two = b4.Allocate(2);
    b4.Free(two->data(), 2);
    b4.Free(two->data(), 2);
    CHECK(b4.NumFreeBlocks() == 4 && b4.DoubleFreeEvents() == 2);
    CHECK(!b4.Allocate(0).ok());
    CHECK(!b4.AppendToTable(0, nullptr, 1).ok());
    CHECK(!b4.AppendToTable(7, nullptr, 1).ok());

    auto iso = sca::BlockManager::Create(16, 3, 4, device);
    sca::BlockManager m = std::move(*iso);
    auto a = m.Allocate(2);
    auto b = m.Allocate(2);
    CHECK(m.AppendToTable(0, a->data(), 2).ok() && m.AppendToTable(1, b->data(), 2).ok());
    const sca::BlockTable& table = m.Table();
    CHECK(table.host[0] == (*a)[0] && table.host[1] == (*a)[1] && table.host[2] == -1);
    CHECK(table.host[4] == (*b)[0]);
    const uint64_t before = table.revision;
    CHECK(m.ResetSeq(0).ok() && table.host[0] == -1 && table.revision > before);
    CHECK(m.NumFreeBlocks() == 14);
    CHECK(m.SyncTableToDevice(nullptr).ok());
    device.synchronize();
    CHECK(m.SyncTableToDevice(nullptr).ok());
    std::vector<int32_t> mirror(table.host.size());
    table.device.copy_to_host(mirror.data(), mirror.size() * 4);
    CHECK(mirror == table.host);
}

void BlockManagerHost() { BlockManagerOn(sci::HostDevice()); }

void WorkspaceAndKvHelpers() {
    auto ws = sca::Workspace::Create(4096, sci::HostDevice());
    CHECK(ws.ok());
    sca::Workspace w = *ws;
    CHECK(w.Slice(0, 256).ok() && w.Slice(256, 512).ok() && w.Slice(0, 256).ok());
    CHECK(!w.Slice(128, 64).ok() && !w.Slice(0, 8192).ok());
    CHECK(w.AllocatedSlices() == 2 && w.PeakBytes() == 768);
    CHECK(w.Reset().ok() && w.AllocatedSlices() == 0);
    sca::KVCacheConfig cfg;
    cfg.num_layers = 32;
    cfg.num_kv_heads = 8;
    cfg.head_dim = 128;
    cfg.block_size = 16;
    cfg.num_blocks = 1536;
    cfg.max_num_seqs = 4;
    auto bytes = sca::KvCacheBytes(cfg);
    CHECK(bytes.ok() && *bytes == 3221225472ull && sca::MaxBlocksForBudget(cfg, *bytes / 2) == 768);
    cfg.block_size = 7;
    CHECK(!sca::KvCacheBytes(cfg).ok());
    const int32_t row[] = {3, 1, 0, -1};
    auto slots = sca::ComputeSlotMapping(row, 17, 5, 16, 4);
    CHECK(slots.ok() && (*slots)[0] == 17 && (*slots)[4] == 21);
    auto empty = sca::ComputeSlotMapping(row, 48, 1, 16, 4);
    CHECK(!empty.ok() && Has(empty.error().message(), "empty"));
}

void CapabilityWithoutGpu() {
    if (sca::DeviceCapability::GpuAvailable()) return;
    const sca::DeviceCapability& cap = sca::DeviceCapability::ForDevice(0);
    CHECK(cap.sm_count == 0 && !cap.has_wgmma && !cap.has_mfma_f16_k16);
    // Attention on host tensors is refused with a reason, never computed on the CPU.
    sci::Tensor q(sci::TensorShape({1, 1, 4, 64}), sci::DType::kFloat16, sci::HostDevice());
    auto r = sca::attention(q, q, q);
    CHECK(!r.ok() && Has(r.error().message(), "GPU"));
}

// ---- GPU cases ----------------------------------------------------------------------------------

void Capability() {
    const sca::DeviceCapability& cap = sca::DeviceCapability::ForDevice(0);
    std::printf("    %s (%s): %d CUs, wave %d, LDS/CU %zu, L2 %zu, HBM %zu\n",
                cap.device_name.c_str(), cap.arch_name.c_str(), cap.sm_count, cap.wave_size,
                cap.smem_per_sm, cap.l2_bytes, cap.total_mem_bytes);
    CHECK(!cap.device_name.empty() && cap.sm_count >= 1 && cap.wave_size == 64);
    CHECK(cap.smem_per_sm > 0 && cap.regs_per_sm > 0 && cap.total_mem_bytes > 0);
    CHECK(cap.has_mfma_f16_k16 && !cap.has_wgmma && !cap.has_cp_async);
}

void BlockManagerGpu() { BlockManagerOn(sci::GpuDevice(0)); }

void AttentionEndToEnd() {
    for (bool causal : {false, true}) {
        const sca::AttentionShape s = Shape(77, 77, 128, 2, 8, 2);
        HostHalf q = RandomHalf(static_cast<size_t>(s.QueryElements()));
        HostHalf k = RandomHalf(static_cast<size_t>(s.KvElements()));
        HostHalf v = RandomHalf(static_cast<size_t>(s.KvElements()));
        sci::Tensor tq = Upload(q, {2, 8, 77, 128});
        sci::Tensor tk = Upload(k, {2, 2, 77, 128});
        sci::Tensor tv = Upload(v, {2, 2, 77, 128});
        sca::AttentionConfig cfg;
        cfg.causal = causal;
        cfg.return_lse = true;
        auto r = sca::attention(tq, tk, tv, cfg);
        CHECK(r.ok());
        if (!r.ok()) {
            std::printf("    %s\n", r.error().message().c_str());
            continue;
        }
        CHECK(r->stats.used_backend == sca::BackendKind::kFlash);
        CHECK(r->stats.workspace_bytes == 0 && r->stats.materialized_score_bytes == 0);
        CHECK(r->lse.num_elements() == 2 * 8 * 77);
        const double rel = RelErr(Download(r->out), Reference(q.values, k.values, v.values, s, causal));
        std::printf("    flash causal=%d rel=%.2e\n", causal ? 1 : 0, rel);
        CHECK(rel <= 2e-3);
    }
    // Decode through the dispatcher (S_q = 1, S_kv >= 256).
    const sca::AttentionShape s = Shape(1, 700, 128, 3, 16, 4);
    HostHalf q = RandomHalf(static_cast<size_t>(s.QueryElements()));
    HostHalf k = RandomHalf(static_cast<size_t>(s.KvElements()));
    HostHalf v = RandomHalf(static_cast<size_t>(s.KvElements()));
    sci::Tensor tq = Upload(q, {3, 16, 1, 128});
    sci::Tensor tk = Upload(k, {3, 4, 700, 128});
    sci::Tensor tv = Upload(v, {3, 4, 700, 128});
    auto r = sca::attention(tq, tk, tv);
    CHECK(r.ok() && r->stats.used_backend == sca::BackendKind::kDecode);
    if (r.ok()) {
        CHECK(r->stats.num_splits >= 1 && (r->stats.num_splits == 1 || r->stats.workspace_bytes > 0));
        const double rel = RelErr(Download(r->out), Reference(q.values, k.values, v.values, s, false));
        std::printf("    decode splits=%lld rel=%.2e\n", static_cast<long long>(r->stats.num_splits), rel);
        CHECK(rel <= 2e-3);
    }
    // Explicit backends that are not built here fail loudly.
    sca::AttentionConfig tiled;
    tiled.backend = sca::BackendKind::kTiled;
    auto refused = sca::attention(tq, tk, tv, tiled);
    CHECK(!refused.ok() && Has(refused.error().message(), "not built for MI355X"));
}

sca::KVCacheConfig KvConfig(int64_t bs, int64_t nb, int64_t max_seqs = 4) {
    sca::KVCacheConfig cfg;
    cfg.num_layers = 1;
    cfg.num_kv_heads = 1;
    cfg.head_dim = 32;
    cfg.block_size = bs;
    cfg.num_blocks = nb;
    cfg.max_num_seqs = max_seqs;
    cfg.dtype = sci::DType::kFloat16;
    return cfg;
}

sci::Tensor Tokens(int64_t n, float base) {
    HostHalf h;
    h.bits.resize(static_cast<size_t>(n * 32));
    for (size_t i = 0; i < h.bits.size(); ++i) h.bits[i] = ToHalf(base + 0.001f * static_cast<float>(i));
    sci::Tensor t(sci::TensorShape({n, 1, 32}), sci::DType::kFloat16, sci::GpuDevice(0));
    t.copy_from(h.bits.data(), h.bits.size() * 2);
    return t;
}

void PagedKvCache() {
    {
        auto made = sca::PagedKVCache::Create(KvConfig(8, 8), sci::GpuDevice(0));
        CHECK(made.ok());
        sca::PagedKVCache cache = std::move(*made);
        sci::Tensor a3 = Tokens(3, 1.0f), b3 = Tokens(3, 100.0f), a6 = Tokens(6, 2.0f);
        CHECK(cache.AppendTokens(0, 0, a3, a3, nullptr).ok());
        CHECK(cache.AppendTokens(1, 0, b3, b3, nullptr).ok());
        CHECK(cache.AppendTokens(0, 0, a6, a6, nullptr).ok());
        CHECK(cache.SeqLength(0) == 9 && cache.SeqLength(1) == 3);
        CHECK(cache.LogicalBlockCount(0) == 2 && cache.LogicalBlockCount(1) == 1);
        const sca::KVCacheStats st = cache.Stats();
        CHECK(st.used_blocks == 3 && st.free_blocks == 5 && st.num_appends == 3);
        CHECK(cache.SyncPageTable(nullptr).ok());
        std::vector<int32_t> dev(cache.PageTableHost().size());
        sci::GpuDevice(0).synchronize();
        sci::GpuDevice(0).copy_to_host(dev.data(), cache.PageTableDevicePtr(), dev.size() * 4);
        CHECK(dev == cache.PageTableHost());
        CHECK(dev[0] == 0 && dev[1] == 2 && dev[8] == 1);
    }
    {
        auto made = sca::PagedKVCache::Create(KvConfig(8, 2), sci::GpuDevice(0));
        sca::PagedKVCache cache = std::move(*made);
        sci::Tensor first = Tokens(16, 1.0f), second = Tokens(8, 2.0f);
        CHECK(cache.AppendTokens(0, 0, first, first, nullptr).ok());
        CHECK(cache.Stats().free_blocks == 0);
        const sci::Status overflow = cache.AppendTokens(1, 0, second, second, nullptr);
        CHECK(!overflow.ok() && sca::ExtractCode(overflow) == sca::AttnStatusCode::kKVCapacityExceeded);
        CHECK(cache.SeqLength(1) == 0 && cache.LogicalBlockCount(1) == 0 && cache.SeqLength(0) == 16);
    }
    {
        auto made = sca::PagedKVCache::Create(KvConfig(8, 2), sci::GpuDevice(0));
        sca::PagedKVCache cache = std::move(*made);
        sci::Tensor t = Tokens(8, 3.0f);
        CHECK(cache.AppendTokens(0, 0, t, t, nullptr).ok());
        CHECK(cache.ResetSeq(0, nullptr).ok());
        const sca::KVCacheStats st = cache.Stats();
        CHECK(cache.SeqLength(0) == 0 && st.free_blocks == 2 && st.num_resets == 1);
        // The released page was zeroed.
        std::vector<uint16_t> page(8 * 32, 0xffff);
        sci::GpuDevice(0).synchronize();
        cache.Storage().K(0).copy_to_host(page.data(), page.size() * 2);
        CHECK(std::all_of(page.begin(), page.end(), [](uint16_t x) { return x == 0; }));
        sci::Tensor other = Tokens(8, -5.0f);
        CHECK(cache.AppendTokens(1, 0, other, other, nullptr).ok());
        CHECK(cache.SeqLength(1) == 8 && cache.Stats().free_blocks == 1);
    }
}

struct Case {
    const char* name;
    const char* group;
    std::function<void()> fn;
};

}  // namespace

int main(int argc, char** argv) {
    const std::string group = argc > 1 ? argv[1] : "cpu";
    const std::vector<Case> cases = {
        {"dispatch_rules", "cpu", DispatchRules},
        {"config_validation", "cpu", ConfigValidation},
        {"status_and_names", "cpu", StatusAndNames},
        {"block_manager_host", "cpu", BlockManagerHost},
        {"workspace_and_kv_helpers", "cpu", WorkspaceAndKvHelpers},
        {"capability_without_gpu", "cpu", CapabilityWithoutGpu},
        {"capability", "gpu", Capability},
        {"block_manager_gpu", "gpu", BlockManagerGpu},
        {"attention_end_to_end", "gpu", AttentionEndToEnd},
        {"paged_kv_cache", "gpu", PagedKvCache},
    };
    int ran = 0;
    for (const Case& c : cases) {
        if (group != c.group) continue;
        const int before = g_failures;
        std::printf("[ RUN  ] %s\n", c.name);
        std::fflush(stdout);
        c.fn();
        std::printf("[ %s ] %s\n", g_failures == before ? " OK " : "FAIL", c.name);
        std::fflush(stdout);
        ++ran;
    }
    std::printf("%d cases, %d checks, %d failures\n", ran, g_checks, g_failures);
    return g_failures == 0 && ran > 0 ? 0 : 1;
}

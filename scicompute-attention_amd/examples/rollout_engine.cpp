// Rollout-style serving loop over the public sca:: API at the Qwen3-4B attention shape
// (H_q = 32, H_kv = 8, D = 128, fp16, 16-token pages): the role of the reference's
// examples/rollout_engine_stub.cpp:138-334, arranged for this build.
//
//   prefill  every prompt of the batch in ONE flash_attention_varlen call over packed
//            [tokens, heads, dim] buffers (causal), then one AppendTokens per request;
//   decode   per step: one AppendTokensBatch (a token for every request), SyncPageTable
//            (changed entries only), the lengths uploaded AFTER they advanced (the reference
//            uploads them before the increment, examples/rollout_engine_stub.cpp:253-254 vs
//            280, so its attention misses the token just appended), then one paged_attention.
//
// One attention layer is driven, as in the reference (layer 0, rollout_engine_stub.cpp:226,
// 246): AppendTokens advances a sequence's length on every call, so multi-layer writes are not
// expressible through that interface. Timings are GPU time from HIP events around each API
// call (dispatch and allocation included). Prints a summary; --json PATH writes it as JSON.
//
//   rollout_engine [--requests N] [--max-new T] [--min-prompt P] [--json PATH]

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

#include "device/device.hpp"
#include "sca_hip.h"
#include "scicompute_attention/attention.hpp"

namespace {

constexpr int64_t kHeadsQ = 32;
constexpr int64_t kHeadsKv = 8;
constexpr int64_t kHeadDim = 128;
constexpr int64_t kBlockSize = 16;

struct Args {
    int64_t requests = 16;
    int64_t max_new = 32;
    int64_t min_prompt = 256;
    std::string json;
};

Args Parse(int argc, char** argv) {
    Args a;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string k = argv[i];
        if (k == "--requests") a.requests = std::atoll(argv[i + 1]);
        else if (k == "--max-new") a.max_new = std::atoll(argv[i + 1]);
        else if (k == "--min-prompt") a.min_prompt = std::atoll(argv[i + 1]);
        else if (k == "--json") a.json = argv[i + 1];
    }
    return a;
}

// IEEE binary16 bits of f, round to nearest even (|f| <= 1 here: no overflow; tiny values
// flush to signed zero).
uint16_t HalfBits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = static_cast<int32_t>((x >> 23) & 0xffu) - 112;
    if (e <= 0) return static_cast<uint16_t>(sign);
    const uint32_t mant = x & 0x7fffffu;
    uint32_t h = sign | (static_cast<uint32_t>(e) << 10) | (mant >> 13);
    const uint32_t rest = mant & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) ++h;
    return static_cast<uint16_t>(h);
}

// Seeded fp16 bits in [-scale, scale] (xorshift32), uploaded to a new device tensor.
sci::Tensor RandomHalf(const std::vector<int64_t>& dims, uint32_t seed, float scale) {
    int64_t n = 1;
    for (int64_t d : dims) n *= d;
    std::vector<uint16_t> bits(static_cast<size_t>(n));
    uint32_t s = seed ? seed : 1u;
    for (auto& b : bits) {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        b = HalfBits(scale * (-1.0f + 2.0f * static_cast<float>(s) / 4294967295.0f));
    }
    sci::Device& dev = sci::GpuDevice(0);
    sci::Tensor t(sci::TensorShape(dims), sci::DType::kFloat16, dev);
    if (t.data() != nullptr) dev.copy_to_device(t.data(), bits.data(), bits.size() * 2);
    return t;
}

struct Timer {
    void* a = nullptr;
    void* b = nullptr;
    Timer() {
        sca_hip_event_create(&a);
        sca_hip_event_create(&b);
    }
    ~Timer() {
        sca_hip_event_destroy(a);
        sca_hip_event_destroy(b);
    }
    void Start() { sca_hip_event_record(a, nullptr); }
    double StopMs() {
        sca_hip_event_record(b, nullptr);
        sca_hip_event_synchronize(b);
        float ms = 0.0f;
        sca_hip_event_elapsed_ms(&ms, a, b);
        return ms;
    }
};

double Percentile(std::vector<double> v, double p) {
    if (v.empty()) return 0.0;
    std::sort(v.begin(), v.end());
    const double r = p * static_cast<double>(v.size() - 1);
    const size_t lo = static_cast<size_t>(r);
    const size_t hi = std::min(lo + 1, v.size() - 1);
    return v[lo] + (v[hi] - v[lo]) * (r - static_cast<double>(lo));
}

int Fail(const char* what, const sci::Status& st) {
    std::printf("[rollout] %s failed: %s\n", what, st.ToString().c_str());
    return 4;
}

}  // namespace

int main(int argc, char** argv) {
    const Args args = Parse(argc, argv);
    int devices = 0;
    if (sca_hip_get_device_count(&devices) != 0 || devices < 1) {
        std::printf("[rollout] no GPU visible; nothing to run\n");
        return 2;
    }
    sci::Device& device = sci::GpuDevice(0);
    const int64_t n = args.requests;

    // Uneven prompt lengths, like a real rollout batch.
    std::vector<int32_t> prompt(static_cast<size_t>(n));
    for (int64_t r = 0; r < n; ++r) {
        prompt[static_cast<size_t>(r)] = static_cast<int32_t>(args.min_prompt + (r * 997) % 1792);
    }
    std::vector<int32_t> cu(static_cast<size_t>(n + 1), 0);
    for (int64_t r = 0; r < n; ++r) cu[static_cast<size_t>(r + 1)] = cu[static_cast<size_t>(r)] + prompt[static_cast<size_t>(r)];
    const int64_t total = cu.back();
    const int64_t max_prompt = *std::max_element(prompt.begin(), prompt.end());

    sca::KVCacheConfig kv;
    kv.num_layers = 1;
    kv.num_kv_heads = kHeadsKv;
    kv.head_dim = kHeadDim;
    kv.block_size = kBlockSize;
    kv.max_num_seqs = n;
    kv.dtype = sci::DType::kFloat16;
    kv.num_blocks = (total + n * args.max_new + kBlockSize - 1) / kBlockSize + n;
    const auto kv_bytes = sca::KvCacheBytes(kv);
    if (!kv_bytes.ok()) return Fail("KV budget", kv_bytes.error());
    const sca::DeviceCapability& cap = sca::DeviceCapability::ForDevice(0);
    if (*kv_bytes > cap.free_mem_bytes / 2) {
        std::printf("[rollout] refusing: the KV cache would exceed half of free memory\n");
        return 3;
    }
    auto created = sca::PagedKVCache::Create(kv, device);
    if (!created.ok()) return Fail("PagedKVCache::Create", created.error());
    sca::PagedKVCache cache = std::move(*created);

    // ---- prefill: the whole batch in one packed launch ------------------------------------------
    sci::Tensor q = RandomHalf({total, kHeadsQ, kHeadDim}, 1000, 1.0f);
    sci::Tensor k = RandomHalf({total, kHeadsKv, kHeadDim}, 2000, 1.0f);
    sci::Tensor v = RandomHalf({total, kHeadsKv, kHeadDim}, 3000, 0.5f);
    sca::AttentionConfig pcfg;
    pcfg.backend = sca::BackendKind::kFlash;
    pcfg.causal = true;
    Timer timer;
    // One untimed call first: code-object loading and first-use allocations are not serving time.
    if (!sca::flash_attention_varlen(q, k, v, n, cu.data(), cu.data(), max_prompt, max_prompt,
                                     pcfg).ok()) {
        std::printf("[rollout] warm-up prefill failed\n");
        return 4;
    }
    timer.Start();
    const auto pre = sca::flash_attention_varlen(q, k, v, n, cu.data(), cu.data(), max_prompt,
                                                 max_prompt, pcfg);
    const double prefill_ms = timer.StopMs();
    if (!pre.ok()) return Fail("prefill", pre.error());
    double prefill_flops = 0.0;
    for (int32_t L : prompt) prefill_flops += 4.0 * kHeadsQ * kHeadDim * (0.5 * L * (L + 1.0));

    timer.Start();
    const int64_t kv_token_bytes = kHeadsKv * kHeadDim * 2;
    for (int64_t r = 0; r < n; ++r) {
        const int64_t off = cu[static_cast<size_t>(r)] * kv_token_bytes;
        const int64_t len = prompt[static_cast<size_t>(r)];
        sci::Tensor kr(sci::TensorShape({len, kHeadsKv, kHeadDim}), sci::DType::kFloat16, device,
                       static_cast<char*>(k.data()) + off);
        sci::Tensor vr(sci::TensorShape({len, kHeadsKv, kHeadDim}), sci::DType::kFloat16, device,
                       static_cast<char*>(v.data()) + off);
        const sci::Status st = cache.AppendTokens(r, 0, kr, vr, nullptr);
        if (!st.ok()) return Fail("prompt append", st);
    }
    const double prompt_append_ms = timer.StopMs();

    // ---- decode loop ----------------------------------------------------------------------------
    std::vector<int64_t> ids(static_cast<size_t>(n));
    for (int64_t r = 0; r < n; ++r) ids[static_cast<size_t>(r)] = r;
    std::vector<int32_t> lens(prompt);
    sci::Tensor seq_lens(sci::TensorShape({n}), sci::DType::kInt32, device);
    sci::Tensor q_step = RandomHalf({n, kHeadsQ, 1, kHeadDim}, 5000, 1.0f);
    sci::Tensor k_step = RandomHalf({n, kHeadsKv, kHeadDim}, 6000, 1.0f);
    sci::Tensor v_step = RandomHalf({n, kHeadsKv, kHeadDim}, 7000, 0.5f);
    sca::AttentionConfig dcfg;
    dcfg.backend = sca::BackendKind::kPaged;
    std::vector<double> append_ms, attend_ms;
    {
        // Untimed attend over the prompts (kernel loading, scratch allocation).
        device.copy_to_device(seq_lens.data(), lens.data(), lens.size() * sizeof(int32_t));
        sca::PagedAttentionParams params;
        params.seq_lens = static_cast<const int32_t*>(seq_lens.data());
        params.num_seqs = n;
        params.block_size = kBlockSize;
        const sci::Status st = cache.SyncPageTable(nullptr);
        if (!st.ok() || !sca::paged_attention(q_step, cache, params, dcfg).ok()) {
            std::printf("[rollout] warm-up decode failed\n");
            return 4;
        }
    }
    double attend_bytes = 0.0;
    for (int64_t step = 0; step < args.max_new; ++step) {
        timer.Start();
        sci::Status st = cache.AppendTokensBatch(ids.data(), n, 0, k_step, v_step, nullptr);
        if (!st.ok()) return Fail("decode append", st);
        st = cache.SyncPageTable(nullptr);
        if (!st.ok()) return Fail("page-table sync", st);
        for (auto& L : lens) ++L;  // the new token is attended in this step
        device.copy_to_device(seq_lens.data(), lens.data(), lens.size() * sizeof(int32_t));
        append_ms.push_back(timer.StopMs());

        sca::PagedAttentionParams params;
        params.page_table = cache.PageTableDevicePtr();
        params.seq_lens = static_cast<const int32_t*>(seq_lens.data());
        params.num_seqs = n;
        params.block_size = kBlockSize;
        params.max_blocks_per_seq = cache.MaxBlocksPerSeq();
        params.layer = 0;
        timer.Start();
        const auto out = sca::paged_attention(q_step, cache, params, dcfg);
        attend_ms.push_back(timer.StopMs());
        if (!out.ok()) return Fail("paged attention", out.error());
        for (int32_t L : lens) attend_bytes += 2.0 * L * kv_token_bytes;
    }

    double attend_total = 0.0, append_total = 0.0;
    for (double t : attend_ms) attend_total += t;
    for (double t : append_ms) append_total += t;
    const int64_t generated = n * args.max_new;
    const double step_ms = (attend_total + append_total) / static_cast<double>(args.max_new);
    const auto stats = cache.Stats();
    std::printf("[rollout] requests=%lld prompts=[%d..%d] tokens=%lld max_new=%lld\n",
                static_cast<long long>(n), *std::min_element(prompt.begin(), prompt.end()),
                static_cast<int>(max_prompt), static_cast<long long>(total),
                static_cast<long long>(args.max_new));
    std::printf("[rollout] prefill  %.3f ms (one varlen launch, %.1f TFLOP/s); prompt appends %.3f ms\n",
                prefill_ms, prefill_flops / (prefill_ms * 1e-3) / 1e12, prompt_append_ms);
    std::printf("[rollout] decode   attend P50=%.3f ms P99=%.3f ms (%.0f GB/s); append+sync P50=%.3f ms\n",
                Percentile(attend_ms, 0.5), Percentile(attend_ms, 0.99),
                attend_bytes / (attend_total * 1e-3) / 1e9, Percentile(append_ms, 0.5));
    std::printf("[rollout] tokens/s per layer=%.0f used_blocks=%lld/%lld\n",
                static_cast<double>(n) / (step_ms * 1e-3), static_cast<long long>(stats.used_blocks),
                static_cast<long long>(stats.num_blocks));
    if (!args.json.empty()) {
        std::ofstream f(args.json);
        f << "{\"engine\": \"rollout_engine\", \"requests\": " << n << ", \"max_new_tokens\": "
          << args.max_new << ", \"prompt_tokens\": " << total << ", \"prefill_ms\": " << prefill_ms
          << ", \"prefill_tflops\": " << prefill_flops / (prefill_ms * 1e-3) / 1e12
          << ", \"decode_attend_ms\": {\"p50\": " << Percentile(attend_ms, 0.5) << ", \"p99\": "
          << Percentile(attend_ms, 0.99) << "}, \"decode_append_sync_ms_p50\": "
          << Percentile(append_ms, 0.5) << ", \"decode_attend_gbps\": "
          << attend_bytes / (attend_total * 1e-3) / 1e9 << ", \"generated_tokens\": " << generated
          << ", \"kv_blocks_used\": " << stats.used_blocks << ", \"shape\": {\"Hq\": " << kHeadsQ
          << ", \"Hkv\": " << kHeadsKv << ", \"D\": " << kHeadDim << "}}\n";
    }
    return 0;
}

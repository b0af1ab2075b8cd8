// Rollout-style serving loop over the public sca:: API at the Qwen3-4B attention shape
// (36 layers, H_q = 32, H_kv = 8, D = 128, fp16, 16-token pages): the role of the reference's
// examples/rollout_engine_stub.cpp:138-334, arranged for this build. Every step drives all the
// layers, as a model does:
//
//   prefill  one ReserveTokensBatch for every prompt token of the batch (the packed token order),
//            then per layer: one causal flash_attention_varlen over that layer's packed
//            [tokens, heads, dim] Q/K/V and one WriteReservedLayer of its K/V;
//   decode   per step: one ReserveTokensBatch (a token for every request: pages, slots and
//            lengths advance once), SyncPageTable (changed entries only), the lengths uploaded
//            AFTER they advanced (the reference uploads them before the increment,
//            examples/rollout_engine_stub.cpp:253-254 vs 280, so its attention misses the token
//            just appended), then per layer: WriteReservedLayer + paged_attention(layer).
//
// The reference drives layer 0 only (rollout_engine_stub.cpp:226, 246): its AppendTokens advances
// a sequence's length on every call, so it cannot store one token in several layers.
// Synthetic activations: each layer reads its Q/K/V as a window of a seeded bank shifted by a
// per-layer (and, in decode, per-step) row offset, so every layer sees different data.
// Timings are GPU time from HIP events (dispatch and allocation included). Prints a summary;
// --json PATH writes it as JSON; --dump DIR writes sampled (layer, sequence) inputs and outputs
// of the prefill and of the first and last decode step as raw fp16 files plus manifest.json,
// for an external check against an attention oracle.
//
//   rollout_engine [--requests N] [--max-new T] [--min-prompt P] [--layers L] [--json PATH]
//                  [--dump DIR]

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
constexpr int64_t kLayerShift = 7;        // prefill bank rows between consecutive layers
constexpr int64_t kDecodeWindow = 2048;   // decode bank rows beyond the batch

int64_t DecodeShift(int64_t layer, int64_t step) { return (layer * 37 + step * 11) % kDecodeWindow; }

struct Args {
    int64_t requests = 16;
    int64_t max_new = 32;
    int64_t min_prompt = 256;
    int64_t layers = 36;
    std::string json;
    std::string dump;
};

Args Parse(int argc, char** argv) {
    Args a;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string k = argv[i];
        if (k == "--requests") a.requests = std::atoll(argv[i + 1]);
        else if (k == "--max-new") a.max_new = std::atoll(argv[i + 1]);
        else if (k == "--min-prompt") a.min_prompt = std::atoll(argv[i + 1]);
        else if (k == "--layers") a.layers = std::atoll(argv[i + 1]);
        else if (k == "--json") a.json = argv[i + 1];
        else if (k == "--dump") a.dump = argv[i + 1];
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

// Seeded fp16 bits in [-scale, scale] (xorshift32).
std::vector<uint16_t> RandomBits(int64_t n, uint32_t seed, float scale) {
    std::vector<uint16_t> bits(static_cast<size_t>(n));
    uint32_t s = seed ? seed : 1u;
    for (auto& b : bits) {
        s ^= s << 13;
        s ^= s >> 17;
        s ^= s << 5;
        b = HalfBits(scale * (-1.0f + 2.0f * static_cast<float>(s) / 4294967295.0f));
    }
    return bits;
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

// A seeded fp16 bank: host bits (kept for the dump) and the device copy.
struct Bank {
    std::vector<uint16_t> host;
    sci::Tensor dev;
    int64_t row_elems = 0;  // elements per token row
};

Bank MakeBank(int64_t rows, int64_t heads, uint32_t seed, float scale) {
    Bank b;
    b.row_elems = heads * kHeadDim;
    b.host = RandomBits(rows * b.row_elems, seed, scale);
    sci::Device& dev = sci::GpuDevice(0);
    b.dev = sci::Tensor(sci::TensorShape({rows, heads, kHeadDim}), sci::DType::kFloat16, dev);
    if (b.dev.data() != nullptr) dev.copy_to_device(b.dev.data(), b.host.data(), b.host.size() * 2);
    return b;
}

// A device view of `rows` token rows starting at row `first`, shaped `dims`.
sci::Tensor View(Bank& b, int64_t first, std::vector<int64_t> dims) {
    return sci::Tensor(sci::TensorShape(std::move(dims)), sci::DType::kFloat16,
                       sci::GpuDevice(0),
                       static_cast<uint16_t*>(b.dev.data()) + first * b.row_elems);
}

// Appends rows [first, first + n) of a bank (host bits) to dst.
void AppendRows(std::vector<uint16_t>& dst, const Bank& b, int64_t first, int64_t n) {
    const auto* p = b.host.data() + first * b.row_elems;
    dst.insert(dst.end(), p, p + n * b.row_elems);
}

struct Dumper {
    std::string dir;
    std::string manifest;
    int count = 0;
    bool on() const { return !dir.empty(); }
    void Write(const std::string& tag, const void* data, size_t bytes,
               const std::vector<int64_t>& shape) {
        const std::string file = tag + ".f16";
        std::ofstream f(dir + "/" + file, std::ios::binary);
        f.write(static_cast<const char*>(data), static_cast<std::streamsize>(bytes));
        manifest += std::string(count++ ? ",\n" : "") + "  \"" + tag + "\": [";
        for (size_t i = 0; i < shape.size(); ++i) {
            manifest += (i ? ", " : "") + std::to_string(shape[i]);
        }
        manifest += "]";
    }
    void Finish(const std::string& extra) {
        std::ofstream f(dir + "/manifest.json");
        f << "{\"arrays\": {\n" << manifest << "\n}, " << extra << "}\n";
    }
};

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
    const int64_t layers = args.layers;
    if (n < 1 || layers < 1 || args.max_new < 1) {
        std::printf("[rollout] --requests, --layers and --max-new must be positive\n");
        return 1;
    }

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
    kv.num_layers = layers;
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

    Dumper dump{args.dump};
    // Sampled (layer, sequence) pairs for the dump.
    const std::vector<int64_t> dump_layers = {0, layers / 2, layers - 1};
    const std::vector<int64_t> dump_seqs = {0, std::min<int64_t>(1, n - 1)};
    auto dumped_layer = [&](int64_t l) {
        return dump.on() && std::find(dump_layers.begin(), dump_layers.end(), l) != dump_layers.end();
    };

    // ---- prefill: reserve every prompt token once, then each layer --------------------------------
    // Layer l reads bank rows [l * kLayerShift, l * kLayerShift + total).
    Bank pq = MakeBank(total + layers * kLayerShift, kHeadsQ, 1000, 1.0f);
    Bank pk = MakeBank(total + layers * kLayerShift, kHeadsKv, 2000, 1.0f);
    Bank pv = MakeBank(total + layers * kLayerShift, kHeadsKv, 3000, 0.5f);
    std::vector<int64_t> packed_ids;
    packed_ids.reserve(static_cast<size_t>(total));
    for (int64_t r = 0; r < n; ++r) packed_ids.insert(packed_ids.end(), prompt[static_cast<size_t>(r)], r);
    sca::AttentionConfig pcfg;
    pcfg.backend = sca::BackendKind::kFlash;
    pcfg.causal = true;
    Timer timer;
    // One untimed call first: code-object loading and first-use allocations are not serving time.
    if (!sca::flash_attention_varlen(View(pq, 0, {total, kHeadsQ, kHeadDim}),
                                     View(pk, 0, {total, kHeadsKv, kHeadDim}),
                                     View(pv, 0, {total, kHeadsKv, kHeadDim}), n, cu.data(),
                                     cu.data(), max_prompt, max_prompt, pcfg).ok()) {
        std::printf("[rollout] warm-up prefill failed\n");
        return 4;
    }
    double prefill_attend_ms = 0.0;
    timer.Start();
    sci::Status st = cache.ReserveTokensBatch(packed_ids.data(), total, nullptr);
    if (!st.ok()) return Fail("prompt reservation", st);
    const double prompt_reserve_ms = timer.StopMs();
    double prompt_write_ms = 0.0;
    for (int64_t l = 0; l < layers; ++l) {
        const int64_t off = l * kLayerShift;
        const sci::Tensor kl = View(pk, off, {total, kHeadsKv, kHeadDim});
        const sci::Tensor vl = View(pv, off, {total, kHeadsKv, kHeadDim});
        timer.Start();
        const auto pre = sca::flash_attention_varlen(View(pq, off, {total, kHeadsQ, kHeadDim}), kl,
                                                     vl, n, cu.data(), cu.data(), max_prompt,
                                                     max_prompt, pcfg);
        prefill_attend_ms += timer.StopMs();
        if (!pre.ok()) return Fail("prefill", pre.error());
        timer.Start();
        st = cache.WriteReservedLayer(l, kl, vl, nullptr);
        prompt_write_ms += timer.StopMs();
        if (!st.ok()) return Fail("prompt layer write", st);
        if (dumped_layer(l)) {
            std::vector<uint16_t> out(static_cast<size_t>(total * kHeadsQ * kHeadDim));
            device.copy_to_host(out.data(), pre->out.data(), out.size() * 2);
            for (int64_t r : dump_seqs) {
                const int64_t a = cu[static_cast<size_t>(r)], L = prompt[static_cast<size_t>(r)];
                const std::string tag = "prefill_l" + std::to_string(l) + "_s" + std::to_string(r);
                std::vector<uint16_t> q, k, v;
                AppendRows(q, pq, off + a, L);
                AppendRows(k, pk, off + a, L);
                AppendRows(v, pv, off + a, L);
                dump.Write(tag + "_q", q.data(), q.size() * 2, {L, kHeadsQ, kHeadDim});
                dump.Write(tag + "_k", k.data(), k.size() * 2, {L, kHeadsKv, kHeadDim});
                dump.Write(tag + "_v", v.data(), v.size() * 2, {L, kHeadsKv, kHeadDim});
                dump.Write(tag + "_out", out.data() + a * kHeadsQ * kHeadDim,
                           static_cast<size_t>(L * kHeadsQ * kHeadDim) * 2, {L, kHeadsQ, kHeadDim});
            }
        }
    }
    double prefill_flops = 0.0;
    for (int32_t L : prompt) prefill_flops += 4.0 * kHeadsQ * kHeadDim * (0.5 * L * (L + 1.0));
    prefill_flops *= static_cast<double>(layers);

    // ---- decode loop ----------------------------------------------------------------------------
    // Step s, layer l reads bank rows [DecodeShift(l, s), DecodeShift(l, s) + n).
    Bank dq = MakeBank(n + kDecodeWindow, kHeadsQ, 5000, 1.0f);
    Bank dk = MakeBank(n + kDecodeWindow, kHeadsKv, 6000, 1.0f);
    Bank dv = MakeBank(n + kDecodeWindow, kHeadsKv, 7000, 0.5f);
    std::vector<int64_t> ids(static_cast<size_t>(n));
    for (int64_t r = 0; r < n; ++r) ids[static_cast<size_t>(r)] = r;
    std::vector<int32_t> lens(prompt);
    sci::Tensor seq_lens(sci::TensorShape({n}), sci::DType::kInt32, device);
    sca::AttentionConfig dcfg;
    dcfg.backend = sca::BackendKind::kPaged;
    {
        // Untimed attend over the prompts (kernel loading, scratch allocation).
        device.copy_to_device(seq_lens.data(), lens.data(), lens.size() * sizeof(int32_t));
        sca::PagedAttentionParams params;
        params.seq_lens = static_cast<const int32_t*>(seq_lens.data());
        params.num_seqs = n;
        params.block_size = kBlockSize;
        st = cache.SyncPageTable(nullptr);
        if (!st.ok() || !sca::paged_attention(View(dq, 0, {n, kHeadsQ, 1, kHeadDim}), cache, params,
                                              dcfg).ok()) {
            std::printf("[rollout] warm-up decode failed\n");
            return 4;
        }
    }
    std::vector<void*> ev(static_cast<size_t>(2 * layers + 2));
    for (auto& e : ev) sca_hip_event_create(&e);
    std::vector<double> step_ms, attend_ms, append_ms;
    double attend_bytes = 0.0;
    for (int64_t step = 0; step < args.max_new; ++step) {
        const bool dump_step = dump.on() && (step == 0 || step == args.max_new - 1);
        sca_hip_event_record(ev[0], nullptr);
        st = cache.ReserveTokensBatch(ids.data(), n, nullptr);
        if (!st.ok()) return Fail("decode reservation", st);
        st = cache.SyncPageTable(nullptr);
        if (!st.ok()) return Fail("page-table sync", st);
        for (auto& L : lens) ++L;  // the new token is attended in this step
        device.copy_to_device(seq_lens.data(), lens.data(), lens.size() * sizeof(int32_t));
        sca::PagedAttentionParams params;
        params.page_table = cache.PageTableDevicePtr();
        params.seq_lens = static_cast<const int32_t*>(seq_lens.data());
        params.num_seqs = n;
        params.block_size = kBlockSize;
        params.max_blocks_per_seq = cache.MaxBlocksPerSeq();
        for (int64_t l = 0; l < layers; ++l) {
            const int64_t off = DecodeShift(l, step);
            st = cache.WriteReservedLayer(l, View(dk, off, {n, kHeadsKv, kHeadDim}),
                                          View(dv, off, {n, kHeadsKv, kHeadDim}), nullptr);
            if (!st.ok()) return Fail("decode layer write", st);
            params.layer = l;
            sca_hip_event_record(ev[static_cast<size_t>(1 + 2 * l)], nullptr);
            const auto out = sca::paged_attention(View(dq, off, {n, kHeadsQ, 1, kHeadDim}), cache,
                                                  params, dcfg);
            sca_hip_event_record(ev[static_cast<size_t>(2 + 2 * l)], nullptr);
            if (!out.ok()) return Fail("paged attention", out.error());
            if (dump_step && dumped_layer(l)) {
                std::vector<uint16_t> o(static_cast<size_t>(n * kHeadsQ * kHeadDim));
                device.copy_to_host(o.data(), out->out.data(), o.size() * 2);
                for (int64_t r : dump_seqs) {
                    const std::string tag = "decode" + std::to_string(step) + "_l" +
                                            std::to_string(l) + "_s" + std::to_string(r);
                    std::vector<uint16_t> q, k, v;
                    AppendRows(q, dq, off + r, 1);
                    // History: the prompt rows of this layer, then this layer's decode rows.
                    AppendRows(k, pk, l * kLayerShift + cu[static_cast<size_t>(r)],
                               prompt[static_cast<size_t>(r)]);
                    AppendRows(v, pv, l * kLayerShift + cu[static_cast<size_t>(r)],
                               prompt[static_cast<size_t>(r)]);
                    for (int64_t s2 = 0; s2 <= step; ++s2) {
                        AppendRows(k, dk, DecodeShift(l, s2) + r, 1);
                        AppendRows(v, dv, DecodeShift(l, s2) + r, 1);
                    }
                    const int64_t L = lens[static_cast<size_t>(r)];
                    dump.Write(tag + "_q", q.data(), q.size() * 2, {1, kHeadsQ, kHeadDim});
                    dump.Write(tag + "_k", k.data(), k.size() * 2, {L, kHeadsKv, kHeadDim});
                    dump.Write(tag + "_v", v.data(), v.size() * 2, {L, kHeadsKv, kHeadDim});
                    dump.Write(tag + "_out", o.data() + r * kHeadsQ * kHeadDim,
                               static_cast<size_t>(kHeadsQ * kHeadDim) * 2, {1, kHeadsQ, kHeadDim});
                }
            }
        }
        sca_hip_event_record(ev.back(), nullptr);
        sca_hip_event_synchronize(ev.back());
        float ms = 0.0f;
        sca_hip_event_elapsed_ms(&ms, ev[0], ev.back());
        if (!dump_step) step_ms.push_back(ms);
        double attend = 0.0;
        for (int64_t l = 0; l < layers; ++l) {
            sca_hip_event_elapsed_ms(&ms, ev[static_cast<size_t>(1 + 2 * l)],
                                     ev[static_cast<size_t>(2 + 2 * l)]);
            attend += ms;
        }
        if (!dump_step) {
            attend_ms.push_back(attend);
            append_ms.push_back(step_ms.back() - attend);
            for (int32_t L : lens) attend_bytes += 2.0 * L * kHeadsKv * kHeadDim * 2 * layers;
        }
    }
    for (auto& e : ev) sca_hip_event_destroy(e);
    if (step_ms.empty()) {  // every step was a dump step
        step_ms.push_back(0.0);
        attend_ms.push_back(0.0);
        append_ms.push_back(0.0);
    }

    double attend_total = 0.0, step_total = 0.0;
    for (double t : attend_ms) attend_total += t;
    for (double t : step_ms) step_total += t;
    const int64_t generated = n * args.max_new;
    const double mean_step = step_total / static_cast<double>(step_ms.size());
    const double tokens_per_s = mean_step > 0.0 ? static_cast<double>(n) / (mean_step * 1e-3) : 0.0;
    const double attend_gbps = attend_total > 0.0 ? attend_bytes / (attend_total * 1e-3) / 1e9 : 0.0;
    const double prefill_tflops = prefill_flops / (prefill_attend_ms * 1e-3) / 1e12;
    const auto stats = cache.Stats();
    std::printf("[rollout] requests=%lld layers=%lld prompts=[%d..%d] tokens=%lld max_new=%lld\n",
                static_cast<long long>(n), static_cast<long long>(layers),
                *std::min_element(prompt.begin(), prompt.end()), static_cast<int>(max_prompt),
                static_cast<long long>(total), static_cast<long long>(args.max_new));
    std::printf("[rollout] prefill  attention %.3f ms over %lld layers (%.1f TFLOP/s); reserve %.3f ms, "
                "layer writes %.3f ms\n",
                prefill_attend_ms, static_cast<long long>(layers), prefill_tflops, prompt_reserve_ms,
                prompt_write_ms);
    std::printf("[rollout] decode   step P50=%.3f ms P99=%.3f ms (all layers); attention %.3f ms/step "
                "(%.0f GB/s); reserve+sync+writes %.3f ms/step\n",
                Percentile(step_ms, 0.5), Percentile(step_ms, 0.99), Percentile(attend_ms, 0.5),
                attend_gbps, Percentile(append_ms, 0.5));
    std::printf("[rollout] decode tokens/s=%.0f (attention and cache only) used_blocks=%lld/%lld\n",
                tokens_per_s, static_cast<long long>(stats.used_blocks),
                static_cast<long long>(stats.num_blocks));
    if (dump.on()) {
        std::string seqs = "[";
        for (size_t i = 0; i < dump_seqs.size(); ++i) seqs += (i ? ", " : "") + std::to_string(dump_seqs[i]);
        std::string lay = "[";
        for (size_t i = 0; i < dump_layers.size(); ++i) lay += (i ? ", " : "") + std::to_string(dump_layers[i]);
        dump.Finish("\"layers\": " + lay + "], \"seqs\": " + seqs + "], \"max_new\": " +
                    std::to_string(args.max_new));
    }
    if (!args.json.empty()) {
        std::ofstream f(args.json);
        f << "{\"engine\": \"rollout_engine\", \"requests\": " << n << ", \"layers\": " << layers
          << ", \"max_new_tokens\": " << args.max_new << ", \"prompt_tokens\": " << total
          << ", \"prefill_attention_ms\": " << prefill_attend_ms << ", \"prefill_tflops\": "
          << prefill_tflops << ", \"prompt_reserve_ms\": " << prompt_reserve_ms
          << ", \"prompt_layer_writes_ms\": " << prompt_write_ms
          << ", \"decode_step_ms\": {\"p50\": " << Percentile(step_ms, 0.5) << ", \"p99\": "
          << Percentile(step_ms, 0.99) << "}, \"decode_attention_ms_p50\": "
          << Percentile(attend_ms, 0.5) << ", \"decode_reserve_sync_writes_ms_p50\": "
          << Percentile(append_ms, 0.5) << ", \"decode_attend_gbps\": " << attend_gbps
          << ", \"decode_tokens_per_s\": " << tokens_per_s << ", \"generated_tokens\": "
          << generated << ", \"kv_blocks_used\": " << stats.used_blocks
          << ", \"shape\": {\"Hq\": " << kHeadsQ << ", \"Hkv\": " << kHeadsKv << ", \"D\": "
          << kHeadDim << "}}\n";
    }
    return 0;
}

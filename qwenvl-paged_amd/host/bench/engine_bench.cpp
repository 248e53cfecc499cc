// The headline decode (one Qwen2-VL-7B attention layer: Hq 28 over Hkv 4,
// head_dim 128, 16 tokens per block, bf16 KV) through the engine's entry
// point instead of the C ABI: a device-placement MemoryAllocator whose free
// list is shuffled (seeded), one sequence per context length created with
// KVCacheManager and grown with reserve_tokens, and every step decoded from
// the sequences' CacheViews by PagedAttentionBatch -- the page-table walk,
// the pack with the decode's work schedule, the upload and the decode, as the
// reference engine calls paged_attention_decode per view after each step's
// bookkeeping (PagedAttention.h:53-58).
//
// Reported (GPU time per step from HIP events on the engine stream, host time
// per step beside it):
//   sequential_step_us   one decode() at a time, the stream idle while the
//                        host walks and packs (median of event pairs);
//   pipelined_step_us    decode() per step enqueued back to back: the host
//                        prepares step n + 1 while step n runs;
//   pack_ahead_step_us   two PagedAttentionBatch objects with pack_ahead():
//                        step n + 1's upload rides in step n's decode launch;
//   kernel_us            the decode kernel alone on the packed batch (the
//                        engine's other layers of a step).
// Frame contents are a constant bf16 pattern: this driver times the entry
// point; the numerics of the same path are checked by the device test suites.
//
// Output: one JSON line. Usage: engine_bench --lens L0,L1,... [--seed S] [--reps N] [--spare PERCENT]
#include "qvp.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/PagedAttention.h"

#include "pipelined_steps.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

using namespace qwenvl_paged;

namespace {

[[noreturn]] void die(const std::string& what) {
    std::fprintf(stderr, "engine_bench: %s\n", what.c_str());
    std::exit(1);
}

void check(bool ok, const std::string& what) {
    if (!ok) die(what);
}

}  // namespace

int main(int argc, char** argv) {
    std::vector<std::uint32_t> lens;
    std::uint64_t seed = 2;
    std::uint32_t reps = 50, spare_percent = 10;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string k = argv[i];
        const std::string v = argv[i + 1];
        if (k == "--lens") {
            std::size_t at = 0;
            while (at < v.size()) {
                const std::size_t end = v.find(',', at);
                lens.push_back(static_cast<std::uint32_t>(std::strtoul(v.substr(at, end - at).c_str(), nullptr, 10)));
                at = end == std::string::npos ? v.size() : end + 1;
            }
        } else if (k == "--seed") {
            seed = std::strtoull(v.c_str(), nullptr, 10);
        } else if (k == "--reps") {
            reps = static_cast<std::uint32_t>(std::max<unsigned long>(5, std::strtoul(v.c_str(), nullptr, 10)));
        } else if (k == "--spare") {
            spare_percent = static_cast<std::uint32_t>(std::strtoul(v.c_str(), nullptr, 10));
        }
    }
    check(!lens.empty(), "--lens is required");
    constexpr std::uint32_t kTpb = 16, kHkv = 4, kHq = 28, kD = 128;
    const BlockShape shape{kTpb, 1, kHkv, kD, 2};
    std::uint64_t need = 0, tokens = 0;
    for (std::uint32_t c : lens) {
        check(c > 0, "zero context length");
        need += (c + kTpb - 1) / kTpb;
        tokens += c;
    }
    const std::uint32_t pool = static_cast<std::uint32_t>(std::ceil(need * (1.0 + spare_percent / 100.0)));

    AllocatorConfig cfg;
    cfg.block_shape = shape;
    cfg.max_blocks = pool;
    cfg.placement = BlockPlacement::Device;
    MemoryAllocator alloc(cfg);
    check(alloc.ok(), "pool: " + alloc.last_error());
    void* stream = alloc.stream();
    check(qvp_fill_bytes(alloc.device_base(), 0x3c, static_cast<std::size_t>(pool) * alloc.block_stride(), stream) ==
              QVP_OK,
          "fill");
    // Shuffle the free list: take every frame, give them back in a seeded
    // order, so the sequences' tables are scattered over the pool.
    {
        std::vector<PhysicalBlockId> all;
        for (std::uint32_t i = 0; i < pool; ++i) {
            const std::optional<PhysicalBlockId> f = alloc.allocate();
            check(f.has_value(), "allocate");
            all.push_back(*f);
        }
        std::mt19937_64 rng(seed);
        std::shuffle(all.begin(), all.end(), rng);
        for (PhysicalBlockId f : all) alloc.release(f);
    }
    KVCacheManager cache(alloc);
    std::vector<CacheView> views;
    for (std::size_t b = 0; b < lens.size(); ++b) {
        const SequenceId id = b + 1;
        check(cache.create_sequence(SequenceMetadata{id, id, {}, {}}), "create_sequence");
        check(cache.reserve_tokens(id, lens[b]), "reserve_tokens");
    }
    for (std::size_t b = 0; b < lens.size(); ++b) views.push_back(*cache.cache_view(b + 1));

    const std::size_t qbytes = lens.size() * kHq * kD * 2;
    void *dq = nullptr, *dout = nullptr;
    check(qvp_malloc(&dq, qbytes) == QVP_OK && qvp_malloc(&dout, qbytes) == QVP_OK, "q/out");
    check(qvp_fill_bytes(dq, 0x3c, qbytes, stream) == QVP_OK, "q fill");
    const float scale = 1.0f / std::sqrt(static_cast<float>(kD));
    PagedAttentionBatch attn;
    check(attn.decode(views, lens, 0, kHq, scale, dq, dout, ElementType::BF16), attn.last_error());
    check(qvp_stream_synchronize(stream) == QVP_OK, "sync");

    // The decode kernel alone: the packed batch decoded again (its schedule is
    // cached), as the engine's other layers of a step. Run first and long
    // enough for the device to reach its sustained clocks.
    const KVBlockLayout layout{shape};
    qvp_decode_args args{};
    args.query = dq;
    args.out = dout;
    args.kv_base = alloc.device_base();
    args.block_stride = alloc.block_stride();
    args.batch = attn.packed();
    args.kv_dtype = QVP_DTYPE_BF16;
    args.out_dtype = QVP_DTYPE_BF16;
    args.num_layers = 1;
    args.num_query_heads = kHq;
    args.num_kv_heads = kHkv;
    args.head_dim = kD;
    args.tokens_per_block = kTpb;
    args.head_stride = layout.head_stride();
    args.token_stride = layout.token_stride();
    args.stream_stride = layout.stream_stride();
    args.layer_stride = layout.layer_stride();
    args.scale = scale;
    auto kernel_step = [&](int) { check(qvp_paged_decode(&args, stream) == QVP_OK, qvp_last_error()); };
    (void)pipelined_steps::measure(stream, 400, kernel_step);
    const pipelined_steps::Times kernel = pipelined_steps::measure(stream, static_cast<int>(reps), kernel_step);

    void *e0 = nullptr, *e1 = nullptr;
    check(qvp_event_create(&e0) == QVP_OK && qvp_event_create(&e1) == QVP_OK, "events");
    std::vector<float> times;
    for (std::uint32_t r = 0; r < reps; ++r) {
        check(qvp_event_record(e0, stream) == QVP_OK, "record");
        check(attn.decode(views, lens, 0, kHq, scale, dq, dout, ElementType::BF16), attn.last_error());
        check(qvp_event_record(e1, stream) == QVP_OK && qvp_stream_synchronize(stream) == QVP_OK, "sync");
        float ms = 0.f;
        check(qvp_event_elapsed_ms(&ms, e0, e1) == QVP_OK, "elapsed");
        times.push_back(ms);
    }
    std::sort(times.begin(), times.end());
    const double sequential_us = 1e3 * times[times.size() / 2];

    PagedAttentionBatch ahead_a, ahead_b;
    const pipelined_steps::Forms piped = pipelined_steps::run_forms(
        attn, ahead_a, ahead_b, views, lens, 0, kHq, scale, dq, dout, ElementType::BF16, stream, static_cast<int>(reps));

    const double kv_bytes = static_cast<double>(tokens) * kHkv * kD * 2 * 2;
    const double n = static_cast<double>(lens.size());
    std::printf(
        "{\"mode\": \"engine_entry\", \"entry\": \"PagedAttentionBatch over CacheViews\", \"sequences\": %zu, "
        "\"cached_tokens\": %llu, \"pool_blocks\": %u, \"kernel_us\": %.3f, \"kernel_kv_GBps\": %.1f, "
        "\"sequential_step_us\": %.3f, \"pipelined_step_us\": %.3f, \"pipelined_host_us_per_step\": %.3f, "
        "\"pack_ahead_step_us\": %.3f, \"pack_ahead_host_us_per_step\": %.3f, \"pack_ahead_over_kernel\": %.4f, "
        "\"decode_tokens_per_s\": %.1f, \"decode_tokens_per_s_pipelined\": %.1f, "
        "\"decode_tokens_per_s_sequential\": %.1f, \"decode_tokens_per_s_kernel_only\": %.1f}\n",
        lens.size(), static_cast<unsigned long long>(tokens), pool, kernel.gpu_us_per_step,
        kv_bytes / (kernel.gpu_us_per_step * 1e-6) / 1e9, sequential_us, piped.loop.gpu_us_per_step,
        piped.loop.host_us_per_step, piped.ahead.gpu_us_per_step, piped.ahead.host_us_per_step,
        piped.ahead.gpu_us_per_step / kernel.gpu_us_per_step, n / (piped.ahead.gpu_us_per_step * 1e-6),
        n / (piped.loop.gpu_us_per_step * 1e-6), n / (sequential_us * 1e-6), n / (kernel.gpu_us_per_step * 1e-6));
    (void)qvp_free(dq);
    (void)qvp_free(dout);
    (void)qvp_event_destroy(e0);
    (void)qvp_event_destroy(e1);
    return 0;
}

// Continuous-batching step trace on device frames (the fifth benchmark
// configuration): 200 requests with prompts uniform on [128, 8192] and outputs
// uniform on [32, 1024] tokens (seeded), Qwen2-VL-7B KV shape (bf16, one layer),
// a pool of 60% of the blocks all requests would need, watermark preemption
// of 64 blocks, a pinned-host swap arena. Every step the Scheduler admits,
// preempts and resumes requests; decoding requests grow their tables
// (reserve_tokens at a block boundary, preempted when the pool is exhausted),
// go through the copy-on-write point and are decoded together by one paged
// decode (repacked every step). Preemption swaps blocks out to the pinned
// arena and resume swaps them back, as batched gathers/scatters on the side
// stream.
//
// Checks at the end: every request finished, the pool and the swap arena are
// empty again. Output: one JSON line with decode tokens/s over the trace (wall
// clock, host scheduling and packing included), the decode kernels' own rate,
// and the swap traffic's rate.
//
// Usage: trace_bench [--requests N] [--seed S] [--pool-percent P] [--watermark B]
#include "qvp.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/PagedAttention.h"
#include "qwenvl_paged/Scheduler.h"
#include "qwenvl_paged/SwapBackend.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <string>
#include <vector>

using namespace qwenvl_paged;

namespace {

std::uint64_t splitmix(std::uint64_t& s) {
    std::uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

[[noreturn]] void die(const std::string& what) {
    std::fprintf(stderr, "trace_bench: %s\n", what.c_str());
    std::exit(1);
}

void check(bool ok, const std::string& what) {
    if (!ok) die(what);
}

}  // namespace

int main(int argc, char** argv) {
    std::uint32_t requests = 200, pool_percent = 60, watermark = 64;
    std::uint64_t seed = 5;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string k = argv[i];
        const std::uint64_t v = std::strtoull(argv[i + 1], nullptr, 10);
        if (k == "--requests") requests = static_cast<std::uint32_t>(v);
        else if (k == "--seed") seed = v;
        else if (k == "--pool-percent") pool_percent = static_cast<std::uint32_t>(v);
        else if (k == "--watermark") watermark = static_cast<std::uint32_t>(v);
    }
    constexpr std::uint32_t kTpb = 16, kHkv = 4, kHq = 28, kD = 128;
    const BlockShape shape{kTpb, 1, kHkv, kD, 2};

    struct Plan {
        std::uint32_t prompt, output;
    };
    std::vector<Plan> plans(requests);
    std::uint64_t s = seed;
    std::uint64_t demand_blocks = 0, total_output = 0;
    for (Plan& p : plans) {
        p.prompt = 128 + static_cast<std::uint32_t>(splitmix(s) % (8192 - 128 + 1));
        p.output = 32 + static_cast<std::uint32_t>(splitmix(s) % (1024 - 32 + 1));
        demand_blocks += (p.prompt + p.output + kTpb - 1) / kTpb;
        total_output += p.output;
    }
    const std::uint32_t pool = static_cast<std::uint32_t>(demand_blocks * pool_percent / 100);

    AllocatorConfig cfg;
    cfg.block_shape = shape;
    cfg.max_blocks = pool;
    cfg.placement = BlockPlacement::Device;
    MemoryAllocator alloc(cfg);
    check(alloc.ok(), "pool: " + alloc.last_error());
    {
        // Give every frame bf16 content (one random frame repeated).
        std::vector<std::uint16_t> frame(shape.byte_size() / 2);
        std::uint64_t r = 99;
        for (auto& x : frame) x = static_cast<std::uint16_t>(0x3c00u | (splitmix(r) & 0x00ffu) | ((r & 1) << 15));
        for (std::uint32_t f = 0; f < pool; ++f) {
            check(alloc.write_block_bytes(f, 0, frame.data(), shape.byte_size()), "fill");
        }
    }
    PinnedSwapBackend swap(alloc, static_cast<std::size_t>(demand_blocks));
    check(swap.ok(), "swap arena");
    alloc.set_swap_backend(&swap);
    KVCacheManager cache(alloc);
    SchedulerConfig sc;
    sc.max_active_requests = 256;
    sc.max_batch_tokens = 16384;
    sc.preemption_watermark_blocks = watermark;
    Scheduler sched(sc, cache, alloc);

    void* stream = alloc.stream();
    void* dq = nullptr;
    void* dout = nullptr;
    const std::size_t qbytes = static_cast<std::size_t>(sc.max_active_requests) * kHq * kD * 2;
    check(qvp_malloc(&dq, qbytes) == QVP_OK && qvp_malloc(&dout, qbytes) == QVP_OK, "q/out");
    check(qvp_fill_bytes(dq, 0x3c, qbytes, stream) == QVP_OK, "q fill");
    void *ed0 = nullptr, *ed1 = nullptr, *es0 = nullptr, *es1 = nullptr;
    check(qvp_event_create(&ed0) == QVP_OK && qvp_event_create(&ed1) == QVP_OK && qvp_event_create(&es0) == QVP_OK &&
              qvp_event_create(&es1) == QVP_OK,
          "events");
    PagedAttentionBatch attn;
    const float scale = 1.0f / std::sqrt(static_cast<float>(kD));

    for (std::uint32_t i = 0; i < requests; ++i) {
        Request r;
        r.request_id = i + 1;
        r.root_sequence_id = i + 1;
        r.prompt_tokens = plans[i].prompt;
        r.sampling.max_decode_tokens = plans[i].output;
        sched.enqueue(r);
    }

    std::map<std::uint64_t, std::uint32_t> length, produced;
    std::deque<std::uint64_t> parked;
    std::uint64_t decode_tokens = 0, steps = 0, finished = 0, preemptions = 0, resumes = 0;
    std::uint64_t swap_launch_before = alloc.swap_launches();
    double decode_gpu_ms = 0.0, swap_gpu_ms = 0.0;
    std::uint64_t swapped_out_blocks = 0, swapped_in_blocks = 0;
    std::vector<CacheView> views;
    std::vector<std::uint32_t> lens;
    std::vector<std::uint64_t> ids;
    const auto t0 = std::chrono::steady_clock::now();
    while (finished < requests && steps < 200000) {
        ++steps;
        bool pending = false;
        for (std::uint32_t i = 0; i < requests && !pending; ++i) {
            const auto st = sched.state(i + 1);
            pending = st && *st == RequestState::Pending;
        }
        if (!pending && !parked.empty()) {
            const std::uint64_t id = parked.front();
            const std::uint32_t blocks = static_cast<std::uint32_t>(cache.cache_view(id)->block_table->size());
            if (sched.resume(id)) {
                parked.pop_front();
                ++resumes;
                swapped_in_blocks += blocks;
            }
        }
        const BatchPlan plan = sched.schedule_next();
        for (std::uint32_t i = 0; i < requests; ++i) {
            const auto st = sched.state(i + 1);
            if (st && *st == RequestState::Preempted &&
                std::find(parked.begin(), parked.end(), i + 1) == parked.end()) {
                parked.push_back(i + 1);
                ++preemptions;
                swapped_out_blocks += sched.preemption_info(i + 1)->swapped_blocks;
            }
        }
        for (std::uint64_t id : plan.prefill_requests) {
            length[id] = plans[id - 1].prompt;
            sched.complete_step(id, 1);
        }
        views.clear();
        lens.clear();
        ids.clear();
        for (std::uint64_t id : plan.decode_requests) {
            const std::uint32_t pos = length[id];
            if (pos / kTpb >= cache.cache_view(id)->block_table->size() && !cache.reserve_tokens(id, 1)) {
                sched.preempt(id, "pool exhausted while growing");
                parked.push_back(id);
                ++preemptions;
                swapped_out_blocks += sched.preemption_info(id)->swapped_blocks;
                continue;
            }
            check(cache.ensure_token_writable(id, pos).has_value(), "append");
            length[id] = pos + 1;
            views.push_back(*cache.cache_view(id));
            lens.push_back(pos + 1);
            ids.push_back(id);
        }
        // Swap traffic and copy-on-write queued by this step run first, on
        // the side stream; the events bracket them as seen from the engine
        // stream.
        const bool swaps = alloc.pending_operations() > 0;
        if (swaps) {
            check(qvp_event_record(es0, stream) == QVP_OK, "record");
            check(alloc.flush(), "flush: " + alloc.last_error());
            check(qvp_event_record(es1, stream) == QVP_OK, "record");
        }
        if (!views.empty()) {
            check(qvp_event_record(ed0, stream) == QVP_OK, "record");
            check(attn.decode(views, lens, 0, kHq, scale, dq, dout, ElementType::BF16), attn.last_error());
            check(qvp_event_record(ed1, stream) == QVP_OK, "record");
        }
        check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
        float ms = 0.f;
        if (swaps) {
            check(qvp_event_elapsed_ms(&ms, es0, es1) == QVP_OK, "elapsed");
            swap_gpu_ms += ms;
        }
        if (!views.empty()) {
            check(qvp_event_elapsed_ms(&ms, ed0, ed1) == QVP_OK, "elapsed");
            decode_gpu_ms += ms;
            decode_tokens += views.size();
        }
        for (std::uint64_t id : ids) {
            sched.complete_step(id, 1);
            if (++produced[id] >= plans[id - 1].output) {
                sched.cancel(id);
                length.erase(id);
                produced.erase(id);
                ++finished;
            }
        }
    }
    const double wall = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    check(alloc.synchronize(), "final sync");
    const AllocatorStats st = alloc.stats();
    const bool drained = st.free_blocks == st.total_blocks && swap.resident_slots() == 0;
    const double swap_bytes = static_cast<double>(swapped_out_blocks + swapped_in_blocks) * shape.byte_size();
    std::printf(
        "{\"mode\": \"config5_trace\", \"requests\": %u, \"finished\": %llu, \"steps\": %llu, \"pool_blocks\": %u, "
        "\"demand_blocks\": %llu, \"decode_tokens\": %llu, \"expected_decode_tokens\": %llu, \"wall_s\": %.4f, "
        "\"decode_tokens_per_s\": %.1f, \"decode_kernel_ms_total\": %.3f, \"decode_tokens_per_s_kernel_only\": "
        "%.1f, \"preemptions\": %llu, \"resumes\": %llu, \"swapped_out_blocks\": %llu, \"swapped_in_blocks\": %llu, "
        "\"swap_bytes\": %.0f, \"swap_ms_total\": %.3f, \"swap_GBps\": %.2f, \"swap_launches\": %llu, "
        "\"drained\": %s}\n",
        requests, static_cast<unsigned long long>(finished), static_cast<unsigned long long>(steps), pool,
        static_cast<unsigned long long>(demand_blocks), static_cast<unsigned long long>(decode_tokens),
        static_cast<unsigned long long>(total_output), wall, decode_tokens / wall, decode_gpu_ms,
        decode_tokens / (decode_gpu_ms * 1e-3), static_cast<unsigned long long>(preemptions),
        static_cast<unsigned long long>(resumes), static_cast<unsigned long long>(swapped_out_blocks),
        static_cast<unsigned long long>(swapped_in_blocks), swap_bytes, swap_gpu_ms,
        swap_gpu_ms > 0 ? swap_bytes / (swap_gpu_ms * 1e-3) / 1e9 : 0.0,
        static_cast<unsigned long long>(alloc.swap_launches() - swap_launch_before), drained ? "true" : "false");
    (void)qvp_free(dq);
    (void)qvp_free(dout);
    return (finished == requests && drained) ? 0 : 2;
}

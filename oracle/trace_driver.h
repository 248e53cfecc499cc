// trace_driver.h - a deterministic continuous-batching trace over the public
// host API (Scheduler, KVCacheManager, MemoryAllocator, SwapBackend).
//
// TEST INFRASTRUCTURE. The same source is compiled twice: against the
// reference's headers into oracle/_ref (ref_shim.cpp, ref_scheduler_trace) and
// against this package's headers into the specification test binaries. Both
// runs write the same event log when the two implementations take the same
// decisions and hand out the same frame and swap-slot ids, which is what the
// committed fixtures tests/golden/scheduler_trace_*.txt pin.
//
// The engine loop is the one the reference's simulations use
// (tests/Scheduler.test.cpp:193-248 of the QwenVL-Paged tree): resume the
// oldest parked request when nothing is pending, schedule, finish prefills,
// grow each decoding request by one token (reserve_tokens(id, 1) at a block
// boundary, preempting the request when the pool is exhausted), and cancel
// requests at their output length. Requests arrive over time.
#pragma once

#include <cstdint>
#include <cstdio>
#include <map>
#include <string>
#include <vector>

namespace trace {

struct Config {
    std::uint32_t requests{32};
    std::uint32_t prompt_lo{16}, prompt_hi{256};
    std::uint32_t output_lo{4}, output_hi{64};
    std::uint32_t arrivals_per_step{2};
    std::uint32_t tokens_per_block{16};
    std::uint32_t pool_percent{60};  // of the blocks all requests would need at once
    std::uint32_t watermark_blocks{4};
    std::uint32_t max_active{16};
    std::uint32_t max_batch_tokens{1024};
    std::uint32_t max_steps{2000};
    std::uint64_t seed{5};
    // Requests that reach their output length are cancelled after every
    // decoding request of the step was handled (an engine cancels after the
    // step's decode ran over all of them), instead of inside the loop.
    bool cancel_after_decodes{false};
};

struct RequestPlan {
    std::uint32_t prompt;
    std::uint32_t output;
};

inline std::uint64_t splitmix(std::uint64_t& s) {
    std::uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline std::vector<RequestPlan> plan_requests(const Config& c) {
    std::uint64_t s = c.seed;
    std::vector<RequestPlan> out(c.requests);
    for (RequestPlan& r : out) {
        r.prompt = c.prompt_lo + static_cast<std::uint32_t>(splitmix(s) % (c.prompt_hi - c.prompt_lo + 1));
        r.output = c.output_lo + static_cast<std::uint32_t>(splitmix(s) % (c.output_hi - c.output_lo + 1));
    }
    return out;
}

inline std::uint32_t pool_blocks(const Config& c) {
    std::uint64_t total = 0;
    for (const RequestPlan& r : plan_requests(c)) {
        total += (r.prompt + r.output + c.tokens_per_block - 1) / c.tokens_per_block;
    }
    return static_cast<std::uint32_t>(total * c.pool_percent / 100);
}

// FNV-1a over 32-bit words.
struct Hash {
    std::uint32_t h{2166136261u};
    void add(std::uint32_t w) {
        for (int i = 0; i < 4; ++i) h = (h ^ ((w >> (8 * i)) & 0xFFu)) * 16777619u;
    }
};

// Runs the trace on an allocator (with its swap backend installed) and
// returns the event log. The template arguments are the qwenvl_paged types of
// the translation unit that instantiates it (reference or this package).
template <typename MemoryAllocator, typename KVCacheManager, typename Scheduler, typename SchedulerConfig,
          typename Request, typename RequestState>
std::string run(const Config& c, MemoryAllocator& allocator) {
    const std::vector<RequestPlan> plans = plan_requests(c);
    KVCacheManager cache(allocator);
    SchedulerConfig sc;
    sc.max_active_requests = c.max_active;
    sc.max_batch_tokens = c.max_batch_tokens;
    sc.preemption_watermark_blocks = c.watermark_blocks;
    Scheduler sched(sc, cache, allocator);

    std::map<std::uint64_t, std::uint32_t> length;   // tokens held by a live sequence
    std::map<std::uint64_t, std::uint32_t> decoded;  // output tokens produced
    std::vector<std::uint64_t> parked;               // preemption order
    std::vector<std::uint64_t> done;                 // finished this step (cancel_after_decodes)
    std::uint32_t arrived = 0, finished = 0;
    std::string log;
    char line[512];

    auto state_is = [&](std::uint64_t id, RequestState s) {
        auto st = sched.state(id);
        return st.has_value() && *st == s;
    };
    // Requests the scheduler preempted on its own (watermark) join the
    // parked list in id order.
    auto note_parked = [&](std::string& events) {
        for (const auto& kv : length) {
            const std::uint64_t id = kv.first;
            if (!state_is(id, RequestState::Preempted)) continue;
            bool known = false;
            for (std::uint64_t p : parked) known = known || p == id;
            if (!known) {
                parked.push_back(id);
                events += " watermark_preempt=" + std::to_string(id);
            }
        }
    };

    for (std::uint32_t step = 0; step < c.max_steps && finished < c.requests; ++step) {
        for (std::uint32_t k = 0; k < c.arrivals_per_step && arrived < c.requests; ++k, ++arrived) {
            Request r;
            r.request_id = arrived + 1;
            r.root_sequence_id = arrived + 1;
            r.prompt_tokens = plans[arrived].prompt;
            r.sampling.max_decode_tokens = plans[arrived].output;
            sched.enqueue(r);
            length[arrived + 1] = 0;
        }
        bool pending = false;
        for (const auto& kv : length) pending = pending || state_is(kv.first, RequestState::Pending);
        std::string events;
        if (!pending && !parked.empty()) {
            const std::uint64_t id = parked.front();
            if (sched.resume(id)) {
                parked.erase(parked.begin());
                events += " resume=" + std::to_string(id);
            }
        }
        const auto plan = sched.schedule_next();
        note_parked(events);
        for (std::uint64_t id : plan.prefill_requests) {
            length[id] = plans[id - 1].prompt;
            sched.complete_step(id, 1);
        }
        for (std::uint64_t id : plan.decode_requests) {
            const std::uint32_t pos = length[id];
            const auto view = cache.cache_view(id);
            if (pos / c.tokens_per_block >= view->block_table->size() && !cache.reserve_tokens(id, 1)) {
                sched.preempt(id, "pool exhausted while growing");
                parked.push_back(id);
                events += " grow_preempt=" + std::to_string(id);
                continue;
            }
            (void)cache.ensure_token_writable(id, pos);
            length[id] = pos + 1;
            if (++decoded[id] >= plans[id - 1].output) {
                if (c.cancel_after_decodes) {
                    done.push_back(id);
                    continue;
                }
                sched.cancel(id);
                length.erase(id);
                decoded.erase(id);
                ++finished;
                events += " done=" + std::to_string(id);
            }
        }
        for (std::uint64_t id : done) {
            sched.cancel(id);
            length.erase(id);
            decoded.erase(id);
            ++finished;
            events += " done=" + std::to_string(id);
        }
        done.clear();
        Hash h;
        for (const auto& kv : length) {
            const auto view = cache.cache_view(kv.first);
            if (!view) continue;
            h.add(static_cast<std::uint32_t>(kv.first));
            for (const auto& e : view->block_table->entries()) {
                h.add(e.physical_id);
                h.add(e.swap_slot ? static_cast<std::uint32_t>(*e.swap_slot) : 0xFFFFFFFFu);
                h.add(e.writable ? 1u : 0u);
            }
        }
        const auto st = allocator.stats();
        std::string pre, dec;
        for (std::uint64_t id : plan.prefill_requests) pre += std::to_string(id) + ",";
        for (std::uint64_t id : plan.decode_requests) dec += std::to_string(id) + ",";
        std::snprintf(line, sizeof line, " tok=%u free=%u shared=%u swapped=%u h=%08x", plan.scheduled_tokens,
                      st.free_blocks, st.shared_blocks, st.swapped_blocks, h.h);
        log += std::to_string(step) + " P=" + pre + " D=" + dec + line;
        log += events;
        log += "\n";
    }
    std::snprintf(line, sizeof line, "finished=%u of %u\n", finished, c.requests);
    log += line;
    return log;
}

}  // namespace trace

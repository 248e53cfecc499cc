#pragma once
// Timing of engine steps enqueued back to back, as a serving loop runs them:
// nothing synchronises between steps, so the host prepares step n + 1 while
// the GPU runs step n. Two forms of the step through PagedAttentionBatch:
//   loop   -- decode() per step: the walk, pack and schedule of step n + 1
//             overlap step n's decode; its upload kernel runs between the two
//             decodes;
//   ahead  -- two objects in turn, pack_ahead() for step n + 1 before step
//             n's decode_packed(): step n + 1's upload rides in the tail of
//             step n's decode launch, so decodes follow each other directly.
// The GPU time per step is the interval of two events around the K steps on
// the engine stream, over K; the host's own time per step (the wall time of
// the enqueueing loop, over K) is reported beside it: a step is host-bound
// when that is the larger.

#include "qvp.h"
#include "qwenvl_paged/PagedAttention.h"

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <utility>
#include <vector>

namespace pipelined_steps {

struct Times {
    double gpu_us_per_step{0.0};
    double host_us_per_step{0.0};
};

// Enqueues step(r) for r = 0 .. reps - 1 back to back on `stream`.
template <typename Step>
Times measure(void* stream, int reps, Step step) {
    void *e0 = nullptr, *e1 = nullptr;
    if (qvp_event_create(&e0) != QVP_OK || qvp_event_create(&e1) != QVP_OK) {
        std::fprintf(stderr, "pipelined_steps: events: %s\n", qvp_last_error());
        std::exit(1);
    }
    Times t;
    if (qvp_stream_synchronize(stream) != QVP_OK || qvp_event_record(e0, stream) != QVP_OK) std::exit(1);
    const auto h0 = std::chrono::steady_clock::now();
    for (int r = 0; r < reps; ++r) step(r);
    const auto h1 = std::chrono::steady_clock::now();
    float ms = 0.f;
    if (qvp_event_record(e1, stream) != QVP_OK || qvp_stream_synchronize(stream) != QVP_OK ||
        qvp_event_elapsed_ms(&ms, e0, e1) != QVP_OK) {
        std::fprintf(stderr, "pipelined_steps: %s\n", qvp_last_error());
        std::exit(1);
    }
    t.gpu_us_per_step = 1e3 * ms / reps;
    t.host_us_per_step = std::chrono::duration<double, std::micro>(h1 - h0).count() / reps;
    (void)qvp_event_destroy(e0);
    (void)qvp_event_destroy(e1);
    return t;
}

// Both forms for one batch of views; `decode_ok` aborts with the message of a
// refused call. Each form runs once untimed first (buffers reach their size).
struct Forms {
    Times loop, ahead;
};

inline Forms run_forms(qwenvl_paged::PagedAttentionBatch& single, qwenvl_paged::PagedAttentionBatch& a,
                       qwenvl_paged::PagedAttentionBatch& b, const std::vector<qwenvl_paged::CacheView>& views,
                       const std::vector<std::uint32_t>& lens, std::uint32_t layer, std::uint32_t heads, float scale,
                       const void* dq, void* dout, qwenvl_paged::ElementType out_type, void* stream, int reps) {
    auto ok = [](bool good, const qwenvl_paged::PagedAttentionBatch& x) {
        if (!good) {
            std::fprintf(stderr, "pipelined_steps: %s\n", x.last_error().c_str());
            std::exit(1);
        }
    };
    Forms f;
    auto loop_step = [&](int) { ok(single.decode(views, lens, layer, heads, scale, dq, dout, out_type), single); };
    (void)measure(stream, 2, loop_step);
    f.loop = measure(stream, reps, loop_step);
    qwenvl_paged::PagedAttentionBatch* cur = &a;
    qwenvl_paged::PagedAttentionBatch* nxt = &b;
    auto ahead_run = [&](int n) {
        ok(cur->pack_ahead(views, lens, layer, heads, scale, dq, dout, out_type), *cur);
        return measure(stream, n, [&](int r) {
            if (r + 1 < n) ok(nxt->pack_ahead(views, lens, layer, heads, scale, dq, dout, out_type), *nxt);
            ok(cur->decode_packed(), *cur);
            std::swap(cur, nxt);
        });
    };
    (void)ahead_run(2);
    f.ahead = ahead_run(reps);
    return f;
}

}  // namespace pipelined_steps

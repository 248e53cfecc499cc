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
// With --engine 1 every step also does the rest of a serving step's GPU work:
// admitted prompts get their K/V appended (KVAppendBatch), are attended by one
// causal prefill (PagedAttentionBatch::prefill) and get M-RoPE positions
// (MRopePositionBatch); decoding requests append their new token's K/V before
// the decode and get their position. K/V and queries are synthetic device
// buffers; each phase is timed with events on the engine stream. When the
// stream runs dry while the host prepares a phase (validation, the
// copy-on-write walk, staging uploads), a phase's event time includes that
// wait; a kernel trace gives the kernels' own time.
//
// Checks at the end: every request finished, the pool and the swap arena are
// empty again. Output: one JSON line with decode tokens/s over the trace (wall
// clock, host scheduling and packing included), the decode kernels' own rate,
// and the swap traffic's rate (plus, with --engine, prefill tokens and the
// time of each phase).
//
// With --log PATH the step-by-step decisions are written to PATH as an event
// log: per step the admitted (P=) and decoding (D=) requests, the scheduled
// tokens, the pool's free / shared / swapped counts, an FNV-1a hash over every
// live sequence's page table (frame, swap slot and writable flag of each
// entry) and the step's resume / preemption / completion events. Its format
// is the one tests/golden/scheduler_trace_config5.txt.gz holds, written by
// the reference's own Scheduler, KVCacheManager and MemoryAllocator for the
// same requests, so equal logs mean equal decisions and equal frame and slot
// ids.
//
// Steps are pipelined: the host prepares the next step (scheduler, cache
// manager, packing, swap queueing) while the GPU runs the current one, with at
// most --in-flight steps enqueued (default 2; 1 runs one step at a time). Swap
// batches run on the allocator's side stream beside the engine stream's work;
// their GPU time and bytes come from the allocator's per-batch events.
//
// With --verify 1 the bytes are checked as well as the decisions. Every K/V
// row is a seeded function of (sequence id, token position) (kv_pattern.h)
// and is written into its frame by the append kernel through the
// copy-on-write point -- prompt rows when a request is admitted, the new token
// every decode step -- so a frame's bytes are known wherever swaps moved them,
// and the queries are a seeded function of the batch row. After the decode of
// every step that follows a resume, and for four sequences of every
// --check-every'th step, the step enqueues on the engine stream (behind the
// decode, nothing synchronised) a gather of the sequence's frames (layer 0,
// K and V) and a download of its decode output into pinned memory; when the
// step retires, every row of those frames below the sequence's length is
// compared byte for byte with the pattern, and the outputs are written to
// --verify-dump PATH (records of step, sequence, batch row, context length and
// the bf16 output rows) for the test suite to compare with the oracle. Swap
// batches keep running on the side stream beside the engine work, as without
// the checks; timings in this mode include the host's pattern generation.
//
// Usage: trace_bench [--requests N] [--seed S] [--pool-percent P] [--watermark B] [--engine 0|1] [--log PATH]
//                    [--in-flight N] [--layers N] [--verify 0|1] [--verify-dump PATH] [--check-every N]
//
// --layers N stores all N layers of the model in each frame (N = 28: whole
// Qwen2-VL-7B frames of 917,504 B); every GPU phase works on layer 0, and swaps
// move whole frames.
#include "qvp.h"
#include "qwenvl_paged/KVAppend.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MRope.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/PagedAttention.h"
#include "qwenvl_paged/Scheduler.h"
#include "qwenvl_paged/SwapBackend.h"

#include "kv_pattern.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <set>
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

// FNV-1a over the four bytes of each 32-bit word.
struct Fnv {
    std::uint32_t h{2166136261u};
    void add(std::uint32_t w) {
        for (int i = 0; i < 4; ++i) h = (h ^ ((w >> (8 * i)) & 0xFFu)) * 16777619u;
    }
};

}  // namespace

int main(int argc, char** argv) {
    std::uint32_t requests = 200, pool_percent = 60, watermark = 64;
    std::uint64_t seed = 5;
    bool engine = false;
    int in_flight = 2;
    std::uint32_t layers = 1;
    bool verify = false;
    std::uint64_t check_every = 50;
    std::string log_path, dump_path;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string k = argv[i];
        if (k == "--log") {
            log_path = argv[i + 1];
            continue;
        }
        if (k == "--verify-dump") {
            dump_path = argv[i + 1];
            continue;
        }
        const std::uint64_t v = std::strtoull(argv[i + 1], nullptr, 10);
        if (k == "--requests") requests = static_cast<std::uint32_t>(v);
        else if (k == "--seed") seed = v;
        else if (k == "--pool-percent") pool_percent = static_cast<std::uint32_t>(v);
        else if (k == "--watermark") watermark = static_cast<std::uint32_t>(v);
        else if (k == "--engine") engine = v != 0;
        else if (k == "--in-flight") in_flight = static_cast<int>(std::max<std::uint64_t>(1, v));
        else if (k == "--layers") layers = static_cast<std::uint32_t>(std::max<std::uint64_t>(1, v));
        else if (k == "--verify") verify = v != 0;
        else if (k == "--check-every") check_every = std::max<std::uint64_t>(1, v);
    }
    constexpr std::uint32_t kTpb = 16, kHkv = 4, kHq = 28, kD = 128;
    const BlockShape shape{kTpb, layers, kHkv, kD, 2};

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
    constexpr std::size_t kQRow = static_cast<std::size_t>(kHq) * kD;  // elements of one query / output row
    constexpr std::size_t kKvRow = static_cast<std::size_t>(kHkv) * kD;  // elements of one token's K (or V) row
    if (verify) {
        // Query row i of every decode is the pattern's row i.
        std::vector<std::uint16_t> q(qbytes / 2);
        for (std::uint32_t r = 0; r < sc.max_active_requests; ++r) kv_pattern::query_row(r, q.data() + r * kQRow, kQRow);
        check(qvp_memcpy_htod(dq, q.data(), qbytes, stream) == QVP_OK && qvp_stream_synchronize(stream) == QVP_OK,
              "q upload");
    } else {
        check(qvp_fill_bytes(dq, 0x3c, qbytes, stream) == QVP_OK, "q fill");
    }
    PagedAttentionBatch attn;
    const float scale = 1.0f / std::sqrt(static_cast<float>(kD));

    // Engine mode: synthetic K/V rows, prefill queries/outputs, positions.
    PagedAttentionBatch prefill_attn;
    KVAppendBatch append;
    MRopePositionBatch positions;
    const std::size_t max_rows = static_cast<std::size_t>(sc.max_batch_tokens) + sc.max_active_requests;
    void *dk = nullptr, *dv = nullptr, *dpq = nullptr, *dpo = nullptr, *dpos = nullptr;
    // K/V rows go through the append kernel in engine mode and whenever bytes
    // are verified (the verified rows come from the pattern).
    const bool write_kv = engine || verify;
    const std::size_t row_bytes = kKvRow * 2;
    const std::size_t qrow_bytes = kQRow * 2;
    if (write_kv) {
        check(qvp_malloc(&dk, max_rows * row_bytes) == QVP_OK && qvp_malloc(&dv, max_rows * row_bytes) == QVP_OK,
              "K/V row buffers");
        check(qvp_fill_bytes(dk, 0x3b, max_rows * row_bytes, stream) == QVP_OK &&
                  qvp_fill_bytes(dv, 0x3c, max_rows * row_bytes, stream) == QVP_OK,
              "K/V row fill");
    }
    if (engine) {
        check(qvp_malloc(&dpq, max_rows * qrow_bytes) == QVP_OK && qvp_malloc(&dpo, max_rows * qrow_bytes) == QVP_OK &&
                  qvp_malloc(&dpos, max_rows * 3 * sizeof(std::int64_t)) == QVP_OK,
              "engine buffers");
        check(qvp_fill_bytes(dpq, 0x3c, max_rows * qrow_bytes, stream) == QVP_OK, "engine fill");
    }
    // Layer 0 of a frame: K rows then V rows, tpb rows of kKvRow elements each.
    const std::size_t stream_bytes = static_cast<std::size_t>(kTpb) * row_bytes;
    const std::size_t check_bytes = 2 * stream_bytes;
    std::FILE* dump = nullptr;
    if (verify && !dump_path.empty()) {
        dump = std::fopen(dump_path.c_str(), "wb");
        check(dump != nullptr, "opening " + dump_path);
    }
    // Per-step GPU timing without stalling the host: each step records
    // begin/end event pairs (append, prefill, decode, positions) and a final
    // event into one of `in_flight` slots; a slot is read back (waiting for
    // its step) only when it comes round again, so the host prepares up to
    // in_flight - 1 steps ahead while the GPU runs (1: one step at a time).
    enum Phase { kAppend = 0, kPrefill, kDecode, kPositions, kPhases };
    // A verified sequence of one step: its frames' layer-0 bytes sit at
    // frame_off in the slot's gather buffer, its output row at out_index.
    struct SeqCheck {
        std::uint64_t seq;
        std::uint32_t len, row, nblocks, out_index;
        std::size_t frame_off;
        bool after_resume;
    };
    struct StepEvents {
        void* ev[2 * kPhases]{};
        bool used[kPhases]{};
        void* fin{nullptr};
        bool pending{false};
        std::uint64_t step{0};
        // Verify mode (pinned; reused when the slot comes round again, after
        // the step that last used it has finished).
        std::uint16_t* rows_k{nullptr};
        std::uint16_t* rows_v{nullptr};
        std::uint8_t* frames{nullptr};
        std::size_t frames_cap{0};
        std::uint16_t* outs{nullptr};
        std::vector<SeqCheck> checks;
    };
    constexpr std::uint32_t kChecksPerStep = 4;  // sequences checked on every check_every'th step
    std::vector<StepEvents> ring(static_cast<std::size_t>(in_flight));
    for (StepEvents& r : ring) {
        for (void*& e : r.ev) check(qvp_event_create(&e) == QVP_OK, "events");
        check(qvp_event_create(&r.fin) == QVP_OK, "events");
        if (verify) {
            void *k = nullptr, *v = nullptr, *o = nullptr;
            check(qvp_host_alloc(&k, max_rows * row_bytes) == QVP_OK && qvp_host_alloc(&v, max_rows * row_bytes) == QVP_OK &&
                      qvp_host_alloc(&o, static_cast<std::size_t>(sc.max_active_requests) * qrow_bytes) == QVP_OK,
                  "verify buffers");
            r.rows_k = static_cast<std::uint16_t*>(k);
            r.rows_v = static_cast<std::uint16_t*>(v);
            r.outs = static_cast<std::uint16_t*>(o);
        }
    }
    double phase_ms[kPhases] = {0.0, 0.0, 0.0, 0.0};
    std::uint64_t seq_checks = 0, resume_checks = 0, rows_checked = 0, row_mismatches = 0, decode_records = 0;
    std::string first_mismatch;
    std::vector<std::uint16_t> expect_row(kKvRow);
    auto verify_slot = [&](StepEvents& r) {
        for (const SeqCheck& c : r.checks) {
            ++seq_checks;
            resume_checks += c.after_resume ? 1 : 0;
            for (std::uint32_t j = 0; j < c.nblocks; ++j) {
                const std::uint8_t* frame = r.frames + c.frame_off + static_cast<std::size_t>(j) * check_bytes;
                for (std::uint32_t t = 0; t < kTpb; ++t) {
                    const std::uint64_t pos = static_cast<std::uint64_t>(j) * kTpb + t;
                    if (pos >= c.len) break;
                    for (std::uint32_t st = 0; st < 2; ++st) {
                        kv_pattern::kv_row(c.seq, pos, st, expect_row.data(), kKvRow);
                        ++rows_checked;
                        if (std::memcmp(frame + st * stream_bytes + t * row_bytes, expect_row.data(), row_bytes) != 0) {
                            if (row_mismatches++ == 0) {
                                first_mismatch = "step " + std::to_string(r.step) + " sequence " + std::to_string(c.seq) +
                                                 " position " + std::to_string(pos) + (st ? " V" : " K") +
                                                 (c.after_resume ? " (after resume)" : "");
                            }
                        }
                    }
                }
            }
            if (dump != nullptr) {
                const std::uint32_t head[4] = {static_cast<std::uint32_t>(r.step), static_cast<std::uint32_t>(c.seq), c.row,
                                               c.len};
                check(std::fwrite(head, sizeof head, 1, dump) == 1 &&
                          std::fwrite(r.outs + static_cast<std::size_t>(c.out_index) * kQRow, qrow_bytes, 1, dump) == 1,
                      "writing the verify dump");
                ++decode_records;
            }
        }
        r.checks.clear();
    };
    auto retire = [&](StepEvents& r) {
        if (!r.pending) return;
        check(qvp_event_synchronize(r.fin) == QVP_OK, "step sync");
        for (int k = 0; k < kPhases; ++k) {
            if (!r.used[k]) continue;
            float ms = 0.f;
            check(qvp_event_elapsed_ms(&ms, r.ev[2 * k], r.ev[2 * k + 1]) == QVP_OK, "elapsed");
            phase_ms[k] += ms;
            r.used[k] = false;
        }
        if (verify) verify_slot(r);
        r.pending = false;
    };
    // Resumed sequences not yet checked (checked at their next decode).
    std::set<std::uint64_t> unchecked_resumes;
    std::uint64_t prefill_tokens = 0;
    std::vector<SequenceId> app_seq, pos_seq;
    std::vector<TokenPosition> app_pos, pos_begin, pos_end;
    std::vector<CacheView> pviews;
    std::vector<std::uint32_t> plens, pfirst;

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
    const std::uint64_t swap_launch_before = alloc.swap_launches();
    const double swap_ms_before = alloc.swap_gpu_ms();
    const std::uint64_t swap_bytes_before = alloc.swap_bytes_moved();
    std::uint64_t swapped_out_blocks = 0, swapped_in_blocks = 0;
    std::vector<CacheView> views;
    std::vector<std::uint32_t> lens;
    std::vector<std::uint64_t> ids;
    const auto t0 = std::chrono::steady_clock::now();
    std::string log;
    std::string events;
    while (finished < requests && steps < 200000) {
        StepEvents& slot = ring[steps % ring.size()];
        retire(slot);
        auto begin_phase = [&](Phase k) {
            slot.used[k] = true;
            check(qvp_event_record(slot.ev[2 * k], stream) == QVP_OK, "record");
        };
        auto end_phase = [&](Phase k) { check(qvp_event_record(slot.ev[2 * k + 1], stream) == QVP_OK, "record"); };
        ++steps;
        events.clear();
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
                events += " resume=" + std::to_string(id);
                if (verify) unchecked_resumes.insert(id);
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
                events += " watermark_preempt=" + std::to_string(i + 1);
            }
        }
        app_seq.clear();
        app_pos.clear();
        pos_seq.clear();
        pos_begin.clear();
        pos_end.clear();
        pviews.clear();
        plens.clear();
        pfirst.clear();
        for (std::uint64_t id : plan.prefill_requests) {
            const std::uint32_t n = plans[id - 1].prompt;
            length[id] = n;
            if (write_kv) {
                for (std::uint32_t t = 0; t < n; ++t) {
                    app_seq.push_back(id);
                    app_pos.push_back(t);
                }
            }
            if (engine) {
                pviews.push_back(*cache.cache_view(id));
                plens.push_back(n);
                pfirst.push_back(0);
                pos_seq.push_back(id);
                pos_begin.push_back(0);
                pos_end.push_back(n);
                prefill_tokens += n;
            }
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
                events += " grow_preempt=" + std::to_string(id);
                continue;
            }
            if (write_kv) {
                app_seq.push_back(id);
                app_pos.push_back(pos);
            } else {
                check(cache.ensure_token_writable(id, pos).has_value(), "append");
            }
            if (engine) {
                pos_seq.push_back(id);
                pos_begin.push_back(pos);
                pos_end.push_back(pos + 1);
            }
            length[id] = pos + 1;
            views.push_back(*cache.cache_view(id));
            lens.push_back(pos + 1);
            ids.push_back(id);
        }
        // Swap traffic queued by this step goes to the side stream now;
        // engine work below waits only where it touches the frames moved.
        check(alloc.flush(), "flush: " + alloc.last_error());
        if (write_kv && !app_seq.empty()) {
            // The step's K/V (prompt rows and decode tokens) through the
            // copy-on-write point: the blocks it shares are copied first, then
            // one store launch covers every row (offsets uploaded once when
            // there are more than 128).
            check(app_seq.size() <= max_rows, "append rows");
            if (verify) {
                // The pattern's rows, staged in this slot's pinned buffers
                // and copied on the engine stream ahead of the append.
                const std::size_t n = app_seq.size();
                for (std::size_t i = 0; i < n; ++i) {
                    kv_pattern::kv_row(app_seq[i], app_pos[i], 0, slot.rows_k + i * kKvRow, kKvRow);
                    kv_pattern::kv_row(app_seq[i], app_pos[i], 1, slot.rows_v + i * kKvRow, kKvRow);
                }
                check(qvp_memcpy_htod(dk, slot.rows_k, n * row_bytes, stream) == QVP_OK &&
                          qvp_memcpy_htod(dv, slot.rows_v, n * row_bytes, stream) == QVP_OK,
                      "row upload");
            }
            begin_phase(kAppend);
            check(append.append(cache, alloc, app_seq, app_pos, 0, 1, dk, dv), "append: " + append.last_error());
            end_phase(kAppend);
        }
        if (engine && !pviews.empty()) {
            begin_phase(kPrefill);
            check(prefill_attn.prefill(pviews, plens, pfirst, 0, kHq, scale, dpq, dpo, ElementType::BF16),
                  "prefill: " + prefill_attn.last_error());
            end_phase(kPrefill);
        }
        if (!views.empty()) {
            begin_phase(kDecode);
            check(attn.decode(views, lens, 0, kHq, scale, dq, dout, ElementType::BF16), attn.last_error());
            end_phase(kDecode);
            decode_tokens += views.size();
        }
        if (verify && !views.empty()) {
            // Sequences resumed since their last decode, and on every
            // check_every'th step four spread over the batch: their frames
            // and outputs as this decode left them, copied behind it on the
            // engine stream into the slot's pinned buffers.
            std::vector<std::size_t> picks;
            std::vector<bool> after_resume;
            for (std::size_t i = 0; i < ids.size(); ++i) {
                if (unchecked_resumes.erase(ids[i]) != 0) {
                    picks.push_back(i);
                    after_resume.push_back(true);
                }
            }
            if (steps % check_every == 0) {
                for (std::uint32_t k = 0; k < kChecksPerStep; ++k) {
                    const std::size_t i = static_cast<std::size_t>(k) * ids.size() / kChecksPerStep;
                    if (std::find(picks.begin(), picks.end(), i) != picks.end()) continue;
                    picks.push_back(i);
                    after_resume.push_back(false);
                }
            }
            std::vector<std::uint32_t> frame_ids;
            std::vector<std::uint64_t> offsets;
            for (std::size_t k = 0; k < picks.size(); ++k) {
                const std::size_t i = picks[k];
                SeqCheck c{};
                c.seq = ids[i];
                c.len = lens[i];
                c.row = static_cast<std::uint32_t>(i);
                c.nblocks = (lens[i] + kTpb - 1) / kTpb;
                c.out_index = static_cast<std::uint32_t>(k);
                c.frame_off = frame_ids.size() * check_bytes;
                c.after_resume = after_resume[k];
                for (std::uint32_t j = 0; j < c.nblocks; ++j) {
                    const std::optional<PhysicalBlockId> f = views[i].block_table->lookup(j);
                    check(f.has_value(), "checked sequence has an unmapped block");
                    offsets.push_back(frame_ids.size() * check_bytes);
                    frame_ids.push_back(*f);
                }
                slot.checks.push_back(c);
            }
            const std::size_t need = frame_ids.size() * check_bytes;
            if (need > slot.frames_cap) {
                // The slot was retired above: nothing reads the old buffer.
                check(qvp_host_free(slot.frames) == QVP_OK, "verify buffer");
                void* buf = nullptr;
                check(qvp_host_alloc(&buf, need) == QVP_OK, "verify buffer");
                slot.frames = static_cast<std::uint8_t*>(buf);
                slot.frames_cap = need;
            }
            if (!frame_ids.empty()) {
                check(qvp_swap_gather(alloc.device_base(), alloc.block_stride(), pool, frame_ids.data(), offsets.data(),
                                      static_cast<std::uint32_t>(frame_ids.size()), slot.frames, slot.frames_cap,
                                      check_bytes, stream) == QVP_OK,
                      std::string("verify gather: ") + qvp_last_error());
            }
            for (std::size_t k = 0; k < picks.size(); ++k) {
                check(qvp_memcpy_dtoh(slot.outs + k * kQRow, static_cast<const std::uint8_t*>(dout) + picks[k] * qrow_bytes,
                                      qrow_bytes, stream) == QVP_OK,
                      "verify output download");
            }
        }
        if (engine && !pos_seq.empty()) {
            begin_phase(kPositions);
            check(positions.materialise(cache, pos_seq, pos_begin, pos_end, static_cast<std::int64_t*>(dpos), stream),
                  "positions: " + positions.last_error());
            end_phase(kPositions);
        }
        check(qvp_event_record(slot.fin, stream) == QVP_OK, "record");
        slot.pending = true;
        slot.step = steps - 1;
        for (std::uint64_t id : ids) {
            sched.complete_step(id, 1);
            if (++produced[id] >= plans[id - 1].output) {
                sched.cancel(id);
                length.erase(id);
                produced.erase(id);
                ++finished;
                events += " done=" + std::to_string(id);
            }
        }
        if (!log_path.empty()) {
            Fnv h;
            for (std::uint32_t i = 1; i <= requests; ++i) {
                const auto view = cache.cache_view(i);
                if (!view) continue;
                h.add(i);
                for (const BlockTableEntry& e : view->block_table->entries()) {
                    h.add(e.physical_id);
                    h.add(e.swap_slot ? static_cast<std::uint32_t>(*e.swap_slot) : 0xFFFFFFFFu);
                    h.add(e.writable ? 1u : 0u);
                }
            }
            const AllocatorStats st = alloc.stats();
            std::string pre, dec;
            for (std::uint64_t id : plan.prefill_requests) pre += std::to_string(id) + ",";
            for (std::uint64_t id : plan.decode_requests) dec += std::to_string(id) + ",";
            char tail[160];
            std::snprintf(tail, sizeof tail, " tok=%u free=%u shared=%u swapped=%u h=%08x", plan.scheduled_tokens,
                          st.free_blocks, st.shared_blocks, st.swapped_blocks, h.h);
            log += std::to_string(steps - 1) + " P=" + pre + " D=" + dec + tail + events + "\n";
        }
    }
    for (StepEvents& r : ring) retire(r);
    check(alloc.synchronize(), "final sync");
    const double wall = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    const double append_gpu_ms = phase_ms[kAppend], prefill_gpu_ms = phase_ms[kPrefill];
    const double decode_gpu_ms = phase_ms[kDecode], mrope_gpu_ms = phase_ms[kPositions];
    const double swap_gpu_ms = alloc.swap_gpu_ms() - swap_ms_before;
    if (!log_path.empty()) {
        log += "finished=" + std::to_string(finished) + " of " + std::to_string(requests) + "\n";
        std::FILE* f = std::fopen(log_path.c_str(), "w");
        check(f != nullptr && std::fwrite(log.data(), 1, log.size(), f) == log.size() && std::fclose(f) == 0,
              "writing " + log_path);
    }
    if (dump != nullptr) check(std::fclose(dump) == 0, "closing the verify dump");
    const AllocatorStats st = alloc.stats();
    const bool drained = st.free_blocks == st.total_blocks && swap.resident_slots() == 0;
    const double swap_bytes = static_cast<double>(alloc.swap_bytes_moved() - swap_bytes_before);
    std::printf(
        "{\"mode\": \"config5_trace\", \"layers\": %u, \"requests\": %u, \"finished\": %llu, \"steps\": %llu, \"pool_blocks\": %u, "
        "\"demand_blocks\": %llu, \"decode_tokens\": %llu, \"expected_decode_tokens\": %llu, \"wall_s\": %.4f, "
        "\"decode_tokens_per_s\": %.1f, \"decode_kernel_ms_total\": %.3f, \"decode_tokens_per_s_kernel_only\": "
        "%.1f, \"preemptions\": %llu, \"resumes\": %llu, \"swapped_out_blocks\": %llu, \"swapped_in_blocks\": %llu, "
        "\"swap_bytes\": %.0f, \"swap_ms_total\": %.3f, \"swap_GBps\": %.2f, \"swap_launches\": %llu, "
        "\"drained\": %s, \"engine\": %s, \"steps_in_flight\": %d, \"prefill_tokens\": %llu, \"prefill_kernel_ms_total\": %.3f, "
        "\"prefill_tokens_per_s_kernel_only\": %.1f, \"append_ms_total\": %.3f, \"mrope_ms_total\": %.3f, "
        "\"verify\": %s, \"check_every\": %llu, \"sequence_checks\": %llu, \"resume_checks\": %llu, "
        "\"unchecked_resumes\": %zu, \"rows_checked\": %llu, \"row_mismatches\": %llu, \"decode_records\": %llu, "
        "\"first_mismatch\": \"%s\"}\n",
        layers, requests, static_cast<unsigned long long>(finished), static_cast<unsigned long long>(steps), pool,
        static_cast<unsigned long long>(demand_blocks), static_cast<unsigned long long>(decode_tokens),
        static_cast<unsigned long long>(total_output), wall, decode_tokens / wall, decode_gpu_ms,
        decode_tokens / (decode_gpu_ms * 1e-3), static_cast<unsigned long long>(preemptions),
        static_cast<unsigned long long>(resumes), static_cast<unsigned long long>(swapped_out_blocks),
        static_cast<unsigned long long>(swapped_in_blocks), swap_bytes, swap_gpu_ms,
        swap_gpu_ms > 0 ? swap_bytes / (swap_gpu_ms * 1e-3) / 1e9 : 0.0,
        static_cast<unsigned long long>(alloc.swap_launches() - swap_launch_before), drained ? "true" : "false",
        engine ? "true" : "false", in_flight, static_cast<unsigned long long>(prefill_tokens), prefill_gpu_ms,
        prefill_gpu_ms > 0 ? prefill_tokens / (prefill_gpu_ms * 1e-3) : 0.0, append_gpu_ms, mrope_gpu_ms,
        verify ? "true" : "false", static_cast<unsigned long long>(check_every),
        static_cast<unsigned long long>(seq_checks), static_cast<unsigned long long>(resume_checks),
        unchecked_resumes.size(), static_cast<unsigned long long>(rows_checked),
        static_cast<unsigned long long>(row_mismatches), static_cast<unsigned long long>(decode_records),
        first_mismatch.c_str());
    (void)qvp_free(dq);
    (void)qvp_free(dout);
    for (void* ptr : {dk, dv, dpq, dpo, dpos}) (void)qvp_free(ptr);
    for (StepEvents& r : ring) {
        for (void* e : r.ev) (void)qvp_event_destroy(e);
        (void)qvp_event_destroy(r.fin);
        for (void* h : {static_cast<void*>(r.rows_k), static_cast<void*>(r.rows_v), static_cast<void*>(r.frames),
                        static_cast<void*>(r.outs)}) {
            (void)qvp_host_free(h);
        }
    }
    return (finished == requests && drained && row_mismatches == 0) ? 0 : 2;
}

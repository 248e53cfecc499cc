// Contract of the continuous-batching scheduler over host-placed frames
// (include/qwenvl_paged/Scheduler.h of the reference; its suite
// tests/Scheduler.test.cpp:73-559 states the same policy: FIFO admission with a
// head-of-line stop, manual preemption by swap-out, all-or-nothing resume, and
// the watermark preemption of the newest pre-existing request).
#include "minitest.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/Scheduler.h"
#include "qwenvl_paged/SwapBackend.h"

#include <functional>
#include <map>

using namespace qwenvl_paged;

namespace {

AllocatorConfig pool_of(std::uint32_t blocks) {
    AllocatorConfig c;
    c.block_shape.tokens_per_block = 16;
    c.block_shape.num_layers = 2;
    c.block_shape.num_kv_heads = 2;
    c.block_shape.head_dim = 8;
    c.block_shape.bytes_per_element = 2;
    c.max_blocks = blocks;
    return c;
}

SchedulerConfig policy(std::uint32_t watermark = 0, std::uint32_t max_active = 8, std::uint32_t max_tokens = 4096) {
    SchedulerConfig c;
    c.max_active_requests = max_active;
    c.max_batch_tokens = max_tokens;
    c.preemption_watermark_blocks = watermark;
    return c;
}

Request req(RequestId id, std::uint32_t prompt = 32) {
    Request r;
    r.request_id = id;
    r.root_sequence_id = id;
    r.prompt_tokens = prompt;
    r.sampling.max_decode_tokens = 8;
    return r;
}

// A pool, an optional host swap store, the cache manager and the scheduler.
struct Engine {
    Engine(std::uint32_t blocks, SchedulerConfig cfg, bool with_swap = true)
        : alloc(pool_of(blocks)), swap(32), cache(alloc), sched(cfg, cache, alloc) {
        if (with_swap) alloc.set_swap_backend(&swap);
    }
    MemoryAllocator alloc;
    HostSwapBackend swap;
    KVCacheManager cache;
    Scheduler sched;
};

// Runs the request loop the reference's simulations use: resume parked work
// only when nothing waits, complete every planned step, retire a request after
// `decode_steps` decode steps; `on_blocked` may preempt when admission stalls.
struct DrainResult {
    std::size_t finished{0};
    bool saw_preempted{false};
};

DrainResult drain(Engine& e, const std::vector<std::uint32_t>& prompts, std::uint32_t decode_steps,
                  const std::function<void(Engine&, const std::vector<RequestId>&)>& on_blocked) {
    std::vector<RequestId> ids;
    for (std::size_t i = 0; i < prompts.size(); ++i) {
        ids.push_back(static_cast<RequestId>(i + 1));
        e.sched.enqueue(req(ids.back(), prompts[i]));
    }
    auto first_in = [&](RequestState s) -> std::optional<RequestId> {
        for (RequestId id : ids) {
            if (e.sched.state(id) == s) return id;
        }
        return std::nullopt;
    };
    DrainResult out;
    std::map<RequestId, std::uint32_t> steps;
    for (int step = 0; step < 200 && out.finished < prompts.size(); ++step) {
        if (!first_in(RequestState::Pending)) {
            if (auto p = first_in(RequestState::Preempted)) (void)e.sched.resume(*p);
        }
        const BatchPlan plan = e.sched.schedule_next();
        out.saw_preempted = out.saw_preempted || first_in(RequestState::Preempted).has_value();
        for (RequestId id : plan.prefill_requests) e.sched.complete_step(id, 1);
        for (RequestId id : plan.decode_requests) {
            e.sched.complete_step(id, 1);
            if (++steps[id] >= decode_steps) {
                e.sched.cancel(id);
                ++out.finished;
            }
        }
        if (plan.prefill_requests.empty() && first_in(RequestState::Pending) && on_blocked) on_blocked(e, ids);
    }
    return out;
}

}  // namespace

TEST(SchedulerTest, LifecycleOfOneRequest) {
    Engine e(64, policy());
    EXPECT_EQ(e.sched.active_size(), 0u);
    EXPECT_FALSE(e.sched.state(1).has_value());
    e.sched.enqueue(req(1));
    EXPECT_EQ(e.sched.state(1), RequestState::Pending);
    BatchPlan p = e.sched.schedule_next();
    ASSERT_EQ(p.prefill_requests.size(), 1u);
    EXPECT_EQ(p.prefill_requests[0], 1u);
    EXPECT_EQ(p.scheduled_tokens, 32u);
    EXPECT_TRUE(p.decode_requests.empty());
    EXPECT_EQ(e.sched.state(1), RequestState::Prefill);
    EXPECT_EQ(e.sched.active_size(), 1u);
    EXPECT_EQ(e.alloc.stats().free_blocks, 62u);
    e.sched.complete_step(1, 1);
    EXPECT_EQ(e.sched.state(1), RequestState::Decode);
    p = e.sched.schedule_next();
    EXPECT_TRUE(p.prefill_requests.empty());
    ASSERT_EQ(p.decode_requests.size(), 1u);
    EXPECT_EQ(p.scheduled_tokens, 1u);
    e.sched.cancel(1);
    EXPECT_EQ(e.sched.active_size(), 0u);
    EXPECT_FALSE(e.sched.state(1).has_value());
    EXPECT_EQ(e.alloc.stats().free_blocks, 64u);
}

TEST(SchedulerTest, AdmissionRespectsTheActiveAndTokenLimits) {
    Engine e(64, policy(0, 2, 100));
    for (RequestId id = 1; id <= 4; ++id) e.sched.enqueue(req(id, 40));
    BatchPlan p = e.sched.schedule_next();
    EXPECT_EQ(p.prefill_requests, (std::vector<RequestId>{1, 2}));
    EXPECT_EQ(p.scheduled_tokens, 80u);
    EXPECT_EQ(e.sched.state(3), RequestState::Pending);
    // Token budget: 40 + 40 + 40 > 100 stops at the head of the queue.
    Engine f(64, policy(0, 8, 100));
    for (RequestId id = 1; id <= 3; ++id) f.sched.enqueue(req(id, 40));
    EXPECT_EQ(f.sched.schedule_next().prefill_requests.size(), 2u);
    EXPECT_EQ(f.sched.state(3), RequestState::Pending);
}

TEST(SchedulerTest, PreemptAndResumeWithoutPressure) {
    Engine e(64, policy());
    e.sched.enqueue(req(1));
    (void)e.sched.schedule_next();
    EXPECT_FALSE(e.sched.preemption_info(1).has_value());
    EXPECT_FALSE(e.sched.preempt(99, "x"));
    EXPECT_TRUE(e.sched.preempt(1, "cache pressure"));
    EXPECT_EQ(e.sched.state(1), RequestState::Preempted);
    EXPECT_EQ(e.sched.active_size(), 0u);
    EXPECT_FALSE(e.sched.preempt(1, "again"));
    EXPECT_TRUE(e.sched.resume(1));
    EXPECT_EQ(e.sched.state(1), RequestState::Decode);
    EXPECT_EQ(e.sched.active_size(), 1u);
    EXPECT_FALSE(e.sched.resume(1));
    EXPECT_FALSE(e.sched.resume(99));
}

TEST(SchedulerTest, PendingRequestsCannotBePreemptedOrCompleted) {
    Engine e(64, policy());
    e.sched.enqueue(req(1));
    EXPECT_FALSE(e.sched.preempt(1, "x"));
    e.sched.complete_step(1, 1);
    EXPECT_EQ(e.sched.state(1), RequestState::Pending);
    e.sched.cancel(1);
    EXPECT_FALSE(e.sched.state(1).has_value());
    EXPECT_TRUE(e.sched.schedule_next().prefill_requests.empty());
}

TEST(SchedulerPressureTest, AHeadThatDoesNotFitLeavesNoState) {
    Engine e(4, policy());
    e.sched.enqueue(req(1, 64));
    e.sched.enqueue(req(2, 32));
    const BatchPlan p = e.sched.schedule_next();
    EXPECT_EQ(p.prefill_requests, (std::vector<RequestId>{1}));
    EXPECT_EQ(e.sched.state(2), RequestState::Pending);
    EXPECT_FALSE(e.cache.contains(2));
    EXPECT_EQ(e.sched.active_size(), 1u);
}

TEST(SchedulerPressureTest, PreemptionSwapsOutAndRecordsWhy) {
    Engine e(4, policy());
    e.sched.enqueue(req(1, 32));
    (void)e.sched.schedule_next();
    ASSERT_EQ(e.alloc.stats().free_blocks, 2u);
    ASSERT_TRUE(e.sched.preempt(1, "cache pressure"));
    EXPECT_EQ(e.alloc.stats().free_blocks, 4u);
    EXPECT_EQ(e.swap.resident_slots(), 2u);
    const auto info = e.sched.preemption_info(1);
    ASSERT_TRUE(info.has_value());
    EXPECT_EQ(info->reason, std::string("cache pressure"));
    EXPECT_EQ(info->swapped_blocks, 2u);
}

TEST(SchedulerPressureTest, PreemptingUnblocksTheQueue) {
    Engine e(4, policy());
    e.sched.enqueue(req(1, 64));
    e.sched.enqueue(req(2, 32));
    (void)e.sched.schedule_next();
    ASSERT_TRUE(e.sched.preempt(1, "cache pressure"));
    const BatchPlan p = e.sched.schedule_next();
    EXPECT_EQ(p.prefill_requests, (std::vector<RequestId>{2}));
    EXPECT_EQ(e.sched.state(2), RequestState::Prefill);
}

TEST(SchedulerPressureTest, ResumeRestoresEveryMapping) {
    Engine e(4, policy());
    e.sched.enqueue(req(1, 32));
    (void)e.sched.schedule_next();
    ASSERT_TRUE(e.sched.preempt(1, "cache pressure"));
    ASSERT_TRUE(e.sched.resume(1));
    EXPECT_EQ(e.swap.resident_slots(), 0u);
    EXPECT_FALSE(e.sched.preemption_info(1).has_value());
    const auto v = e.cache.cache_view(1);
    ASSERT_TRUE(v.has_value());
    EXPECT_EQ(v->block_table->size(), 2u);
    for (const BlockTableEntry& entry : v->block_table->entries()) {
        EXPECT_FALSE(entry.swap_slot.has_value());
        EXPECT_TRUE(v->block_table->lookup(entry.logical.index).has_value());
    }
}

TEST(SchedulerPressureTest, ResumeWaitsForFreeFrames) {
    Engine e(4, policy());
    e.sched.enqueue(req(1, 32));
    e.sched.enqueue(req(2, 64));
    (void)e.sched.schedule_next();
    ASSERT_TRUE(e.sched.preempt(1, "cache pressure"));
    (void)e.sched.schedule_next();
    ASSERT_EQ(e.sched.state(2), RequestState::Prefill);
    ASSERT_EQ(e.alloc.stats().free_blocks, 0u);
    EXPECT_FALSE(e.sched.resume(1));
    EXPECT_EQ(e.sched.state(1), RequestState::Preempted);
    EXPECT_EQ(e.swap.resident_slots(), 2u);
    EXPECT_TRUE(e.sched.preemption_info(1).has_value());
    e.sched.cancel(2);
    EXPECT_TRUE(e.sched.resume(1));
}

TEST(SchedulerPressureTest, CancelOfAParkedRequestDropsItsSlots) {
    Engine e(4, policy());
    e.sched.enqueue(req(1, 32));
    (void)e.sched.schedule_next();
    ASSERT_TRUE(e.sched.preempt(1, "cache pressure"));
    e.sched.cancel(1);
    EXPECT_FALSE(e.sched.state(1).has_value());
    EXPECT_FALSE(e.sched.preemption_info(1).has_value());
    EXPECT_EQ(e.swap.resident_slots(), 0u);
    EXPECT_EQ(e.alloc.stats().free_blocks, 4u);
}

TEST(SchedulerPressureTest, ManualPreemptionDrainsNineBlocksThroughFour) {
    Engine e(4, policy());
    const DrainResult r = drain(e, {16, 48, 32, 16, 64}, 2, [](Engine& eng, const std::vector<RequestId>& ids) {
        for (RequestId id : ids) {
            if (eng.sched.state(id) == RequestState::Decode) {
                EXPECT_TRUE(eng.sched.preempt(id, "cache pressure"));
                return;
            }
        }
    });
    EXPECT_EQ(r.finished, 5u);
    EXPECT_EQ(e.alloc.stats().free_blocks, 4u);
    EXPECT_EQ(e.alloc.stats().swapped_blocks, 0u);
    EXPECT_EQ(e.swap.resident_slots(), 0u);
}

TEST(SchedulerWatermarkTest, ZeroWatermarkNeverPreempts) {
    Engine e(4, policy(0));
    e.sched.enqueue(req(1, 64));
    ASSERT_EQ(e.sched.schedule_next().prefill_requests.size(), 1u);
    e.sched.enqueue(req(2, 32));
    EXPECT_TRUE(e.sched.schedule_next().prefill_requests.empty());
    EXPECT_EQ(e.sched.state(1), RequestState::Prefill);
    EXPECT_EQ(e.sched.state(2), RequestState::Pending);
    EXPECT_FALSE(e.sched.preemption_info(1).has_value());
}

TEST(SchedulerWatermarkTest, AdmissionEvictsToKeepTheReserve) {
    Engine e(4, policy(1));
    e.sched.enqueue(req(1, 32));
    ASSERT_EQ(e.sched.schedule_next().prefill_requests.size(), 1u);
    e.sched.enqueue(req(2, 32));  // 2 frames + 1 reserve > 2 free
    const BatchPlan p = e.sched.schedule_next();
    EXPECT_EQ(p.prefill_requests, (std::vector<RequestId>{2}));
    EXPECT_EQ(e.sched.state(1), RequestState::Preempted);
    const auto info = e.sched.preemption_info(1);
    ASSERT_TRUE(info.has_value());
    EXPECT_FALSE(info->reason.empty());
    EXPECT_EQ(info->swapped_blocks, 2u);
}

TEST(SchedulerWatermarkTest, TheNewestEarlierRequestIsTheVictim) {
    Engine e(4, policy(1));
    e.sched.enqueue(req(1, 16));
    (void)e.sched.schedule_next();
    e.sched.enqueue(req(2, 16));
    (void)e.sched.schedule_next();
    e.sched.enqueue(req(3, 32));
    ASSERT_EQ(e.sched.schedule_next().prefill_requests.size(), 1u);
    EXPECT_EQ(e.sched.state(1), RequestState::Prefill);
    EXPECT_EQ(e.sched.state(2), RequestState::Preempted);
    EXPECT_EQ(e.sched.state(3), RequestState::Prefill);
}

TEST(SchedulerWatermarkTest, RequestsAdmittedInTheSameStepAreNotVictims) {
    Engine e(6, policy(1));
    e.sched.enqueue(req(1, 32));  // 2 frames
    e.sched.enqueue(req(2, 32));  // 2 frames, 2 left; reserve of 1 holds
    e.sched.enqueue(req(3, 48));  // 3 frames of 2 free, but 1 and 2 are in this plan
    const BatchPlan p = e.sched.schedule_next();
    EXPECT_EQ(p.prefill_requests, (std::vector<RequestId>{1, 2}));
    EXPECT_EQ(e.sched.state(3), RequestState::Pending);
    EXPECT_EQ(e.sched.state(1), RequestState::Prefill);
    EXPECT_EQ(e.sched.state(2), RequestState::Prefill);
}

TEST(SchedulerWatermarkTest, ReserveHoldsAfterEachAdmission) {
    Engine e(4, policy(2));
    e.sched.enqueue(req(1, 32));
    ASSERT_EQ(e.sched.schedule_next().prefill_requests.size(), 1u);
    EXPECT_GE(e.alloc.stats().free_blocks, 2u);
    e.sched.enqueue(req(2, 16));
    ASSERT_EQ(e.sched.schedule_next().prefill_requests.size(), 1u);
    EXPECT_EQ(e.sched.state(1), RequestState::Preempted);
    EXPECT_GE(e.alloc.stats().free_blocks, 2u);
}

TEST(SchedulerWatermarkTest, AWholePoolPromptIsStillAdmitted) {
    Engine e(4, policy(2));
    e.sched.enqueue(req(1, 16));
    (void)e.sched.schedule_next();
    e.sched.enqueue(req(2, 64));
    const BatchPlan p = e.sched.schedule_next();
    EXPECT_EQ(p.prefill_requests, (std::vector<RequestId>{2}));
    EXPECT_EQ(e.sched.state(1), RequestState::Preempted);
    EXPECT_EQ(e.alloc.stats().free_blocks, 0u);
}

TEST(SchedulerWatermarkTest, APromptLargerThanThePoolEvictsNobody) {
    Engine e(4, policy(1));
    e.sched.enqueue(req(1, 16));
    (void)e.sched.schedule_next();
    e.sched.enqueue(req(2, 80));
    EXPECT_TRUE(e.sched.schedule_next().prefill_requests.empty());
    EXPECT_EQ(e.sched.state(1), RequestState::Prefill);
    EXPECT_EQ(e.sched.state(2), RequestState::Pending);
    EXPECT_FALSE(e.cache.contains(2));
}

TEST(SchedulerWatermarkTest, WithoutSwapSpaceOnePreemptionIsEnough) {
    Engine e(4, policy(1), /*with_swap=*/false);
    for (RequestId id = 1; id <= 3; ++id) {
        e.sched.enqueue(req(id, 16));
        ASSERT_EQ(e.sched.schedule_next().prefill_requests.size(), 1u);
    }
    e.sched.enqueue(req(4, 32));
    const BatchPlan p = e.sched.schedule_next();
    int parked = 0;
    for (RequestId id = 1; id <= 4; ++id) parked += e.sched.state(id) == RequestState::Preempted;
    EXPECT_EQ(parked, 1);
    EXPECT_TRUE(p.prefill_requests.empty());
    EXPECT_EQ(e.sched.state(4), RequestState::Pending);
    EXPECT_EQ(e.sched.preemption_info(3)->swapped_blocks, 0u);
}

TEST(SchedulerWatermarkTest, ThePolicyAloneDrainsNineBlocksThroughFour) {
    Engine e(4, policy(1));
    const DrainResult r = drain(e, {16, 48, 32, 16, 64}, 2, nullptr);
    EXPECT_TRUE(r.saw_preempted);
    EXPECT_EQ(r.finished, 5u);
    EXPECT_EQ(e.alloc.stats().free_blocks, 4u);
    EXPECT_EQ(e.alloc.stats().swapped_blocks, 0u);
    EXPECT_EQ(e.swap.resident_slots(), 0u);
}

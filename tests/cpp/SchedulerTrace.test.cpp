// The continuous-batching trace of oracle/trace_driver.h on this package's
// host API must reproduce, line for line, the event log the reference's own
// Scheduler / KVCacheManager / MemoryAllocator / HostSwapBackend wrote into
// tests/golden/scheduler_trace_*.txt: the same admissions, preemptions,
// resumes and completions, and the same frame and swap-slot ids (hashed per
// step).
#include "../../oracle/trace_driver.h"
#include "golden_path.h"
#include "minitest.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/Scheduler.h"
#include "qwenvl_paged/SwapBackend.h"

using namespace qwenvl_paged;

namespace {

// The settings tests/golden/make_golden.py gave the reference.
trace::Config trace_config(std::uint64_t seed, std::uint32_t pool_percent, std::uint32_t watermark) {
    trace::Config c;
    c.requests = 32;
    c.seed = seed;
    c.pool_percent = pool_percent;
    c.watermark_blocks = watermark;
    return c;
}

AllocatorConfig trace_pool(const trace::Config& c) {
    AllocatorConfig a;
    a.block_shape.tokens_per_block = c.tokens_per_block;
    a.block_shape.num_layers = 1;
    a.block_shape.num_kv_heads = 1;
    a.block_shape.head_dim = 8;
    a.block_shape.bytes_per_element = 4;
    a.max_blocks = trace::pool_blocks(c);
    return a;
}

void check_trace(const char* fixture, const trace::Config& c) {
    std::string expected;
    ASSERT_TRUE(golden::read(fixture, expected)) << "missing fixture " << golden::dir() << "/" << fixture;
    MemoryAllocator allocator(trace_pool(c));
    HostSwapBackend swap(1u << 20);
    allocator.set_swap_backend(&swap);
    const std::string log =
        trace::run<MemoryAllocator, KVCacheManager, Scheduler, SchedulerConfig, Request, RequestState>(c, allocator);
    EXPECT_TRUE(log == expected) << golden::first_difference(log, expected);
    EXPECT_NE(log.find("finished=32 of 32"), std::string::npos);
}

}  // namespace

TEST(SchedulerTraceTest, WatermarkTraceMatchesTheReference) {
    check_trace("scheduler_trace_w4.txt", trace_config(5, 30, 4));
}

TEST(SchedulerTraceTest, GrowthPreemptionTraceMatchesTheReference) {
    check_trace("scheduler_trace_w0.txt", trace_config(11, 30, 0));
}

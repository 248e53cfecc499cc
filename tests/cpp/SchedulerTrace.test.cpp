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
    const std::string name = fixture;
    const bool gz = name.size() > 3 && name.compare(name.size() - 3, 3, ".gz") == 0;
    ASSERT_TRUE(gz ? golden::read_gz(name, expected) : golden::read(name, expected))
        << "missing fixture " << golden::dir() << "/" << fixture;
    MemoryAllocator allocator(trace_pool(c));
    HostSwapBackend swap(1u << 20);
    allocator.set_swap_backend(&swap);
    const std::string log =
        trace::run<MemoryAllocator, KVCacheManager, Scheduler, SchedulerConfig, Request, RequestState>(c, allocator);
    EXPECT_TRUE(log == expected) << golden::first_difference(log, expected);
    const std::string all = "finished=" + std::to_string(c.requests) + " of " + std::to_string(c.requests);
    EXPECT_NE(log.find(all), std::string::npos);
}

}  // namespace

TEST(SchedulerTraceTest, WatermarkTraceMatchesTheReference) {
    check_trace("scheduler_trace_w4.txt", trace_config(5, 30, 4));
}

TEST(SchedulerTraceTest, GrowthPreemptionTraceMatchesTheReference) {
    check_trace("scheduler_trace_w0.txt", trace_config(11, 30, 0));
}

// The fifth benchmark configuration at full size (the settings of
// tests/golden/make_golden.py's CONFIG5_PARAMS): 200 requests at once, prompts
// [128, 8192], outputs [32, 1024], pool 60 % of demand, watermark 64 blocks,
// 256 active requests, 16384 scheduled tokens, cancels after the step's
// decodes.
TEST(SchedulerTraceTest, Config5TraceMatchesTheReference) {
    trace::Config c;
    c.requests = 200;
    c.prompt_lo = 128;
    c.prompt_hi = 8192;
    c.output_lo = 32;
    c.output_hi = 1024;
    c.arrivals_per_step = 200;
    c.tokens_per_block = 16;
    c.pool_percent = 60;
    c.watermark_blocks = 64;
    c.max_active = 256;
    c.max_batch_tokens = 16384;
    c.max_steps = 200000;
    c.cancel_after_decodes = true;
    c.seed = 5;
    check_trace("scheduler_trace_config5.txt.gz", c);
}

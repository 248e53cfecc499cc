// Engine loop on device frames: scheduler admission, K/V appends through the
// copy-on-write point, GPU decode per position, preemption with swap-out to
// the pinned arena and resume (the scenarios of tests/EndToEnd.test.cpp:184-351
// of the reference), plus a beam-style fork fan-out whose branches diverge.
#include "device_harness.h"

#include <map>

using namespace device_test;

namespace {

constexpr std::uint32_t kTpb = 4, kLayers = 2, kKvHeads = 2, kDim = 4, kHeads = 4;
constexpr float kScale = 0.5f;
constexpr float kTol = 1e-5f;

float token_value(SequenceId seq, std::uint32_t layer, KVStream s, std::uint32_t t, std::uint32_t h, std::uint32_t d) {
    return mix_pattern({std::uint32_t(seq), layer, s == KVStream::Key ? 0u : 1u, t, h, d});
}

class EngineTest : public testing::Test {
protected:
    EngineTest() : h_(shape_of(kTpb, kLayers, kKvHeads, kDim), 16, 16), sched_(config(), h_.cache, h_.allocator) {}

    static SchedulerConfig config() {
        SchedulerConfig c;
        c.max_active_requests = 4;
        c.max_batch_tokens = 64;
        return c;
    }

    // Token `pos` of `seq` as written by `writer` (the content owner; a forked
    // branch keeps its parent's tokens until it overwrites them).
    void append(SequenceId seq, TokenPosition pos, SequenceId writer) {
        ASSERT_TRUE(h_.ready());
        for (std::uint32_t layer = 0; layer < kLayers; ++layer) {
            for (KVStream st : {KVStream::Key, KVStream::Value}) {
                for (std::uint32_t kh = 0; kh < kKvHeads; ++kh) {
                    std::vector<float> v(kDim);
                    for (std::uint32_t d = 0; d < kDim; ++d) v[d] = token_value(writer, layer, st, pos, kh, d);
                    ASSERT_TRUE(write_head(h_, seq, st, layer, pos, kh, v)) << "seq " << seq << " pos " << pos;
                }
            }
        }
        owner_[seq].resize(std::max<std::size_t>(owner_[seq].size(), pos + 1));
        owner_[seq][pos] = writer;
    }

    void grow_to(SequenceId seq, TokenPosition pos) {
        if (pos / kTpb >= h_.cache.cache_view(seq)->block_table->size()) {
            ASSERT_TRUE(h_.cache.reserve_tokens(seq, 1));
        }
    }

    std::vector<float> query_for(SequenceId seq, TokenPosition pos) const {
        std::vector<float> q(kHeads * kDim);
        for (std::uint32_t i = 0; i < q.size(); ++i) q[i] = mix_pattern({std::uint32_t(seq), 9u, pos, i});
        return q;
    }

    void check(SequenceId seq, TokenPosition pos) {
        const auto view = h_.cache.cache_view(seq);
        ASSERT_TRUE(view.has_value());
        const auto q = query_for(seq, pos);
        const std::vector<SequenceId>& own = owner_[seq];
        for (std::uint32_t layer = 0; layer < kLayers; ++layer) {
            PagedAttentionParams p;
            p.layer = layer;
            p.num_query_heads = kHeads;
            p.context_len = pos + 1;
            p.scale = kScale;
            std::vector<float> out(q.size());
            ASSERT_TRUE(paged_attention_decode<float>(*view, q.data(), p, out.data()))
                << "seq " << seq << " pos " << pos << ": " << paged_attention_last_error();
            const auto expect = textbook_attention(
                q, kHeads, kKvHeads, kDim, pos + 1, kScale,
                [&](auto t, auto kh, auto d) { return token_value(own[t], layer, KVStream::Key, t, kh, d); },
                [&](auto t, auto kh, auto d) { return token_value(own[t], layer, KVStream::Value, t, kh, d); });
            for (std::size_t i = 0; i < out.size(); ++i) {
                ASSERT_NEAR(out[i], expect[i], kTol) << "seq " << seq << " pos " << pos << " layer " << layer;
            }
        }
    }

    DeviceHarness h_;
    Scheduler sched_;
    std::map<SequenceId, std::vector<SequenceId>> owner_;
};

Request make_request(RequestId id, std::uint32_t prompt) {
    Request r;
    r.request_id = id;
    r.root_sequence_id = id;
    r.prompt_tokens = prompt;
    r.sampling.max_decode_tokens = 3;
    return r;
}

}  // namespace

TEST_F(EngineTest, PrefillThenDecodeForThreeRequests) {
    ASSERT_TRUE(h_.ready());
    for (RequestId id = 1; id <= 3; ++id) sched_.enqueue(make_request(id, 6));
    const BatchPlan prefill = sched_.schedule_next();
    ASSERT_EQ(prefill.prefill_requests.size(), 3u);
    EXPECT_EQ(prefill.scheduled_tokens, 18u);
    for (RequestId id : prefill.prefill_requests) {
        for (TokenPosition p = 0; p < 6; ++p) ASSERT_NO_FATAL_FAILURE(append(id, p, id));
        // Causal prefill = decode at every prompt position with a growing context.
        for (TokenPosition p = 0; p < 6; ++p) ASSERT_NO_FATAL_FAILURE(check(id, p));
        sched_.complete_step(id, 1);
    }
    for (std::uint32_t step = 0; step < 3; ++step) {
        const BatchPlan plan = sched_.schedule_next();
        ASSERT_EQ(plan.decode_requests.size(), 3u);
        const TokenPosition pos = 6 + step;
        for (RequestId id : plan.decode_requests) {
            ASSERT_NO_FATAL_FAILURE(grow_to(id, pos));
            ASSERT_NO_FATAL_FAILURE(append(id, pos, id));
            ASSERT_NO_FATAL_FAILURE(check(id, pos));
            sched_.complete_step(id, 1);
        }
    }
    bool any_scattered = false;
    for (RequestId id = 1; id <= 3; ++id) any_scattered = any_scattered || scattered(*h_.cache.cache_view(id)->block_table);
    EXPECT_TRUE(any_scattered);
    for (RequestId id = 1; id <= 3; ++id) sched_.cancel(id);
    const AllocatorStats s = h_.allocator.stats();
    EXPECT_EQ(s.free_blocks, s.total_blocks);
    EXPECT_EQ(s.swapped_blocks, 0u);
}

TEST_F(EngineTest, PreemptedRequestResumesWithItsCache) {
    ASSERT_TRUE(h_.ready());
    sched_.enqueue(make_request(1, 6));
    ASSERT_EQ(sched_.schedule_next().prefill_requests.size(), 1u);
    for (TokenPosition p = 0; p < 6; ++p) ASSERT_NO_FATAL_FAILURE(append(1, p, 1));
    sched_.complete_step(1, 1);
    ASSERT_NO_FATAL_FAILURE(check(1, 5));
    ASSERT_TRUE(sched_.preempt(1, "cache pressure"));
    EXPECT_EQ(sched_.preemption_info(1)->swapped_blocks, 2u);
    // While out, the frames belong to whoever takes them: fill them all.
    sched_.enqueue(make_request(2, 64));
    ASSERT_EQ(sched_.schedule_next().prefill_requests.size(), 1u);
    for (TokenPosition p = 0; p < 64; ++p) ASSERT_NO_FATAL_FAILURE(append(2, p, 2));
    {
        const auto q = query_for(1, 5);
        std::vector<float> out(q.size(), -1.0f);
        PagedAttentionParams p;
        p.num_query_heads = kHeads;
        p.context_len = 6;
        p.scale = kScale;
        EXPECT_FALSE(paged_attention_decode<float>(*h_.cache.cache_view(1), q.data(), p, out.data()));
        EXPECT_EQ(out[0], -1.0f);
    }
    EXPECT_FALSE(sched_.resume(1));  // no free frame yet
    sched_.cancel(2);
    ASSERT_TRUE(sched_.resume(1));
    ASSERT_NO_FATAL_FAILURE(check(1, 5));
    ASSERT_NO_FATAL_FAILURE(grow_to(1, 6));
    ASSERT_NO_FATAL_FAILURE(append(1, 6, 1));
    ASSERT_NO_FATAL_FAILURE(check(1, 6));
    sched_.cancel(1);
    EXPECT_EQ(h_.allocator.stats().free_blocks, 16u);
    EXPECT_EQ(h_.swap.resident_slots(), 0u);
}

TEST_F(EngineTest, ForkedBeamsShareThePrefixAndDiverge) {
    ASSERT_TRUE(h_.ready());
    ASSERT_TRUE(h_.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(h_.cache.reserve_tokens(1, 6));
    for (TokenPosition p = 0; p < 6; ++p) ASSERT_NO_FATAL_FAILURE(append(1, p, 1));
    for (SequenceId b = 2; b <= 4; ++b) {
        ASSERT_TRUE(h_.cache.fork_sequence(1, SequenceMetadata{b, 1, {}, {}}));
        owner_[b] = owner_[1];
    }
    // Each beam rewrites token 5 (inside the shared second block, so the block
    // is copied first), then appends token 6 to its now private copy.
    for (SequenceId b = 2; b <= 4; ++b) {
        ASSERT_NO_FATAL_FAILURE(append(b, 5, b));
        ASSERT_NO_FATAL_FAILURE(grow_to(b, 6));
        ASSERT_NO_FATAL_FAILURE(append(b, 6, b));
    }
    for (SequenceId s = 1; s <= 4; ++s) ASSERT_NO_FATAL_FAILURE(check(s, s == 1 ? 5 : 6));
    // The first block is still one frame for all four sequences.
    const PhysicalBlockId shared = *h_.cache.cache_view(1)->block_table->lookup(0);
    for (SequenceId b = 2; b <= 4; ++b) EXPECT_EQ(*h_.cache.cache_view(b)->block_table->lookup(0), shared);
    EXPECT_EQ(h_.allocator.info(shared)->ref_count, 4u);
}

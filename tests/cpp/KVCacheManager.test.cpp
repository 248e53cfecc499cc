// Contract of the sequence cache lifecycle over host-placed frames
// (include/qwenvl_paged/KVCacheManager.h of the reference; its suite
// tests/KVCacheManager.test.cpp:42-379 states the same rules).
#include "minitest.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/SwapBackend.h"

using namespace qwenvl_paged;

namespace {

constexpr std::uint32_t kTpb = 16;

AllocatorConfig pool_of(std::uint32_t blocks) {
    AllocatorConfig c;
    c.block_shape.tokens_per_block = kTpb;
    c.block_shape.num_layers = 2;
    c.block_shape.num_kv_heads = 2;
    c.block_shape.head_dim = 8;
    c.block_shape.bytes_per_element = 2;
    c.max_blocks = blocks;
    return c;
}

SequenceMetadata seq(SequenceId id, RequestId request = 1) {
    SequenceMetadata m;
    m.sequence_id = id;
    m.request_id = request;
    return m;
}

void paint(PhysicalBlock& b, unsigned seed) {
    for (std::size_t i = 0; i < b.size_bytes(); ++i) b.data()[i] = static_cast<std::byte>((i ^ seed) * 7 % 251);
}

bool painted(const PhysicalBlock& b, unsigned seed) {
    for (std::size_t i = 0; i < b.size_bytes(); ++i) {
        if (b.data()[i] != static_cast<std::byte>((i ^ seed) * 7 % 251)) return false;
    }
    return true;
}

PhysicalBlockId frame_of(const KVCacheManager& m, SequenceId s, LogicalBlockIndex i) {
    const auto v = m.cache_view(s);
    const auto f = v ? v->block_table->lookup(i) : std::nullopt;
    return f ? *f : 0xFFFFFFFFu;
}

class KVCacheManagerTest : public testing::Test {
protected:
    explicit KVCacheManagerTest(std::uint32_t blocks = 32) : alloc_(pool_of(blocks)), cache_(alloc_) {}
    MemoryAllocator alloc_;
    KVCacheManager cache_;
};

class KVCacheSwapTest : public testing::Test {
protected:
    KVCacheSwapTest() : alloc_(pool_of(4)), swap_(8), cache_(alloc_) { alloc_.set_swap_backend(&swap_); }
    MemoryAllocator alloc_;
    HostSwapBackend swap_;
    KVCacheManager cache_;
};

}  // namespace

TEST_F(KVCacheManagerTest, SequencesAreCreatedOnce) {
    EXPECT_FALSE(cache_.contains(1));
    EXPECT_TRUE(cache_.create_sequence(seq(1)));
    EXPECT_TRUE(cache_.contains(1));
    EXPECT_FALSE(cache_.create_sequence(seq(1, 7)));
    EXPECT_EQ(cache_.metadata(1)->request_id, 1u);
    EXPECT_EQ(cache_.metadata(2), nullptr);
}

TEST_F(KVCacheManagerTest, NewSequenceHasAnEmptyTextView) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    const auto v = cache_.cache_view(1);
    ASSERT_TRUE(v.has_value());
    EXPECT_EQ(v->sequence_id, 1u);
    EXPECT_EQ(v->cache_kind, CacheKind::TextKV);
    ASSERT_NE(v->block_table, nullptr);
    EXPECT_TRUE(v->block_table->empty());
    EXPECT_FALSE(cache_.cache_view(99).has_value());
}

TEST_F(KVCacheManagerTest, ReserveMapsWholeBlocksAfterTheExistingOnes) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb + 1));  // 2 blocks
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));      // 1 more
    const auto v = cache_.cache_view(1);
    ASSERT_EQ(v->block_table->size(), 3u);
    LogicalBlockIndex expect = 0;
    for (const BlockTableEntry& e : v->block_table->entries()) {
        EXPECT_EQ(e.logical.index, expect);
        EXPECT_EQ(e.logical.start_token, expect * kTpb);
        EXPECT_EQ(e.logical.token_count, kTpb);
        EXPECT_EQ(e.logical.sequence_id, 1u);
        EXPECT_TRUE(e.writable);
        ++expect;
    }
    // Frames come off the LIFO free list: 31, 30, 29.
    EXPECT_EQ(frame_of(cache_, 1, 0), 31u);
    EXPECT_EQ(frame_of(cache_, 1, 2), 29u);
    EXPECT_TRUE(cache_.reserve_tokens(1, 0));
    EXPECT_EQ(cache_.cache_view(1)->block_table->size(), 3u);
}

TEST_F(KVCacheManagerTest, ReserveIsRefusedWholeWhenThePoolIsShort) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    EXPECT_FALSE(cache_.reserve_tokens(99, kTpb));
    EXPECT_FALSE(cache_.reserve_tokens(1, 33 * kTpb));
    EXPECT_EQ(alloc_.stats().free_blocks, 32u);
    EXPECT_TRUE(cache_.cache_view(1)->block_table->empty());
}

TEST_F(KVCacheManagerTest, ReleaseReturnsEveryFrame) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, 2 * kTpb));
    EXPECT_EQ(alloc_.stats().free_blocks, 30u);
    cache_.release_sequence(1);
    EXPECT_FALSE(cache_.contains(1));
    EXPECT_EQ(alloc_.stats().free_blocks, 32u);
    cache_.release_sequence(1);  // unknown now: no effect
    EXPECT_EQ(alloc_.stats().free_blocks, 32u);
}

TEST_F(KVCacheManagerTest, ForkSharesFramesAndCountsReferences) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, 2 * kTpb));
    ASSERT_TRUE(cache_.fork_sequence(1, seq(2)));
    ASSERT_TRUE(cache_.fork_sequence(1, seq(3)));
    EXPECT_FALSE(cache_.fork_sequence(99, seq(4)));
    EXPECT_FALSE(cache_.fork_sequence(1, seq(2)));  // child id taken
    for (LogicalBlockIndex i = 0; i < 2; ++i) {
        const PhysicalBlockId f = frame_of(cache_, 1, i);
        EXPECT_EQ(frame_of(cache_, 2, i), f);
        EXPECT_EQ(frame_of(cache_, 3, i), f);
        EXPECT_EQ(alloc_.info(f)->ref_count, 3u);
        EXPECT_EQ(alloc_.info(f)->state, BlockState::Shared);
        EXPECT_FALSE(cache_.cache_view(2)->block_table->entry(i)->writable);
    }
    // Releasing the parent leaves the children's frames alive.
    cache_.release_sequence(1);
    EXPECT_EQ(alloc_.info(frame_of(cache_, 2, 0))->ref_count, 2u);
    EXPECT_EQ(alloc_.stats().free_blocks, 30u);
}

TEST_F(KVCacheManagerTest, WritingASharedBlockCopiesItFirst) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, 2 * kTpb));
    paint(*alloc_.block(frame_of(cache_, 1, 1)), 42);
    ASSERT_TRUE(cache_.fork_sequence(1, seq(2)));
    const PhysicalBlockId shared = frame_of(cache_, 1, 1);
    const auto mine = cache_.ensure_token_writable(2, kTpb + 3);
    ASSERT_TRUE(mine.has_value());
    EXPECT_NE(*mine, shared);
    EXPECT_EQ(frame_of(cache_, 2, 1), *mine);
    EXPECT_EQ(frame_of(cache_, 1, 1), shared);
    EXPECT_TRUE(painted(*alloc_.block(*mine), 42));
    EXPECT_EQ(alloc_.info(shared)->ref_count, 1u);
    EXPECT_TRUE(cache_.cache_view(2)->block_table->entry(1)->writable);
    // Block 0 is still shared; a second write to block 1 is now in place.
    EXPECT_EQ(frame_of(cache_, 2, 0), frame_of(cache_, 1, 0));
    const std::uint32_t free_now = alloc_.stats().free_blocks;
    EXPECT_EQ(cache_.ensure_token_writable(2, kTpb), mine);
    EXPECT_EQ(alloc_.stats().free_blocks, free_now);
    // The parent is now the sole owner of its block 1: in place too, and its
    // read-only flag (had it one) would be lifted.
    EXPECT_EQ(cache_.ensure_token_writable(1, kTpb), shared);
}

TEST_F(KVCacheManagerTest, SoleOwnerWritesInPlace) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));
    const PhysicalBlockId owned = frame_of(cache_, 1, 0);
    const std::uint32_t free_before = alloc_.stats().free_blocks;
    EXPECT_EQ(cache_.ensure_token_writable(1, 5), owned);
    EXPECT_EQ(alloc_.stats().free_blocks, free_before);
}

TEST_F(KVCacheManagerTest, WritesOutsideTheReservationAreRefused) {
    EXPECT_FALSE(cache_.ensure_token_writable(99, 0).has_value());
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    EXPECT_FALSE(cache_.ensure_token_writable(1, 0).has_value());  // nothing reserved
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));
    EXPECT_FALSE(cache_.ensure_token_writable(1, kTpb).has_value());
}

TEST_F(KVCacheManagerTest, CopyOnWriteFailsCleanlyWhenThePoolIsFull) {
    MemoryAllocator small(pool_of(1));
    KVCacheManager m(small);
    ASSERT_TRUE(m.create_sequence(seq(1)));
    ASSERT_TRUE(m.reserve_tokens(1, kTpb));
    ASSERT_TRUE(m.fork_sequence(1, seq(2)));
    EXPECT_FALSE(m.ensure_token_writable(2, 0).has_value());
    EXPECT_EQ(frame_of(m, 2, 0), frame_of(m, 1, 0));
    EXPECT_EQ(small.info(frame_of(m, 1, 0))->ref_count, 2u);
}

TEST_F(KVCacheSwapTest, SwapOutFreesFramesAndKeepsTheMapping) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, 2 * kTpb));
    ASSERT_EQ(alloc_.stats().free_blocks, 2u);
    EXPECT_EQ(cache_.swap_out_sequence(1), 2u);
    EXPECT_EQ(alloc_.stats().free_blocks, 4u);
    EXPECT_EQ(swap_.resident_slots(), 2u);
    const auto v = cache_.cache_view(1);
    EXPECT_EQ(v->block_table->size(), 2u);
    for (const BlockTableEntry& e : v->block_table->entries()) {
        EXPECT_TRUE(e.swap_slot.has_value());
        EXPECT_FALSE(v->block_table->lookup(e.logical.index).has_value());
    }
    // Already out: nothing more to swap; a write cannot land anywhere.
    EXPECT_EQ(cache_.swap_out_sequence(1), 0u);
    EXPECT_FALSE(cache_.ensure_token_writable(1, 0).has_value());
    EXPECT_EQ(cache_.swap_out_sequence(99), 0u);
}

TEST_F(KVCacheManagerTest, SwapOutWithoutABackendKeepsEverything) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));
    EXPECT_EQ(cache_.swap_out_sequence(1), 0u);
    EXPECT_TRUE(cache_.cache_view(1)->block_table->lookup(0).has_value());
}

TEST_F(KVCacheSwapTest, SharedFramesStayResident) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, 2 * kTpb));
    ASSERT_TRUE(cache_.fork_sequence(1, seq(2)));
    ASSERT_TRUE(cache_.ensure_token_writable(1, kTpb).has_value());  // block 1 private again
    EXPECT_EQ(cache_.swap_out_sequence(1), 1u);
    const auto v = cache_.cache_view(1);
    EXPECT_TRUE(v->block_table->lookup(0).has_value());
    EXPECT_FALSE(v->block_table->lookup(1).has_value());
    EXPECT_TRUE(cache_.cache_view(2)->block_table->lookup(0).has_value());
    EXPECT_TRUE(cache_.cache_view(2)->block_table->lookup(1).has_value());
}

TEST(KVCacheSwapSingleFrameTest, SwapInRestoresBytesIntoAReusedFrame) {
    MemoryAllocator alloc(pool_of(1));
    HostSwapBackend swap(4);
    alloc.set_swap_backend(&swap);
    KVCacheManager cache(alloc);
    ASSERT_TRUE(cache.create_sequence(seq(1)));
    ASSERT_TRUE(cache.reserve_tokens(1, kTpb));
    const PhysicalBlockId f = frame_of(cache, 1, 0);
    paint(*alloc.block(f), 21);
    ASSERT_EQ(cache.swap_out_sequence(1), 1u);
    const auto other = alloc.allocate();
    ASSERT_TRUE(other.has_value());
    paint(*alloc.block(*other), 130);
    alloc.release(*other);
    EXPECT_TRUE(cache.swap_in_sequence(1));
    const PhysicalBlockId back = frame_of(cache, 1, 0);
    EXPECT_FALSE(cache.cache_view(1)->block_table->entry(0)->swap_slot.has_value());
    EXPECT_EQ(swap.resident_slots(), 0u);
    EXPECT_TRUE(painted(*alloc.block(back), 21));
}

TEST_F(KVCacheSwapTest, SwapInIsAllOrNothing) {
    MemoryAllocator alloc(pool_of(2));
    HostSwapBackend swap(8);
    alloc.set_swap_backend(&swap);
    KVCacheManager cache(alloc);
    ASSERT_TRUE(cache.create_sequence(seq(1)));
    ASSERT_TRUE(cache.reserve_tokens(1, 2 * kTpb));
    ASSERT_EQ(cache.swap_out_sequence(1), 2u);
    ASSERT_TRUE(alloc.allocate().has_value());
    EXPECT_FALSE(cache.swap_in_sequence(1));
    EXPECT_EQ(alloc.stats().free_blocks, 1u);
    EXPECT_EQ(swap.resident_slots(), 2u);
    for (const BlockTableEntry& e : cache.cache_view(1)->block_table->entries()) {
        EXPECT_TRUE(e.swap_slot.has_value());
    }
    EXPECT_FALSE(cache.swap_in_sequence(99));
}

TEST_F(KVCacheSwapTest, SwapInOfAResidentSequenceDoesNothing) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));
    const std::uint32_t free_before = alloc_.stats().free_blocks;
    EXPECT_TRUE(cache_.swap_in_sequence(1));
    EXPECT_EQ(alloc_.stats().free_blocks, free_before);
}

TEST_F(KVCacheSwapTest, ReleaseDropsSwappedSlots) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, 2 * kTpb));
    ASSERT_EQ(cache_.swap_out_sequence(1), 2u);
    cache_.release_sequence(1);
    EXPECT_FALSE(cache_.contains(1));
    EXPECT_EQ(swap_.resident_slots(), 0u);
    EXPECT_EQ(alloc_.stats().free_blocks, 4u);
    EXPECT_EQ(alloc_.stats().swapped_blocks, 0u);
}

TEST_F(KVCacheSwapTest, ASwappedParentCannotBeForked) {
    ASSERT_TRUE(cache_.create_sequence(seq(1)));
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));
    ASSERT_EQ(cache_.swap_out_sequence(1), 1u);
    EXPECT_FALSE(cache_.fork_sequence(1, seq(2)));
    EXPECT_FALSE(cache_.contains(2));
    ASSERT_TRUE(cache_.swap_in_sequence(1));
    EXPECT_TRUE(cache_.fork_sequence(1, seq(2)));
}

// Contract of the per-sequence page table (include/qwenvl_paged/BlockTable.h
// of the reference; tests/BlockTable.test.cpp:31-196 states the same rules).
// entries() order is what the ragged-batch packer flattens, so it is checked
// against a sorted model under random insertion orders too.
#include "minitest.h"
#include "qwenvl_paged/BlockTable.h"

#include <algorithm>
#include <map>
#include <random>

using namespace qwenvl_paged;

namespace {

LogicalBlock logical(SequenceId seq, LogicalBlockIndex index, std::uint32_t tpb = 16) {
    LogicalBlock l;
    l.sequence_id = seq;
    l.index = index;
    l.start_token = index * tpb;
    l.token_count = tpb;
    return l;
}

}  // namespace

TEST(BlockTableTest, FreshTableIsEmptyAndKeepsItsIdentity) {
    BlockTable t(42, CacheKind::VisionKV);
    EXPECT_EQ(t.sequence_id(), 42u);
    EXPECT_EQ(t.cache_kind(), CacheKind::VisionKV);
    EXPECT_TRUE(t.empty());
    EXPECT_EQ(t.size(), 0u);
    EXPECT_EQ(BlockTable(1).cache_kind(), CacheKind::TextKV);
}

TEST(BlockTableTest, MapLookupAndReplace) {
    BlockTable t(1);
    t.map(logical(1, 0), 100, true);
    ASSERT_TRUE(t.lookup(0).has_value());
    EXPECT_EQ(*t.lookup(0), 100u);
    t.map(logical(1, 0), 200, false);
    EXPECT_EQ(t.size(), 1u);
    EXPECT_EQ(*t.lookup(0), 200u);
    EXPECT_FALSE(t.entry(0)->writable);
    EXPECT_FALSE(t.lookup(1).has_value());
    EXPECT_EQ(t.entry(1), nullptr);
    EXPECT_EQ(t.mutable_entry(1), nullptr);
}

TEST(BlockTableTest, UnmapReturnsTheFrameOnce) {
    BlockTable t(1);
    t.map(logical(1, 3), 7, true);
    const auto first = t.unmap(3);
    ASSERT_TRUE(first.has_value());
    EXPECT_EQ(*first, 7u);
    EXPECT_FALSE(t.unmap(3).has_value());
    EXPECT_TRUE(t.empty());
}

TEST(BlockTableTest, WritableFlagAndInPlaceEdits) {
    BlockTable t(1);
    t.map(logical(1, 0), 100, false);
    t.set_writable(0, true);
    EXPECT_TRUE(t.entry(0)->writable);
    t.set_writable(9, true);  // unmapped: no effect, no entry created
    EXPECT_EQ(t.size(), 1u);
    t.mutable_entry(0)->physical_id = 555;
    EXPECT_EQ(*t.lookup(0), 555u);
}

TEST(BlockTableTest, EntriesAreSortedWhateverTheInsertionOrder) {
    std::mt19937 rng(1234);
    for (int trial = 0; trial < 20; ++trial) {
        std::vector<LogicalBlockIndex> order(64);
        for (std::size_t i = 0; i < order.size(); ++i) order[i] = static_cast<LogicalBlockIndex>(i * 3);
        std::shuffle(order.begin(), order.end(), rng);
        BlockTable t(5);
        std::map<LogicalBlockIndex, PhysicalBlockId> model;
        for (LogicalBlockIndex idx : order) {
            const PhysicalBlockId frame = static_cast<PhysicalBlockId>(rng() % 100000);
            t.map(logical(5, idx), frame, true);
            model[idx] = frame;
        }
        // Remove a third of them again.
        for (std::size_t i = 0; i < order.size(); i += 3) {
            EXPECT_EQ(*t.unmap(order[i]), model[order[i]]);
            model.erase(order[i]);
        }
        ASSERT_EQ(t.size(), model.size());
        auto it = model.begin();
        for (const BlockTableEntry& e : t.entries()) {
            EXPECT_EQ(e.logical.index, it->first);
            EXPECT_EQ(e.physical_id, it->second);
            ++it;
        }
    }
}

TEST(BlockTableTest, SwappedEntryStaysButDoesNotResolve) {
    BlockTable t(1);
    t.map(logical(1, 0), 100, true);
    EXPECT_FALSE(t.entry(0)->swap_slot.has_value());
    t.mutable_entry(0)->swap_slot = SwapSlotId{7};
    EXPECT_FALSE(t.lookup(0).has_value());
    ASSERT_NE(t.entry(0), nullptr);
    EXPECT_EQ(*t.entry(0)->swap_slot, SwapSlotId{7});
    EXPECT_EQ(t.size(), 1u);
    // Restored into another frame: resolves again.
    t.mutable_entry(0)->physical_id = 200;
    t.mutable_entry(0)->swap_slot.reset();
    EXPECT_EQ(*t.lookup(0), 200u);
}

TEST(BlockTableTest, RemappingClearsTheSwapSlot) {
    BlockTable t(1);
    t.map(logical(1, 0), 100, true);
    t.mutable_entry(0)->swap_slot = SwapSlotId{3};
    t.map(logical(1, 0), 101, true);
    EXPECT_FALSE(t.entry(0)->swap_slot.has_value());
    EXPECT_EQ(*t.lookup(0), 101u);
}

TEST(BlockTableTest, ForkSharesFramesReadOnly) {
    BlockTable parent(1);
    for (LogicalBlockIndex i = 0; i < 4; ++i) parent.map(logical(1, i), 100 + i, true);
    const BlockTable child = parent.fork(2);
    EXPECT_EQ(child.sequence_id(), 2u);
    ASSERT_EQ(child.size(), parent.size());
    for (LogicalBlockIndex i = 0; i < 4; ++i) {
        EXPECT_EQ(child.lookup(i), parent.lookup(i));
        EXPECT_FALSE(child.entry(i)->writable);
        EXPECT_EQ(child.entry(i)->logical.sequence_id, 2u);
        // The parent keeps its flags.
        EXPECT_TRUE(parent.entry(i)->writable);
    }
}

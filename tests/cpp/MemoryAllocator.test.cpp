// Contract of the physical block pool with host-placed frames
// (include/qwenvl_paged/MemoryAllocator.h of the reference; its suite
// tests/MemoryAllocator.test.cpp:38-425 states the same rules). The copy-on-write
// copy, commented out there, is checked here byte for byte.
#include "minitest.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/SwapBackend.h"

#include <algorithm>
#include <set>

using namespace qwenvl_paged;

namespace {

AllocatorConfig config_with(std::uint32_t blocks) {
    AllocatorConfig c;
    c.block_shape.tokens_per_block = 16;
    c.block_shape.num_layers = 2;
    c.block_shape.num_kv_heads = 2;
    c.block_shape.head_dim = 8;
    c.block_shape.bytes_per_element = 4;
    c.max_blocks = blocks;
    return c;
}

std::byte pattern_byte(std::size_t i, unsigned seed) { return static_cast<std::byte>((i * 13 + seed) % 253); }

void paint(PhysicalBlock& b, unsigned seed) {
    for (std::size_t i = 0; i < b.size_bytes(); ++i) b.data()[i] = pattern_byte(i, seed);
}

bool painted(const PhysicalBlock& b, unsigned seed) {
    for (std::size_t i = 0; i < b.size_bytes(); ++i) {
        if (b.data()[i] != pattern_byte(i, seed)) return false;
    }
    return true;
}

}  // namespace

TEST(MemoryAllocatorTest, FreshPoolIsAllFree) {
    MemoryAllocator a(config_with(4));
    const AllocatorStats s = a.stats();
    EXPECT_EQ(s.total_blocks, 4u);
    EXPECT_EQ(s.free_blocks, 4u);
    EXPECT_EQ(s.active_blocks, 0u);
    EXPECT_EQ(s.shared_blocks, 0u);
    EXPECT_EQ(s.swapped_blocks, 0u);
    EXPECT_EQ(s.bytes_reserved, 4u * a.block(0)->size_bytes());
    EXPECT_EQ(a.placement(), BlockPlacement::Host);
    EXPECT_TRUE(a.ok());
}

TEST(MemoryAllocatorTest, HandsOutEveryFrameOnceHighestIdFirst) {
    MemoryAllocator a(config_with(5));
    std::vector<PhysicalBlockId> got;
    while (auto id = a.allocate()) got.push_back(*id);
    // LIFO over a free list initialised 0..N-1: N-1 comes out first.
    EXPECT_EQ(got, (std::vector<PhysicalBlockId>{4, 3, 2, 1, 0}));
    EXPECT_FALSE(a.allocate().has_value());
    EXPECT_EQ(a.stats().free_blocks, 0u);
}

TEST(MemoryAllocatorTest, ReleasedFrameIsTheNextOneHandedOut) {
    MemoryAllocator a(config_with(3));
    const auto x = a.allocate();
    const auto y = a.allocate();
    ASSERT_TRUE(x && y);
    a.release(*x);
    EXPECT_EQ(*a.allocate(), *x);
    a.release(*y);
    EXPECT_EQ(*a.allocate(), *y);
}

TEST(MemoryAllocatorTest, RetainNeedsAMatchingRelease) {
    MemoryAllocator a(config_with(1));
    const auto id = a.allocate();
    ASSERT_TRUE(id.has_value());
    a.retain(*id);
    EXPECT_EQ(a.info(*id)->ref_count, 2u);
    EXPECT_EQ(a.info(*id)->state, BlockState::Shared);
    EXPECT_EQ(a.stats().shared_blocks, 1u);
    a.release(*id);
    EXPECT_EQ(a.info(*id)->state, BlockState::Active);
    EXPECT_FALSE(a.allocate().has_value());
    a.release(*id);
    EXPECT_EQ(a.info(*id)->state, BlockState::Free);
    EXPECT_TRUE(a.allocate().has_value());
}

TEST(MemoryAllocatorTest, ReleaseAdvancesTheGenerationAndIgnoresFreeFrames) {
    MemoryAllocator a(config_with(2));
    const auto id = a.allocate();
    const std::uint64_t g0 = a.info(*id)->generation;
    a.release(*id);
    EXPECT_EQ(a.info(*id)->generation, g0 + 1);
    a.release(*id);  // already free: no effect, no double entry on the free list
    EXPECT_EQ(a.info(*id)->generation, g0 + 1);
    EXPECT_EQ(a.stats().free_blocks, 2u);
    std::set<PhysicalBlockId> ids;
    while (auto x = a.allocate()) ids.insert(*x);
    EXPECT_EQ(ids.size(), 2u);
    a.retain(77);
    a.release(77);  // invalid ids are ignored
}

TEST(MemoryAllocatorTest, CopyBlockCopiesTheWholeFrame) {
    MemoryAllocator a(config_with(3));
    const auto src = a.allocate();
    const auto dst = a.allocate();
    paint(*a.block(*src), 9);
    paint(*a.block(*dst), 1);
    a.copy_block(*src, *dst);
    EXPECT_TRUE(painted(*a.block(*dst), 9));
    EXPECT_TRUE(painted(*a.block(*src), 9));
    a.copy_block(*src, 1000);  // invalid destination: silently nothing
    a.copy_block(1000, *dst);
    EXPECT_TRUE(painted(*a.block(*dst), 9));
}

TEST(MemoryAllocatorTest, InvalidIdsResolveToNull) {
    MemoryAllocator a(config_with(2));
    EXPECT_EQ(a.block(2), nullptr);
    EXPECT_EQ(a.info(2), nullptr);
    EXPECT_NE(a.block(1), nullptr);
}

TEST(MemoryAllocatorTest, StatsFollowAllocateAndRelease) {
    MemoryAllocator a(config_with(4));
    const auto x = a.allocate();
    const auto y = a.allocate();
    EXPECT_EQ(a.stats().free_blocks, 2u);
    EXPECT_EQ(a.stats().active_blocks, 2u);
    a.release(*x);
    EXPECT_EQ(a.stats().free_blocks, 3u);
    EXPECT_EQ(a.stats().active_blocks, 1u);
    (void)y;
}

// stats() keeps running counts; a recount of every block's state after a
// seeded mix of allocate / retain / release / swap must give the same figures.
TEST(MemoryAllocatorTest, RunningStatsEqualARecount) {
    MemoryAllocator a(config_with(24));
    HostSwapBackend swap(64);
    a.set_swap_backend(&swap);
    std::vector<PhysicalBlockId> held;
    std::vector<SwapSlotId> slots;
    std::uint64_t rng = 12345;
    auto next = [&rng](std::uint64_t n) {
        rng = rng * 6364136223846793005ull + 1442695040888963407ull;
        return (rng >> 33) % n;
    };
    for (int step = 0; step < 3000; ++step) {
        const std::uint64_t op = next(6);
        if (op == 0 || held.empty()) {
            if (const auto id = a.allocate()) held.push_back(*id);
        } else if (op == 1) {
            const PhysicalBlockId id = held[next(held.size())];
            a.retain(id);
            held.push_back(id);
        } else if (op == 2 || op == 3) {
            const std::size_t k = next(held.size());
            a.release(held[k]);
            held.erase(held.begin() + static_cast<std::ptrdiff_t>(k));
        } else if (op == 4) {
            const std::size_t k = next(held.size());
            if (const auto slot = a.swap_out(held[k])) {
                slots.push_back(*slot);
                held.erase(held.begin() + static_cast<std::ptrdiff_t>(k));
            }
        } else if (!slots.empty()) {
            const std::size_t k = next(slots.size());
            if (const auto id = a.swap_in(slots[k])) {
                held.push_back(*id);
                slots.erase(slots.begin() + static_cast<std::ptrdiff_t>(k));
            }
        }
        std::uint32_t free_n = 0, active_n = 0, shared_n = 0;
        for (PhysicalBlockId id = 0; id < 24; ++id) {
            switch (a.info(id)->state) {
                case BlockState::Free: ++free_n; break;
                case BlockState::Active: ++active_n; break;
                case BlockState::Shared: ++shared_n; break;
                case BlockState::Swapped: break;
            }
        }
        const AllocatorStats st = a.stats();
        ASSERT_EQ(st.total_blocks, 24u);
        ASSERT_EQ(st.free_blocks, free_n);
        ASSERT_EQ(st.active_blocks, active_n);
        ASSERT_EQ(st.shared_blocks, shared_n);
        ASSERT_EQ(st.swapped_blocks, static_cast<std::uint32_t>(slots.size()));
        ASSERT_EQ(st.bytes_reserved, 24u * a.block(0)->size_bytes());
    }
}

TEST(MemoryAllocatorTest, CanAllocateComparesWithTheFreeCount) {
    MemoryAllocator a(config_with(2));
    EXPECT_TRUE(a.can_allocate(0));
    EXPECT_TRUE(a.can_allocate(2));
    EXPECT_FALSE(a.can_allocate(3));
    ASSERT_TRUE(a.allocate().has_value());
    EXPECT_TRUE(a.can_allocate(1));
    EXPECT_FALSE(a.can_allocate(2));
}

TEST(MemoryAllocatorSwapTest, NoBackendNoSwap) {
    MemoryAllocator a(config_with(1));
    const auto id = a.allocate();
    EXPECT_FALSE(a.swap_out(*id).has_value());
    EXPECT_EQ(a.info(*id)->ref_count, 1u);
    EXPECT_FALSE(a.swap_in(1).has_value());
}

TEST(MemoryAllocatorSwapTest, SwapOutFreesTheFrameAndAdvancesItsGeneration) {
    MemoryAllocator a(config_with(1));
    HostSwapBackend swap(2);
    a.set_swap_backend(&swap);
    const auto id = a.allocate();
    const std::uint64_t g0 = a.info(*id)->generation;
    ASSERT_FALSE(a.can_allocate(1));
    const auto slot = a.swap_out(*id);
    ASSERT_TRUE(slot.has_value());
    EXPECT_EQ(swap.resident_slots(), 1u);
    EXPECT_EQ(a.info(*id)->ref_count, 0u);
    EXPECT_GT(a.info(*id)->generation, g0);
    EXPECT_TRUE(a.can_allocate(1));
    EXPECT_TRUE(a.allocate().has_value());
}

TEST(MemoryAllocatorSwapTest, SharedFreeAndUnknownFramesStay) {
    MemoryAllocator a(config_with(2));
    HostSwapBackend swap(4);
    a.set_swap_backend(&swap);
    const auto shared = a.allocate();
    a.retain(*shared);
    EXPECT_FALSE(a.swap_out(*shared).has_value());
    EXPECT_EQ(a.info(*shared)->ref_count, 2u);
    const auto freed = a.allocate();
    a.release(*freed);
    EXPECT_FALSE(a.swap_out(*freed).has_value());
    EXPECT_FALSE(a.swap_out(500).has_value());
    EXPECT_EQ(swap.resident_slots(), 0u);
}

TEST(MemoryAllocatorSwapTest, FullSwapSpaceLeavesTheFrameResident) {
    MemoryAllocator a(config_with(2));
    HostSwapBackend swap(1);
    a.set_swap_backend(&swap);
    const auto x = a.allocate();
    const auto y = a.allocate();
    ASSERT_TRUE(a.swap_out(*x).has_value());
    EXPECT_FALSE(a.swap_out(*y).has_value());
    EXPECT_EQ(a.info(*y)->ref_count, 1u);
    EXPECT_EQ(a.info(*y)->state, BlockState::Active);
}

TEST(MemoryAllocatorSwapTest, RoundTripRestoresTheBytesAndConsumesTheSlot) {
    MemoryAllocator a(config_with(2));
    HostSwapBackend swap(2);
    a.set_swap_backend(&swap);
    const auto id = a.allocate();
    paint(*a.block(*id), 5);
    const auto slot = a.swap_out(*id);
    ASSERT_TRUE(slot.has_value());
    // Someone else takes the frame and overwrites it.
    const auto other = a.allocate();
    ASSERT_TRUE(other.has_value());
    paint(*a.block(*other), 200);
    const auto restored = a.swap_in(*slot);
    ASSERT_TRUE(restored.has_value());
    EXPECT_NE(*restored, *other);
    EXPECT_TRUE(painted(*a.block(*restored), 5));
    EXPECT_EQ(a.info(*restored)->ref_count, 1u);
    EXPECT_EQ(a.info(*restored)->state, BlockState::Active);
    EXPECT_EQ(swap.resident_slots(), 0u);
    EXPECT_FALSE(a.swap_in(*slot).has_value());
}

TEST(MemoryAllocatorSwapTest, SwapInWithAFullPoolKeepsTheSlot) {
    MemoryAllocator a(config_with(1));
    HostSwapBackend swap(1);
    a.set_swap_backend(&swap);
    const auto id = a.allocate();
    const auto slot = a.swap_out(*id);
    ASSERT_TRUE(a.allocate().has_value());
    EXPECT_FALSE(a.swap_in(*slot).has_value());
    EXPECT_EQ(swap.resident_slots(), 1u);
    EXPECT_EQ(a.stats().free_blocks, 0u);
}

TEST(MemoryAllocatorSwapTest, UnknownSlotTakesNoFrame) {
    MemoryAllocator a(config_with(2));
    HostSwapBackend swap(1);
    a.set_swap_backend(&swap);
    EXPECT_FALSE(a.swap_in(4242).has_value());
    EXPECT_EQ(a.stats().free_blocks, 2u);
}

TEST(MemoryAllocatorSwapTest, SwappedBlocksAreCountedApartFromFrames) {
    MemoryAllocator a(config_with(2));
    HostSwapBackend swap(2);
    a.set_swap_backend(&swap);
    const auto x = a.allocate();
    const auto y = a.allocate();
    const auto sx = a.swap_out(*x);
    ASSERT_TRUE(a.swap_out(*y).has_value());
    AllocatorStats s = a.stats();
    EXPECT_EQ(s.swapped_blocks, 2u);
    EXPECT_EQ(s.free_blocks, 2u);
    EXPECT_EQ(s.active_blocks, 0u);
    ASSERT_TRUE(a.swap_in(*sx).has_value());
    s = a.stats();
    EXPECT_EQ(s.swapped_blocks, 1u);
    EXPECT_EQ(s.active_blocks, 1u);
    a.discard_swapped(99);  // unknown: ignored
    EXPECT_EQ(a.stats().swapped_blocks, 1u);
}

TEST(MemoryAllocatorEvictionTest, SelectorIsAdvisoryOnly) {
    MemoryAllocator a(config_with(2));
    EXPECT_FALSE(a.select_eviction_candidate().has_value());
    const auto victim = a.allocate();
    std::uint32_t seen_total = 0;
    int calls = 0;
    a.set_eviction_selector([&](const MemoryAllocator& alloc) -> std::optional<PhysicalBlockId> {
        ++calls;
        seen_total = alloc.stats().total_blocks;
        return victim;
    });
    EXPECT_EQ(a.select_eviction_candidate(), victim);
    EXPECT_EQ(seen_total, 2u);
    // Exhausting the pool never calls the selector or swaps anything.
    HostSwapBackend swap(2);
    a.set_swap_backend(&swap);
    ASSERT_TRUE(a.allocate().has_value());
    const int before = calls;
    EXPECT_FALSE(a.allocate().has_value());
    EXPECT_EQ(calls, before);
    EXPECT_EQ(swap.resident_slots(), 0u);
    a.set_eviction_selector([](const MemoryAllocator&) { return std::optional<PhysicalBlockId>{}; });
    EXPECT_FALSE(a.select_eviction_candidate().has_value());
}

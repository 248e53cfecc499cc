// Contract of the host swap store (include/qwenvl_paged/SwapBackend.h of the
// reference; tests/SwapBackend.test.cpp:58-179 states the same rules). The
// pinned-arena backend of the device allocator is held to the same rules in
// DeviceAllocator.test.cpp.
#include "minitest.h"
#include "qwenvl_paged/SwapBackend.h"

#include <cstring>
#include <set>

using namespace qwenvl_paged;

namespace {

BlockShape swap_shape() {
    BlockShape s;
    s.tokens_per_block = 16;
    s.num_layers = 2;
    s.num_kv_heads = 2;
    s.head_dim = 8;
    s.bytes_per_element = 4;
    return s;
}

void paint(PhysicalBlock& b, unsigned seed) {
    for (std::size_t i = 0; i < b.size_bytes(); ++i) b.data()[i] = static_cast<std::byte>((i * 31 + seed) % 241);
}

bool same_bytes(const PhysicalBlock& a, const PhysicalBlock& b) {
    return a.size_bytes() == b.size_bytes() && std::memcmp(a.data(), b.data(), a.size_bytes()) == 0;
}

}  // namespace

TEST(HostSwapBackendTest, EmptyWithItsCapacity) {
    HostSwapBackend s(4);
    EXPECT_EQ(s.resident_slots(), 0u);
    EXPECT_EQ(s.capacity_slots(), 4u);
}

TEST(HostSwapBackendTest, SlotsAreDistinctNonZeroAndNeverReused) {
    HostSwapBackend s(3);
    PhysicalBlock b(0, swap_shape());
    std::set<SwapSlotId> seen;
    for (int round = 0; round < 5; ++round) {
        const auto x = s.store(b);
        const auto y = s.store(b);
        ASSERT_TRUE(x && y);
        EXPECT_NE(*x, 0u);
        EXPECT_TRUE(seen.insert(*x).second);
        EXPECT_TRUE(seen.insert(*y).second);
        EXPECT_EQ(s.resident_slots(), 2u);
        s.discard(*x);
        s.discard(*y);
    }
}

TEST(HostSwapBackendTest, LoadRestoresTheStoredBytesAndKeepsTheSlot) {
    HostSwapBackend s(2);
    PhysicalBlock src(0, swap_shape());
    PhysicalBlock dst(1, swap_shape());
    paint(src, 7);
    paint(dst, 100);
    ASSERT_FALSE(same_bytes(src, dst));
    const auto slot = s.store(src);
    ASSERT_TRUE(slot.has_value());
    EXPECT_TRUE(s.load(*slot, dst));
    EXPECT_TRUE(same_bytes(src, dst));
    EXPECT_EQ(s.resident_slots(), 1u);
    paint(dst, 3);
    EXPECT_TRUE(s.load(*slot, dst));  // retry after a failed consumer
    EXPECT_TRUE(same_bytes(src, dst));
}

TEST(HostSwapBackendTest, StoredBytesAreACopy) {
    HostSwapBackend s(2);
    PhysicalBlock src(0, swap_shape());
    PhysicalBlock expect(1, swap_shape());
    PhysicalBlock out(2, swap_shape());
    paint(src, 11);
    paint(expect, 11);
    const auto slot = s.store(src);
    paint(src, 99);
    ASSERT_TRUE(s.load(*slot, out));
    EXPECT_TRUE(same_bytes(out, expect));
}

TEST(HostSwapBackendTest, UnknownAndDiscardedSlotsDoNotLoad) {
    HostSwapBackend s(2);
    PhysicalBlock b(0, swap_shape());
    EXPECT_FALSE(s.load(12345, b));
    const auto slot = s.store(b);
    s.discard(*slot);
    EXPECT_EQ(s.resident_slots(), 0u);
    EXPECT_FALSE(s.load(*slot, b));
    s.discard(*slot);  // twice: no effect
    EXPECT_EQ(s.resident_slots(), 0u);
}

TEST(HostSwapBackendTest, FullUntilADiscard) {
    HostSwapBackend s(1);
    PhysicalBlock a(0, swap_shape());
    PhysicalBlock b(1, swap_shape());
    const auto first = s.store(a);
    ASSERT_TRUE(first.has_value());
    EXPECT_FALSE(s.store(b).has_value());
    EXPECT_EQ(s.resident_slots(), 1u);
    s.discard(*first);
    EXPECT_TRUE(s.store(b).has_value());
    HostSwapBackend none(0);
    EXPECT_FALSE(none.store(a).has_value());
}

TEST(HostSwapBackendTest, LoadRefusesATooSmallBlock) {
    HostSwapBackend s(1);
    PhysicalBlock big(0, swap_shape());
    BlockShape small = swap_shape();
    small.num_layers = 1;
    small.tokens_per_block = 1;
    PhysicalBlock tiny(1, small);
    ASSERT_LT(tiny.size_bytes(), big.size_bytes());
    const auto slot = s.store(big);
    EXPECT_FALSE(s.load(*slot, tiny));
    EXPECT_EQ(s.resident_slots(), 1u);
}

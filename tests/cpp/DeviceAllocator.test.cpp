// Device placement of the block pool: frames in one HBM allocation, copy-on-write
// copies and swap gathers/scatters queued and run as batched launches. The
// results must be byte-identical to the host placement (the reference's
// synchronous memcpy semantics, src/MemoryAllocator.cpp:76-85,105-158 and
// src/SwapBackend.cpp:10-51), which the replay test checks over a random
// operation mix.
#include "../../oracle/trace_driver.h"
#include "device_harness.h"
#include "golden_path.h"

#include <map>
#include <random>

using namespace device_test;

namespace {

std::vector<std::uint8_t> random_bytes(std::size_t n, std::uint32_t seed) {
    std::mt19937 rng(seed);
    std::vector<std::uint8_t> v(n);
    for (auto& b : v) b = static_cast<std::uint8_t>(rng());
    return v;
}

std::vector<std::uint8_t> read_frame(MemoryAllocator& a, PhysicalBlockId id) {
    std::vector<std::uint8_t> v(a.block(id)->size_bytes());
    EXPECT_TRUE(a.read_block_bytes(id, 0, v.data(), v.size()));
    return v;
}

void write_frame(MemoryAllocator& a, PhysicalBlockId id, const std::vector<std::uint8_t>& v) {
    EXPECT_TRUE(a.write_block_bytes(id, 0, v.data(), v.size()));
}

BlockShape small_shape() { return shape_of(4, 2, 2, 8, 4); }  // 1024 bytes

}  // namespace

TEST(DeviceAllocatorTest, FramesAreOnePoolAtAFixedStride) {
    MemoryAllocator a(device_config(shape_of(3, 1, 1, 8, 4), 10));  // 192 bytes -> stride 256
    ASSERT_TRUE(a.ok()) << a.last_error();
    EXPECT_EQ(a.placement(), BlockPlacement::Device);
    ASSERT_NE(a.device_base(), nullptr);
    EXPECT_EQ(a.block_stride(), 256u);
    for (PhysicalBlockId i = 0; i < 10; ++i) {
        EXPECT_EQ(a.block(i)->data(), static_cast<std::byte*>(a.device_base()) + i * 256u);
        EXPECT_EQ(a.block(i)->placement(), BlockPlacement::Device);
        EXPECT_EQ(a.block(i)->size_bytes(), 256u);
    }
    EXPECT_EQ(a.stats().bytes_reserved, 2560u);
    EXPECT_NE(a.stream(), nullptr);
    EXPECT_NE(a.side_stream(), nullptr);
}

TEST(DeviceAllocatorTest, HostBytesRoundTripThroughFrames) {
    MemoryAllocator a(device_config(small_shape(), 4));
    ASSERT_TRUE(a.ok());
    for (PhysicalBlockId i = 0; i < 4; ++i) write_frame(a, i, random_bytes(1024, 10 + i));
    for (PhysicalBlockId i = 0; i < 4; ++i) EXPECT_TRUE(read_frame(a, i) == random_bytes(1024, 10 + i));
    std::vector<std::uint8_t> part = {1, 2, 3, 4, 5};
    EXPECT_TRUE(a.write_block_bytes(2, 1019, part.data(), 5));
    EXPECT_FALSE(a.write_block_bytes(2, 1020, part.data(), 5));  // past the frame
    EXPECT_FALSE(a.write_block_bytes(7, 0, part.data(), 1));     // no such frame
    const auto back = read_frame(a, 2);
    EXPECT_EQ(back[1019], 1u);
    EXPECT_EQ(back[1023], 5u);
}

TEST(DeviceAllocatorTest, IndependentCopiesRunAsOneLaunch) {
    MemoryAllocator a(device_config(small_shape(), 12));
    ASSERT_TRUE(a.ok());
    for (PhysicalBlockId i = 0; i < 12; ++i) write_frame(a, i, random_bytes(1024, 100 + i));
    const std::uint64_t launches = a.copy_launches();
    // Frames 0..4 fan out to 6..10; frame 0 is read twice.
    const std::pair<PhysicalBlockId, PhysicalBlockId> copies[] = {{0, 6}, {1, 7}, {2, 8}, {0, 9}, {4, 10}};
    for (auto [s, d] : copies) a.copy_block(s, d);
    EXPECT_EQ(a.pending_operations(), 5u);
    ASSERT_TRUE(a.flush());
    EXPECT_EQ(a.pending_operations(), 0u);
    EXPECT_EQ(a.copy_launches() - launches, 1u);
    for (auto [s, d] : copies) EXPECT_TRUE(read_frame(a, d) == random_bytes(1024, 100 + s)) << s << "->" << d;
    EXPECT_TRUE(read_frame(a, 11) == random_bytes(1024, 111));
    a.copy_block(3, 3);  // self copy: nothing to do
    a.copy_block(3, 99);
    EXPECT_EQ(a.pending_operations(), 0u);
}

TEST(DeviceAllocatorTest, DependentCopiesKeepTheirOrder) {
    MemoryAllocator a(device_config(small_shape(), 6));
    ASSERT_TRUE(a.ok());
    for (PhysicalBlockId i = 0; i < 6; ++i) write_frame(a, i, random_bytes(1024, 200 + i));
    const std::uint64_t launches = a.copy_launches();
    a.copy_block(0, 1);  // 1 := 0
    a.copy_block(1, 2);  // 2 := 1 (reads what the first wrote)
    a.copy_block(3, 0);  // 0 := 3 (overwrites what the first read)
    a.copy_block(4, 2);  // 2 := 4 (writes what the second wrote)
    ASSERT_TRUE(a.flush());
    EXPECT_GE(a.copy_launches() - launches, 3u);
    EXPECT_TRUE(read_frame(a, 1) == random_bytes(1024, 200));
    EXPECT_TRUE(read_frame(a, 2) == random_bytes(1024, 204));
    EXPECT_TRUE(read_frame(a, 0) == random_bytes(1024, 203));
}

TEST(DeviceAllocatorTest, ForkFanOutCopiesInOneLaunch) {
    DeviceHarness h(small_shape(), 32);
    ASSERT_TRUE(h.ready());
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(1, 10));  // 3 blocks
    const auto parent = h.cache.cache_view(1);
    std::vector<std::vector<std::uint8_t>> originals;
    for (LogicalBlockIndex i = 0; i < 3; ++i) {
        originals.push_back(random_bytes(1024, 300 + i));
        write_frame(h.allocator, *parent->block_table->lookup(i), originals.back());
    }
    for (SequenceId c = 2; c < 10; ++c) ASSERT_TRUE(h.cache.fork_sequence(1, SequenceMetadata{c, 1, {}, {}}));
    const std::uint64_t launches = h.allocator.copy_launches();
    std::map<SequenceId, PhysicalBlockId> private_frame;
    for (SequenceId c = 2; c < 10; ++c) {
        const auto f = h.cache.ensure_token_writable(c, 9);
        ASSERT_TRUE(f.has_value());
        private_frame[c] = *f;
    }
    // Every child copies: the parent keeps the shared frame to the end.
    EXPECT_EQ(h.allocator.pending_operations(), 8u);
    ASSERT_TRUE(h.allocator.flush());
    EXPECT_EQ(h.allocator.copy_launches() - launches, 1u);
    for (auto [c, f] : private_frame) {
        EXPECT_TRUE(read_frame(h.allocator, f) == originals[2]) << "child " << c;
        EXPECT_EQ(*h.cache.cache_view(c)->block_table->lookup(2), f);
    }
}

TEST(DeviceAllocatorTest, SwapRoundTripIsBitExactAndBatched) {
    DeviceHarness h(small_shape(), 6, 8);
    ASSERT_TRUE(h.ready());
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(1, 16));  // 4 blocks
    for (LogicalBlockIndex i = 0; i < 4; ++i) {
        write_frame(h.allocator, *h.cache.cache_view(1)->block_table->lookup(i), random_bytes(1024, 400 + i));
    }
    const std::uint64_t launches = h.allocator.swap_launches();
    ASSERT_EQ(h.cache.swap_out_sequence(1), 4u);
    EXPECT_EQ(h.swap.resident_slots(), 4u);
    // The arena holds the frames' bytes once the gathers ran.
    for (LogicalBlockIndex i = 0; i < 4; ++i) {
        const auto slot = *h.cache.cache_view(1)->block_table->entry(i)->swap_slot;
        const std::byte* bytes = h.swap.slot_bytes(slot);
        ASSERT_NE(bytes, nullptr);
        EXPECT_EQ(std::memcmp(bytes, random_bytes(1024, 400 + i).data(), 1024), 0) << "block " << i;
    }
    EXPECT_EQ(h.allocator.swap_launches() - launches, 1u);
    // Another sequence takes and scribbles over every frame.
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{2, 2, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(2, 24));
    for (LogicalBlockIndex i = 0; i < 6; ++i) {
        write_frame(h.allocator, *h.cache.cache_view(2)->block_table->lookup(i), random_bytes(1024, 900 + i));
    }
    EXPECT_FALSE(h.cache.swap_in_sequence(1));  // pool full: all or nothing
    h.cache.release_sequence(2);
    ASSERT_TRUE(h.cache.swap_in_sequence(1));
    EXPECT_EQ(h.swap.resident_slots(), 0u);
    for (LogicalBlockIndex i = 0; i < 4; ++i) {
        const auto f = h.cache.cache_view(1)->block_table->lookup(i);
        ASSERT_TRUE(f.has_value());
        EXPECT_TRUE(read_frame(h.allocator, *f) == random_bytes(1024, 400 + i)) << "block " << i;
    }
}

TEST(DeviceAllocatorTest, PinnedBackendFollowsTheSwapContract) {
    MemoryAllocator a(device_config(small_shape(), 4));
    PinnedSwapBackend s(a, 2);
    ASSERT_TRUE(a.ok() && s.ok());
    EXPECT_EQ(s.capacity_slots(), 2u);
    EXPECT_EQ(s.slot_stride(), a.block_stride());
    const auto x = s.store(*a.block(0));
    const auto y = s.store(*a.block(1));
    ASSERT_TRUE(x && y);
    EXPECT_NE(*x, *y);
    EXPECT_FALSE(s.store(*a.block(2)).has_value());  // full
    EXPECT_TRUE(s.load(*x, *a.block(3)));
    EXPECT_EQ(s.resident_slots(), 2u);  // load keeps the slot
    EXPECT_FALSE(s.load(777, *a.block(3)));
    s.discard(*x);
    EXPECT_FALSE(s.load(*x, *a.block(3)));
    EXPECT_EQ(s.slot_bytes(*x), nullptr);
    EXPECT_TRUE(s.store(*a.block(2)).has_value());
    // Frames of another pool, or host blocks, cannot be named by this pool's queue.
    MemoryAllocator other(device_config(small_shape(), 4));
    PhysicalBlock host_block(0, small_shape());
    s.discard(*y);
    EXPECT_FALSE(s.store(*other.block(0)).has_value());
    EXPECT_FALSE(s.store(host_block).has_value());
    EXPECT_TRUE(a.synchronize());
}

TEST(DeviceAllocatorTest, DeviceEngineReplaysTheHostEngineByteForByte) {
    // The same random mix of create / reserve / fork / token writes / swap
    // out / swap in / release on host frames (the reference's memcpy
    // semantics) and on device frames (queued, batched launches on two
    // streams). Every decision and every byte of every frame must agree.
    const BlockShape shape = small_shape();
    constexpr std::uint32_t kFrames = 24;
    HostHarness host(shape, kFrames, 32);
    DeviceHarness dev(shape, kFrames, 32);
    ASSERT_TRUE(dev.ready());
    const std::vector<std::uint8_t> zero(1024, 0);
    for (PhysicalBlockId f = 0; f < kFrames; ++f) {
        ASSERT_TRUE(host.allocator.write_block_bytes(f, 0, zero.data(), zero.size()));
        ASSERT_TRUE(dev.allocator.write_block_bytes(f, 0, zero.data(), zero.size()));
    }
    std::mt19937 rng(2024);
    std::map<SequenceId, std::uint32_t> tokens;  // reserved tokens per live sequence
    SequenceId next_id = 1;
    int writes = 0, forks = 0, swaps_out = 0, swaps_in = 0;
    for (int op = 0; op < 600; ++op) {
        const std::uint32_t kind = rng() % 8;
        auto pick = [&]() -> std::optional<SequenceId> {
            if (tokens.empty()) return std::nullopt;
            auto it = tokens.begin();
            std::advance(it, rng() % tokens.size());
            return it->first;
        };
        if (kind == 0 || tokens.empty()) {
            const SequenceId id = next_id++;
            const std::uint32_t n = 1 + rng() % 12;
            SequenceMetadata m{id, id, {}, {}};
            ASSERT_EQ(host.cache.create_sequence(m), dev.cache.create_sequence(m));
            const bool a = host.cache.reserve_tokens(id, n);
            ASSERT_EQ(a, dev.cache.reserve_tokens(id, n)) << "op " << op;
            tokens[id] = a ? ((n + 3) / 4) * 4 : 0;
        } else if (kind == 1) {
            const SequenceId parent = *pick();
            const SequenceId id = next_id++;
            SequenceMetadata m{id, parent, {}, {}};
            const bool a = host.cache.fork_sequence(parent, m);
            ASSERT_EQ(a, dev.cache.fork_sequence(parent, m)) << "op " << op;
            if (a) {
                tokens[id] = tokens[parent];
                ++forks;
            }
        } else if (kind <= 4) {
            const SequenceId id = *pick();
            if (tokens[id] == 0) continue;
            const TokenPosition t = rng() % tokens[id];
            const auto hf = host.cache.ensure_token_writable(id, t);
            const auto df = dev.cache.ensure_token_writable(id, t);
            ASSERT_EQ(hf, df) << "op " << op;
            if (!hf) continue;
            // Write every layer/stream/head vector of the token.
            for (std::uint32_t layer = 0; layer < shape.num_layers; ++layer) {
                for (KVStream st : {KVStream::Key, KVStream::Value}) {
                    for (std::uint32_t hd = 0; hd < shape.num_kv_heads; ++hd) {
                        std::vector<float> v(shape.head_dim);
                        for (auto& x : v) x = static_cast<float>(rng() % 1000) * 0.001f;
                        const std::size_t off = *host.layout.element_offset(layer, st, t % 4, hd) * 4;
                        ASSERT_TRUE(host.allocator.write_block_bytes(*hf, off, v.data(), v.size() * 4));
                        ASSERT_TRUE(dev.allocator.write_block_bytes(*df, off, v.data(), v.size() * 4));
                    }
                }
            }
            ++writes;
        } else if (kind == 5) {
            const SequenceId id = *pick();
            const std::uint32_t a = host.cache.swap_out_sequence(id);
            ASSERT_EQ(a, dev.cache.swap_out_sequence(id)) << "op " << op;
            swaps_out += a > 0;
        } else if (kind == 6) {
            const SequenceId id = *pick();
            const bool a = host.cache.swap_in_sequence(id);
            ASSERT_EQ(a, dev.cache.swap_in_sequence(id)) << "op " << op;
            swaps_in += a;
        } else {
            const SequenceId id = *pick();
            host.cache.release_sequence(id);
            dev.cache.release_sequence(id);
            tokens.erase(id);
        }
        const AllocatorStats hs = host.allocator.stats(), ds = dev.allocator.stats();
        ASSERT_EQ(hs.free_blocks, ds.free_blocks) << "op " << op;
        ASSERT_EQ(hs.shared_blocks, ds.shared_blocks) << "op " << op;
        ASSERT_EQ(hs.swapped_blocks, ds.swapped_blocks) << "op " << op;
    }
    EXPECT_GT(writes, 50);
    EXPECT_GT(forks, 10);
    EXPECT_GT(swaps_out, 5);
    EXPECT_GT(swaps_in, 2);
    for (const auto& [id, n] : tokens) {
        const auto hv = host.cache.cache_view(id);
        const auto dv = dev.cache.cache_view(id);
        ASSERT_EQ(hv->block_table->size(), dv->block_table->size());
        for (std::size_t i = 0; i < hv->block_table->size(); ++i) {
            const BlockTableEntry& he = hv->block_table->entries()[i];
            const BlockTableEntry& de = dv->block_table->entries()[i];
            EXPECT_EQ(he.physical_id, de.physical_id);
            EXPECT_EQ(he.swap_slot, de.swap_slot);
            EXPECT_EQ(he.writable, de.writable);
        }
    }
    for (PhysicalBlockId f = 0; f < kFrames; ++f) {
        std::vector<std::uint8_t> hb(1024), db(1024);
        ASSERT_TRUE(host.allocator.read_block_bytes(f, 0, hb.data(), hb.size()));
        ASSERT_TRUE(dev.allocator.read_block_bytes(f, 0, db.data(), db.size()));
        EXPECT_TRUE(hb == db) << "frame " << f;
    }
}

TEST(DeviceAllocatorTest, DeviceEngineReproducesTheReferenceSchedulerTrace) {
    // The trace of oracle/trace_driver.h with the reference's settings
    // (tests/golden/make_golden.py), on device frames and the pinned arena.
    for (auto [fixture, seed, watermark] : {std::tuple<const char*, std::uint64_t, std::uint32_t>{
                                                "scheduler_trace_w4.txt", 5, 4},
                                            {"scheduler_trace_w0.txt", 11, 0}}) {
        trace::Config c;
        c.requests = 32;
        c.seed = seed;
        c.pool_percent = 30;
        c.watermark_blocks = watermark;
        std::string expected;
        ASSERT_TRUE(golden::read(fixture, expected)) << fixture;
        MemoryAllocator allocator(device_config(shape_of(c.tokens_per_block, 1, 1, 8, 4), trace::pool_blocks(c)));
        PinnedSwapBackend swap(allocator, 4 * trace::pool_blocks(c));
        ASSERT_TRUE(allocator.ok() && swap.ok());
        allocator.set_swap_backend(&swap);
        const std::string log =
            trace::run<MemoryAllocator, KVCacheManager, Scheduler, SchedulerConfig, Request, RequestState>(c, allocator);
        EXPECT_TRUE(log == expected) << fixture << " " << golden::first_difference(log, expected);
        EXPECT_TRUE(allocator.synchronize());
        EXPECT_GT(allocator.swap_launches(), 0u);
    }
}

TEST(DeviceAllocatorTest, DeviceEngineReproducesTheConfig5Trace) {
    // The fifth benchmark configuration's trace at full size (200 requests,
    // pool 60 % of demand, watermark 64; tests/golden/make_golden.py
    // CONFIG5_PARAMS), on device frames and the pinned arena.
    trace::Config c;
    c.requests = 200;
    c.prompt_lo = 128;
    c.prompt_hi = 8192;
    c.output_lo = 32;
    c.output_hi = 1024;
    c.arrivals_per_step = 200;
    c.pool_percent = 60;
    c.watermark_blocks = 64;
    c.max_active = 256;
    c.max_batch_tokens = 16384;
    c.max_steps = 200000;
    c.cancel_after_decodes = true;
    c.seed = 5;
    std::string expected;
    ASSERT_TRUE(golden::read_gz("scheduler_trace_config5.txt.gz", expected));
    MemoryAllocator allocator(device_config(shape_of(c.tokens_per_block, 1, 1, 8, 4), trace::pool_blocks(c)));
    PinnedSwapBackend swap(allocator, trace::pool_blocks(c));
    ASSERT_TRUE(allocator.ok() && swap.ok());
    allocator.set_swap_backend(&swap);
    const std::string log =
        trace::run<MemoryAllocator, KVCacheManager, Scheduler, SchedulerConfig, Request, RequestState>(c, allocator);
    EXPECT_TRUE(log == expected) << golden::first_difference(log, expected);
    EXPECT_TRUE(allocator.synchronize());
    EXPECT_GT(allocator.swap_launches(), 0u);
}

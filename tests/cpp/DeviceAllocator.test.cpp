// Device placement of the block pool: frames in one HBM allocation, copy-on-write
// copies and swap gathers/scatters queued and run as batched launches. The
// results must be byte-identical to the host placement (the reference's
// synchronous memcpy semantics, src/MemoryAllocator.cpp:76-85,105-158 and
// src/SwapBackend.cpp:10-51), which the replay test checks over a random
// operation mix.
#include "../../oracle/trace_driver.h"
#include "../../qwenvl-paged_amd/host/bench/kv_pattern.h"
#include "device_harness.h"
#include "golden_path.h"
#include "qvp.h"
#include "qwenvl_paged/KVAppend.h"

#include <deque>
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

namespace {

float bf16_value(std::uint16_t bits) {
    const std::uint32_t u = static_cast<std::uint32_t>(bits) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// Device work of the swap-beside-engine test: K/V rows of the seeded pattern
// appended through KVAppendBatch, and batched decodes into their own output
// buffers, all enqueued on the allocator's engine stream without waiting.
struct EngineSteps {
    static constexpr std::uint32_t kHq = 28, kHkv = 4, kD = 128, kRow = kHkv * kD, kQRow = kHq * kD;

    explicit EngineSteps(DeviceHarness& harness) : h(harness) {}
    ~EngineSteps() {
        for (void* p : buffers) (void)qvp_free(p);
    }

    void* device_copy(const std::vector<std::uint16_t>& host) {
        void* d = nullptr;
        if (qvp_malloc(&d, host.size() * 2) != QVP_OK) return nullptr;
        buffers.push_back(d);
        if (qvp_memcpy_htod(d, host.data(), host.size() * 2, h.allocator.stream()) != QVP_OK) return nullptr;
        return d;
    }

    // Rows [from, to) of sequence seq.
    bool append(SequenceId seq, std::uint32_t from, std::uint32_t to) {
        std::vector<SequenceId> seqs;
        std::vector<TokenPosition> pos;
        std::vector<std::uint16_t>& k = staged.emplace_back(static_cast<std::size_t>(to - from) * kRow);
        std::vector<std::uint16_t>& v = staged.emplace_back(static_cast<std::size_t>(to - from) * kRow);
        for (std::uint32_t t = from; t < to; ++t) {
            seqs.push_back(seq);
            pos.push_back(t);
            kv_pattern::kv_row(seq, t, 0, k.data() + static_cast<std::size_t>(t - from) * kRow, kRow);
            kv_pattern::kv_row(seq, t, 1, v.data() + static_cast<std::size_t>(t - from) * kRow, kRow);
        }
        void* dk = device_copy(k);
        void* dv = device_copy(v);
        if (dk == nullptr || dv == nullptr) return false;
        KVAppendBatch batch;
        const bool ok = batch.append(h.cache, h.allocator, seqs, pos, 0, 1, dk, dv);
        if (!ok) std::fprintf(stderr, "append: %s\n", batch.last_error().c_str());
        return ok;
    }

    struct Decoded {
        std::vector<SequenceId> seqs;
        std::vector<std::uint32_t> lens;
        void* out;
    };

    bool decode(const std::vector<SequenceId>& seqs, const std::vector<std::uint32_t>& lens) {
        std::vector<CacheView> views;
        for (SequenceId s : seqs) views.push_back(*h.cache.cache_view(s));
        if (query == nullptr) {
            std::vector<std::uint16_t> q(8 * kQRow);
            for (std::uint32_t r = 0; r < 8; ++r) kv_pattern::query_row(r, q.data() + r * kQRow, kQRow);
            query_host = q;
            query = device_copy(q);
            if (query == nullptr) return false;
        }
        void* out = nullptr;
        if (qvp_malloc(&out, seqs.size() * kQRow * 4) != QVP_OK) return false;
        buffers.push_back(out);
        batches.emplace_back();
        PagedAttentionBatch& b = batches.back();
        if (!b.decode(views, lens, 0, kHq, 1.0f / std::sqrt(128.0f), query, out, ElementType::F32)) {
            std::fprintf(stderr, "decode: %s\n", b.last_error().c_str());
            return false;
        }
        decoded.push_back({seqs, lens, out});
        return true;
    }

    DeviceHarness& h;
    std::deque<std::vector<std::uint16_t>> staged;  // host rows, alive until the copies ran
    std::deque<PagedAttentionBatch> batches;         // packed arrays read by enqueued decodes
    std::vector<void*> buffers;
    std::vector<std::uint16_t> query_host;
    void* query{nullptr};
    std::vector<Decoded> decoded;
};

}  // namespace

TEST(DeviceAllocatorTest, SwapsBesideDecodesAndAppendsKeepEveryByte) {
    // Engine work enqueued while swap batches still run on the side stream,
    // with no host read or write of a frame (which would flush and wait) in
    // between: a sequence swapped out has its frames taken at once by a new
    // sequence whose append overwrites them (the append must wait for the
    // gathers), a sequence swapped back in lands in frames a decode enqueued
    // just before still reads (the scatters must wait for it), and a token
    // appended right after a swap-in writes a frame its scatter fills. Every
    // decode must equal float64 attention over the pattern's rows, and every
    // frame of the surviving sequences must hold exactly those rows.
    DeviceHarness h(shape_of(16, 1, 4, 128, 2), 256, 256);
    ASSERT_TRUE(h.ready());
    EngineSteps e(h);
    const std::uint32_t lenA = 1500, lenB = 1200, lenC = 1500, lenD = 1000;
    for (auto [id, n] : {std::pair<SequenceId, std::uint32_t>{1, lenA}, {2, lenB}}) {
        ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{id, id, {}, {}}));
        ASSERT_TRUE(h.cache.reserve_tokens(id, n));
        ASSERT_TRUE(e.append(id, 0, n));
    }
    ASSERT_TRUE(e.decode({1, 2}, {lenA, lenB}));
    const std::vector<PhysicalBlockId> a_frames = [&] {
        std::vector<PhysicalBlockId> f;
        for (const BlockTableEntry& x : h.cache.cache_view(1)->block_table->entries()) f.push_back(x.physical_id);
        return f;
    }();
    // A out; C takes A's frames and overwrites them.
    ASSERT_EQ(h.cache.swap_out_sequence(1), 94u);
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{3, 3, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(3, lenC));
    std::size_t reused = 0;
    for (const BlockTableEntry& x : h.cache.cache_view(3)->block_table->entries()) {
        reused += std::count(a_frames.begin(), a_frames.end(), x.physical_id);
    }
    EXPECT_EQ(reused, a_frames.size());  // LIFO free list: C holds every frame A left
    ASSERT_TRUE(e.append(3, 0, lenC));
    ASSERT_TRUE(e.decode({2, 3}, {lenB, lenC}));
    // B released while that decode may still read it; A comes back into B's frames.
    h.cache.release_sequence(2);
    ASSERT_TRUE(h.cache.swap_in_sequence(1));
    ASSERT_TRUE(h.cache.reserve_tokens(1, 1));
    ASSERT_TRUE(e.append(1, lenA, lenA + 1));
    ASSERT_TRUE(e.decode({1, 3}, {lenA + 1, lenC}));
    // C out, D over its frames, then C back in place of D.
    ASSERT_EQ(h.cache.swap_out_sequence(3), 94u);
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{4, 4, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(4, lenD));
    ASSERT_TRUE(e.append(4, 0, lenD));
    ASSERT_TRUE(e.decode({1, 4}, {lenA + 1, lenD}));
    h.cache.release_sequence(4);
    ASSERT_TRUE(h.cache.swap_in_sequence(3));
    ASSERT_TRUE(e.decode({3, 1}, {lenC, lenA + 1}));
    EXPECT_GT(h.allocator.swap_launches(), 0u);
    ASSERT_TRUE(h.allocator.synchronize());

    for (std::size_t k = 0; k < e.decoded.size(); ++k) {
        const EngineSteps::Decoded& dec = e.decoded[k];
        std::vector<float> got(dec.seqs.size() * EngineSteps::kQRow);
        ASSERT_EQ(qvp_memcpy_dtoh(got.data(), dec.out, got.size() * 4, h.allocator.stream()), QVP_OK);
        ASSERT_EQ(qvp_stream_synchronize(h.allocator.stream()), QVP_OK);
        for (std::size_t b = 0; b < dec.seqs.size(); ++b) {
            const SequenceId s = dec.seqs[b];
            // Cache every row of the sequence once, as float.
            std::vector<float> K(static_cast<std::size_t>(dec.lens[b]) * EngineSteps::kRow), V(K.size());
            std::vector<std::uint16_t> row(EngineSteps::kRow);
            for (std::uint32_t t = 0; t < dec.lens[b]; ++t) {
                kv_pattern::kv_row(s, t, 0, row.data(), row.size());
                for (std::uint32_t i = 0; i < EngineSteps::kRow; ++i) K[t * EngineSteps::kRow + i] = bf16_value(row[i]);
                kv_pattern::kv_row(s, t, 1, row.data(), row.size());
                for (std::uint32_t i = 0; i < EngineSteps::kRow; ++i) V[t * EngineSteps::kRow + i] = bf16_value(row[i]);
            }
            std::vector<float> q(EngineSteps::kQRow);
            for (std::uint32_t i = 0; i < EngineSteps::kQRow; ++i) q[i] = bf16_value(e.query_host[b * EngineSteps::kQRow + i]);
            const auto expect = textbook_attention(
                q, EngineSteps::kHq, EngineSteps::kHkv, EngineSteps::kD, dec.lens[b], 1.0f / std::sqrt(128.0f),
                [&](auto t, auto kh, auto d) { return double(K[t * EngineSteps::kRow + kh * EngineSteps::kD + d]); },
                [&](auto t, auto kh, auto d) { return double(V[t * EngineSteps::kRow + kh * EngineSteps::kD + d]); });
            for (std::size_t i = 0; i < expect.size(); ++i) {
                const double tol = 2e-3 + std::fabs(expect[i]) / 256.0;
                ASSERT_NEAR(got[b * EngineSteps::kQRow + i], expect[i], tol)
                    << "decode " << k << " sequence " << s << " element " << i;
            }
        }
    }
    // Frames of A (swapped out, in, one token appended) and C (swapped out and in).
    for (auto [s, n] : {std::pair<SequenceId, std::uint32_t>{1, lenA + 1}, {3, lenC}}) {
        const auto view = h.cache.cache_view(s);
        ASSERT_TRUE(view.has_value());
        std::vector<std::uint16_t> expect(EngineSteps::kRow), frame(h.allocator.block_stride() / 2);
        for (std::uint32_t j = 0; j < (n + 15) / 16; ++j) {
            const auto f = view->block_table->lookup(j);
            ASSERT_TRUE(f.has_value());
            ASSERT_TRUE(h.allocator.read_block_bytes(*f, 0, frame.data(), frame.size() * 2));
            for (std::uint32_t t = 0; t < 16 && j * 16 + t < n; ++t) {
                for (std::uint32_t st = 0; st < 2; ++st) {
                    kv_pattern::kv_row(s, j * 16 + t, st, expect.data(), expect.size());
                    const std::uint16_t* at = frame.data() + st * 16 * EngineSteps::kRow + t * EngineSteps::kRow;
                    ASSERT_EQ(std::memcmp(at, expect.data(), expect.size() * 2), 0)
                        << "sequence " << s << " position " << j * 16 + t << " stream " << st;
                }
            }
        }
    }
}

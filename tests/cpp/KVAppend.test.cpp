// KVAppendBatch: one step's K/V stores through the copy-on-write point, the
// batched form of the reference harnesses' write_head_vector / write_token
// (tests/PagedAttention.test.cpp:97-127, tests/EndToEnd.test.cpp:157-179).
// Device frames (one qvp_append_kv launch per call) must end byte for byte
// where host frames (memcpy, the reference's placement) end, and a decode
// must see exactly what was appended.
#include "device_harness.h"
#include "qwenvl_paged/KVAppend.h"

#include "qvp.h"

#include <map>
#include <random>

using namespace device_test;

namespace {

// Fills `n` tokens x `layers` of K and V rows with a pattern keyed by step and
// token index (elem_bytes-sized elements, as raw bytes).
std::vector<std::uint8_t> rows(std::size_t n, std::uint32_t layers, const BlockShape& s, std::uint32_t step,
                               std::uint32_t stream) {
    const std::size_t bytes = n * layers * s.num_kv_heads * s.head_dim * s.bytes_per_element;
    std::vector<std::uint8_t> out(bytes);
    for (std::size_t i = 0; i < bytes; ++i) out[i] = static_cast<std::uint8_t>((i * 7 + step * 131 + stream * 17) % 251);
    return out;
}

struct DeviceRows {
    void* k{nullptr};
    void* v{nullptr};
    DeviceRows(const std::vector<std::uint8_t>& hk, const std::vector<std::uint8_t>& hv) {
        if (qvp_malloc(&k, hk.size()) != QVP_OK || qvp_malloc(&v, hv.size()) != QVP_OK) return;
        (void)qvp_memcpy_htod(k, hk.data(), hk.size(), nullptr);
        (void)qvp_memcpy_htod(v, hv.data(), hv.size(), nullptr);
        (void)qvp_device_synchronize();
    }
    ~DeviceRows() {
        (void)qvp_free(k);
        (void)qvp_free(v);
    }
};

std::vector<std::uint8_t> frame_bytes(MemoryAllocator& a, PhysicalBlockId id) {
    std::vector<std::uint8_t> out(a.block(id)->size_bytes());
    EXPECT_TRUE(a.read_block_bytes(id, 0, out.data(), out.size()));
    return out;
}

}  // namespace

TEST(KVAppendTest, DeviceAppendsEqualHostAppendsByteForByte) {
    // Random steps over live and forked sequences: each step appends the next
    // token of a random subset (growing tables at block boundaries), sometimes
    // rewrites a token inside a block shared with a fork (copy-on-write), and
    // writes either every layer or a layer range.
    for (const std::uint32_t bpe : {4u, 2u}) {
        const BlockShape shape = shape_of(4, 3, 2, 8, bpe);
        constexpr std::uint32_t kFrames = 40;
        HostHarness host(shape, kFrames);
        DeviceHarness dev(shape, kFrames);
        ASSERT_TRUE(dev.ready());
        const std::vector<std::uint8_t> zero(shape.byte_size(), 0);
        for (PhysicalBlockId f = 0; f < kFrames; ++f) {
            ASSERT_TRUE(host.allocator.write_block_bytes(f, 0, zero.data(), zero.size()));
            ASSERT_TRUE(dev.allocator.write_block_bytes(f, 0, zero.data(), zero.size()));
        }
        KVAppendBatch host_batch, dev_batch;
        std::map<SequenceId, std::uint32_t> length;
        for (SequenceId id = 1; id <= 3; ++id) {
            SequenceMetadata m{id, id, {}, {}};
            ASSERT_TRUE(host.cache.create_sequence(m));
            ASSERT_TRUE(dev.cache.create_sequence(m));
            length[id] = 0;
        }
        std::mt19937 rng(77 + bpe);
        int copies = 0;
        for (std::uint32_t step = 0; step < 40; ++step) {
            if (step == 10 || step == 20) {
                const SequenceId parent = 1 + rng() % 3;
                const SequenceId child = 10 + step;
                SequenceMetadata m{child, parent, {}, {}};
                ASSERT_TRUE(host.cache.fork_sequence(parent, m));
                ASSERT_TRUE(dev.cache.fork_sequence(parent, m));
                length[child] = length[parent];
            }
            std::vector<SequenceId> seqs;
            std::vector<TokenPosition> pos;
            for (const auto& [id, len] : length) {
                if (rng() % 4 == 0) continue;
                TokenPosition p = len;
                if (len > 0 && rng() % 5 == 0) p = rng() % len;  // rewrite an old token
                if (p == len) {
                    if (p / shape.tokens_per_block >= host.cache.cache_view(id)->block_table->size()) {
                        const bool a = host.cache.reserve_tokens(id, 1);
                        ASSERT_EQ(a, dev.cache.reserve_tokens(id, 1));
                        if (!a) continue;
                    }
                }
                seqs.push_back(id);
                pos.push_back(p);
            }
            if (seqs.empty()) continue;
            const std::uint32_t first_layer = step % 3 == 0 ? 1 : 0;
            const std::uint32_t layer_count = step % 3 == 0 ? 2 : 3;
            const auto hk = rows(seqs.size(), layer_count, shape, step, 0);
            const auto hv = rows(seqs.size(), layer_count, shape, step, 1);
            DeviceRows d(hk, hv);
            ASSERT_NE(d.k, nullptr);
            const std::uint64_t launches = dev.allocator.copy_launches();
            const bool a = host_batch.append(host.cache, host.allocator, seqs, pos, first_layer, layer_count,
                                             hk.data(), hv.data());
            const bool b = dev_batch.append(dev.cache, dev.allocator, seqs, pos, first_layer, layer_count, d.k, d.v);
            ASSERT_TRUE(a) << host_batch.last_error();
            ASSERT_TRUE(b) << dev_batch.last_error();
            copies += static_cast<int>(dev.allocator.copy_launches() - launches);
            for (std::size_t i = 0; i < seqs.size(); ++i) length[seqs[i]] = std::max(length[seqs[i]], pos[i] + 1);
            ASSERT_TRUE(dev.allocator.synchronize());
            for (PhysicalBlockId f = 0; f < kFrames; ++f) {
                ASSERT_EQ(frame_bytes(dev.allocator, f), frame_bytes(host.allocator, f))
                    << "bpe " << bpe << " step " << step << " frame " << f;
            }
        }
        EXPECT_GT(copies, 0) << "no step exercised copy-on-write";
    }
}

TEST(KVAppendTest, RefusedCallsWriteNothing) {
    const BlockShape shape = shape_of(4, 2, 2, 8, 2);
    DeviceHarness dev(shape, 8);
    ASSERT_TRUE(dev.ready());
    const std::vector<std::uint8_t> fill(shape.byte_size(), 0x5a);
    for (PhysicalBlockId f = 0; f < 8; ++f) ASSERT_TRUE(dev.allocator.write_block_bytes(f, 0, fill.data(), fill.size()));
    ASSERT_TRUE(dev.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(dev.cache.reserve_tokens(1, 6));
    const auto hk = rows(2, 2, shape, 1, 0);
    const auto hv = rows(2, 2, shape, 1, 1);
    DeviceRows d(hk, hv);
    KVAppendBatch batch;
    EXPECT_FALSE(batch.append(dev.cache, dev.allocator, {1, 1}, {3, 3}, 0, 2, d.k, d.v));   // token twice
    EXPECT_FALSE(batch.append(dev.cache, dev.allocator, {1, 1}, {3, 8}, 0, 2, d.k, d.v));   // unmapped block
    EXPECT_FALSE(batch.append(dev.cache, dev.allocator, {1, 2}, {3, 0}, 0, 2, d.k, d.v));   // unknown sequence
    EXPECT_FALSE(batch.append(dev.cache, dev.allocator, {1, 1}, {3, 4}, 1, 2, d.k, d.v));   // layers past the shape
    EXPECT_FALSE(batch.append(dev.cache, dev.allocator, {1, 1}, {3, 4}, 0, 0, d.k, d.v));   // no layer
    EXPECT_FALSE(batch.append(dev.cache, dev.allocator, {1, 1}, {3, 4}, 0, 2, nullptr, d.v));
    EXPECT_FALSE(batch.append(dev.cache, dev.allocator, {1}, {3, 4}, 0, 2, d.k, d.v));      // sizes differ
    EXPECT_FALSE(batch.last_error().empty());
    ASSERT_TRUE(dev.allocator.synchronize());
    for (PhysicalBlockId f = 0; f < 8; ++f) {
        EXPECT_EQ(frame_bytes(dev.allocator, f), fill) << "frame " << f;
    }
    EXPECT_TRUE(batch.append(dev.cache, dev.allocator, {}, {}, 0, 2, d.k, d.v));  // empty step
}

TEST(KVAppendTest, DecodeSeesEveryTokenTheBatchAppended) {
    // Three sequences grow one token per step, all layers appended by one call
    // per step; after each step every sequence's decode of every layer equals
    // float64 textbook attention over the values written so far. Two of them
    // are forks of the first, diverging at a shared block.
    constexpr std::uint32_t kTpb = 4, kLayers = 2, kKv = 2, kDim = 8, kHeads = 4;
    const BlockShape shape = shape_of(kTpb, kLayers, kKv, kDim, 4);
    DeviceHarness dev(shape, 32);
    ASSERT_TRUE(dev.ready());
    auto value = [](SequenceId writer, std::uint32_t layer, std::uint32_t s, std::uint32_t t, std::uint32_t h,
                    std::uint32_t dd) { return mix_pattern({std::uint32_t(writer), layer, s, t, h, dd}); };
    std::map<SequenceId, std::vector<SequenceId>> owner;
    KVAppendBatch batch;
    auto step = [&](const std::vector<SequenceId>& seqs, const std::vector<TokenPosition>& pos) {
        std::vector<float> k(seqs.size() * kLayers * kKv * kDim), v(k.size());
        for (std::size_t i = 0; i < seqs.size(); ++i) {
            for (std::uint32_t l = 0; l < kLayers; ++l)
                for (std::uint32_t h = 0; h < kKv; ++h)
                    for (std::uint32_t dd = 0; dd < kDim; ++dd) {
                        const std::size_t at = ((i * kLayers + l) * kKv + h) * kDim + dd;
                        k[at] = value(seqs[i], l, 0, pos[i], h, dd);
                        v[at] = value(seqs[i], l, 1, pos[i], h, dd);
                    }
            auto& own = owner[seqs[i]];
            own.resize(std::max<std::size_t>(own.size(), pos[i] + 1));
            own[pos[i]] = seqs[i];
        }
        DeviceRows d(std::vector<std::uint8_t>(reinterpret_cast<const std::uint8_t*>(k.data()),
                                               reinterpret_cast<const std::uint8_t*>(k.data() + k.size())),
                     std::vector<std::uint8_t>(reinterpret_cast<const std::uint8_t*>(v.data()),
                                               reinterpret_cast<const std::uint8_t*>(v.data() + v.size())));
        ASSERT_TRUE(batch.append(dev.cache, dev.allocator, seqs, pos, 0, kLayers, d.k, d.v)) << batch.last_error();
        ASSERT_TRUE(dev.allocator.synchronize());
    };
    auto check = [&](SequenceId seq, std::uint32_t ctx) {
        const auto view = dev.cache.cache_view(seq);
        ASSERT_TRUE(view.has_value());
        std::vector<float> q(kHeads * kDim);
        for (std::uint32_t i = 0; i < q.size(); ++i) q[i] = mix_pattern({std::uint32_t(seq), 5u, ctx, i});
        const auto& own = owner[seq];
        for (std::uint32_t layer = 0; layer < kLayers; ++layer) {
            PagedAttentionParams p;
            p.layer = layer;
            p.num_query_heads = kHeads;
            p.context_len = ctx;
            p.scale = 0.35f;
            std::vector<float> out(q.size());
            ASSERT_TRUE(paged_attention_decode<float>(*view, q.data(), p, out.data())) << paged_attention_last_error();
            const auto expect = textbook_attention(
                q, kHeads, kKv, kDim, ctx, 0.35f, [&](auto t, auto h, auto dd) { return value(own[t], layer, 0, t, h, dd); },
                [&](auto t, auto h, auto dd) { return value(own[t], layer, 1, t, h, dd); });
            for (std::size_t i = 0; i < out.size(); ++i) {
                ASSERT_NEAR(out[i], expect[i], 1e-5) << "seq " << seq << " ctx " << ctx << " layer " << layer;
            }
        }
    };
    ASSERT_TRUE(dev.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    for (TokenPosition p = 0; p < 6; ++p) {
        if (p % kTpb == 0) {
            ASSERT_TRUE(dev.cache.reserve_tokens(1, 1));
        }
        ASSERT_NO_FATAL_FAILURE(step({1}, {p}));
    }
    for (SequenceId b : {2, 3}) {
        ASSERT_TRUE(dev.cache.fork_sequence(1, SequenceMetadata{b, 1, {}, {}}));
        owner[b] = owner[1];
    }
    // Both forks rewrite token 5 in the block they share with the parent (one
    // call, two copies), then all three grow together.
    ASSERT_NO_FATAL_FAILURE(step({2, 3}, {5, 5}));
    for (TokenPosition p = 6; p < 11; ++p) {
        for (SequenceId s : {1, 2, 3}) {
            if (p % kTpb == 0) {
                ASSERT_TRUE(dev.cache.reserve_tokens(s, 1));
            }
        }
        ASSERT_NO_FATAL_FAILURE(step({1, 2, 3}, {p, p, p}));
        for (SequenceId s : {1, 2, 3}) ASSERT_NO_FATAL_FAILURE(check(s, p + 1));
    }
    const PhysicalBlockId shared = *dev.cache.cache_view(1)->block_table->lookup(0);
    for (SequenceId b : {2, 3}) EXPECT_EQ(*dev.cache.cache_view(b)->block_table->lookup(0), shared);
}

TEST(KVAppendTest, StepCopiesJoinTheAppendLaunchUnlessARowGoesIntoACopySource) {
    // Forks whose next token lands in the block they share with their parent:
    // every fork's copy runs inside the append's own launch (one copy launch
    // counted, nothing left queued). In the second form the parent writes into
    // the shared frame in the same step as its forks copy it -- a row into a
    // copy's source -- and the copies run first, as their own launch. Both
    // forms end byte for byte where host frames (memcpy) end.
    for (const bool parent_writes : {false, true}) {
        const BlockShape shape = shape_of(4, 2, 2, 8, 2);
        constexpr std::uint32_t kFrames = 24;
        HostHarness host(shape, kFrames);
        DeviceHarness dev(shape, kFrames);
        ASSERT_TRUE(dev.ready());
        std::vector<std::uint8_t> fill(shape.byte_size());
        for (PhysicalBlockId f = 0; f < kFrames; ++f) {
            for (std::size_t i = 0; i < fill.size(); ++i) fill[i] = static_cast<std::uint8_t>((i * 13 + f * 29) % 251);
            ASSERT_TRUE(host.allocator.write_block_bytes(f, 0, fill.data(), fill.size()));
            ASSERT_TRUE(dev.allocator.write_block_bytes(f, 0, fill.data(), fill.size()));
        }
        for (auto* cache : {&host.cache, &dev.cache}) {
            ASSERT_TRUE(cache->create_sequence(SequenceMetadata{1, 1, {}, {}}));
            ASSERT_TRUE(cache->reserve_tokens(1, 6));  // block 1 holds tokens 4, 5 and room for 6, 7
            for (SequenceId b : {2, 3, 4}) ASSERT_TRUE(cache->fork_sequence(1, SequenceMetadata{b, 1, {}, {}}));
        }
        std::vector<SequenceId> seqs{2, 3, 4};
        std::vector<TokenPosition> pos{6, 6, 6};
        if (parent_writes) {
            seqs.push_back(1);
            pos.push_back(6);
        }
        const auto hk = rows(seqs.size(), 2, shape, 3, 0);
        const auto hv = rows(seqs.size(), 2, shape, 3, 1);
        DeviceRows d(hk, hv);
        ASSERT_NE(d.k, nullptr);
        KVAppendBatch host_batch, dev_batch;
        const std::uint64_t launches = dev.allocator.copy_launches();
        ASSERT_TRUE(host_batch.append(host.cache, host.allocator, seqs, pos, 0, 2, hk.data(), hv.data()))
            << host_batch.last_error();
        ASSERT_TRUE(dev_batch.append(dev.cache, dev.allocator, seqs, pos, 0, 2, d.k, d.v)) << dev_batch.last_error();
        EXPECT_EQ(dev.allocator.pending_operations(), 0u);
        EXPECT_EQ(dev.allocator.copy_launches() - launches, 1u) << "parent_writes " << parent_writes;
        ASSERT_TRUE(dev.allocator.synchronize());
        for (PhysicalBlockId f = 0; f < kFrames; ++f) {
            ASSERT_EQ(frame_bytes(dev.allocator, f), frame_bytes(host.allocator, f))
                << "parent_writes " << parent_writes << " frame " << f;
        }
        // The forks own their tail frames now; the parent keeps the original.
        const PhysicalBlockId tail = *dev.cache.cache_view(1)->block_table->lookup(1);
        for (SequenceId b : {2, 3, 4}) EXPECT_NE(*dev.cache.cache_view(b)->block_table->lookup(1), tail);
    }
}

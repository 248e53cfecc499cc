// Element layout inside a block and the read contract CacheView
// (include/qwenvl_paged/CacheLayout.h, KVCacheManager.h of the reference;
// tests/CacheView.test.cpp:103-332 states the same rules). The decode kernels
// take exactly these strides, so the layout is also checked in bytes against
// the shapes of the benchmark configurations.
#include "minitest.h"
#include "qwenvl_paged/CacheLayout.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/SwapBackend.h"

#include <cstring>
#include <vector>

using namespace qwenvl_paged;

namespace {

BlockShape shape_of(std::uint32_t tpb, std::uint32_t layers, std::uint32_t heads, std::uint32_t dim,
                    std::uint32_t bpe) {
    BlockShape s;
    s.tokens_per_block = tpb;
    s.num_layers = layers;
    s.num_kv_heads = heads;
    s.head_dim = dim;
    s.bytes_per_element = bpe;
    return s;
}

constexpr std::uint32_t kTpb = 4, kLayers = 2, kHeads = 2, kDim = 4;

KVBlockLayout small_layout() { return KVBlockLayout{shape_of(kTpb, kLayers, kHeads, kDim, 4)}; }

// Writes a head vector filled with `value` through the copy-on-write point,
// the way an attention backend appends K or V.
bool put_vector(KVCacheManager& cache, MemoryAllocator& alloc, SequenceId seq, KVStream stream, std::uint32_t layer,
                TokenPosition token, std::uint32_t head, float value) {
    const auto frame = cache.ensure_token_writable(seq, token);
    if (!frame) return false;
    const KVBlockLayout layout{alloc.block(*frame)->shape()};
    const auto off = layout.element_offset(layer, stream, token % layout.shape.tokens_per_block, head);
    if (!off) return false;
    float* dst = reinterpret_cast<float*>(alloc.block(*frame)->data()) + *off;
    for (std::uint32_t d = 0; d < layout.shape.head_dim; ++d) dst[d] = value;
    return true;
}

class CacheViewTest : public testing::Test {
protected:
    CacheViewTest() : alloc_(make_config()), cache_(alloc_) {}

    static AllocatorConfig make_config() {
        AllocatorConfig c;
        c.block_shape = shape_of(kTpb, kLayers, kHeads, kDim, 4);
        c.max_blocks = 8;
        return c;
    }

    void SetUp() override {
        ASSERT_TRUE(cache_.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    }

    MemoryAllocator alloc_;
    KVCacheManager cache_;
};

}  // namespace

TEST(KVBlockLayoutTest, StridesNestLayerStreamTokenHead) {
    const KVBlockLayout l = small_layout();
    EXPECT_EQ(l.head_stride(), kDim);
    EXPECT_EQ(l.token_stride(), kHeads * kDim);
    EXPECT_EQ(l.stream_stride(), kTpb * kHeads * kDim);
    EXPECT_EQ(l.layer_stride(), 2u * kTpb * kHeads * kDim);
    EXPECT_EQ(l.element_count(), kLayers * l.layer_stride());
    EXPECT_EQ(l.element_count() * 4u, l.shape.byte_size());
}

TEST(KVBlockLayoutTest, ByteStridesOfTheBenchmarkShapes) {
    struct Case {
        BlockShape shape;
        std::size_t head, token, stream, layer;
    };
    const Case cases[] = {
        {shape_of(16, 1, 2, 64, 4), 256, 512, 8192, 16384},    // fp32, Hkv2, D64
        {shape_of(16, 1, 4, 128, 2), 256, 1024, 16384, 32768},  // bf16, Hkv4, D128
        {shape_of(16, 1, 8, 128, 2), 256, 2048, 32768, 65536},  // bf16, Hkv8, D128
    };
    for (const Case& c : cases) {
        const KVBlockLayout l{c.shape};
        const std::size_t bpe = c.shape.bytes_per_element;
        EXPECT_EQ(l.head_stride() * bpe, c.head);
        EXPECT_EQ(l.token_stride() * bpe, c.token);
        EXPECT_EQ(l.stream_stride() * bpe, c.stream);
        EXPECT_EQ(l.layer_stride() * bpe, c.layer);
        EXPECT_EQ(l.element_count() * bpe, c.shape.byte_size());
    }
}

TEST(KVBlockLayoutTest, OffsetIsTheClosedFormAndCoversTheBlockExactlyOnce) {
    for (const BlockShape& s : {shape_of(4, 2, 2, 4, 4), shape_of(3, 3, 1, 5, 2), shape_of(16, 2, 4, 8, 2)}) {
        const KVBlockLayout l{s};
        std::vector<int> hits(l.element_count(), 0);
        for (std::uint32_t layer = 0; layer < s.num_layers; ++layer) {
            for (std::uint32_t st = 0; st < 2; ++st) {
                const KVStream stream = st == 0 ? KVStream::Key : KVStream::Value;
                for (std::uint32_t t = 0; t < s.tokens_per_block; ++t) {
                    for (std::uint32_t h = 0; h < s.num_kv_heads; ++h) {
                        const auto off = l.element_offset(layer, stream, t, h);
                        ASSERT_TRUE(off.has_value());
                        const std::size_t expect =
                            ((static_cast<std::size_t>(layer) * 2 + st) * s.tokens_per_block + t) * s.num_kv_heads *
                                s.head_dim +
                            static_cast<std::size_t>(h) * s.head_dim;
                        EXPECT_EQ(*off, expect);
                        for (std::uint32_t d = 0; d < s.head_dim; ++d) {
                            ASSERT_LT(*off + d, hits.size());
                            hits[*off + d] += 1;
                        }
                    }
                }
            }
        }
        for (std::size_t i = 0; i < hits.size(); ++i) ASSERT_EQ(hits[i], 1) << "element " << i;
    }
}

TEST(KVBlockLayoutTest, OutOfRangeCoordinatesHaveNoOffset) {
    const KVBlockLayout l = small_layout();
    EXPECT_FALSE(l.element_offset(kLayers, KVStream::Key, 0, 0).has_value());
    EXPECT_FALSE(l.element_offset(0, KVStream::Value, kTpb, 0).has_value());
    EXPECT_FALSE(l.element_offset(0, KVStream::Key, 0, kHeads).has_value());
    EXPECT_TRUE(l.element_offset(kLayers - 1, KVStream::Value, kTpb - 1, kHeads - 1).has_value());
}

TEST(CacheViewStaticTest, DefaultViewIsInvalidAndResolvesNothing) {
    const CacheView v;
    EXPECT_FALSE(v.valid());
    EXPECT_EQ(v.block_bytes(0), nullptr);
    EXPECT_EQ(v.slot<float>(KVStream::Key, 0, 0, 0), nullptr);
}

TEST_F(CacheViewTest, ViewDescribesTheSequence) {
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));
    const auto v = cache_.cache_view(1);
    ASSERT_TRUE(v.has_value());
    EXPECT_TRUE(v->valid());
    EXPECT_EQ(v->sequence_id, 1u);
    EXPECT_EQ(v->allocator, &alloc_);
    ASSERT_NE(v->block_table, nullptr);
    EXPECT_EQ(v->layout.shape.tokens_per_block, kTpb);
    EXPECT_EQ(v->layout.shape.head_dim, kDim);
    EXPECT_FALSE(cache_.cache_view(99).has_value());
}

TEST_F(CacheViewTest, BlockBytesAreTheMappedFrames) {
    ASSERT_TRUE(cache_.reserve_tokens(1, 3 * kTpb));
    const auto v = cache_.cache_view(1);
    for (LogicalBlockIndex i = 0; i < 3; ++i) {
        const auto frame = v->block_table->lookup(i);
        ASSERT_TRUE(frame.has_value());
        EXPECT_EQ(v->block_bytes(i), alloc_.block(*frame)->data());
    }
    EXPECT_EQ(v->block_bytes(3), nullptr);
}

TEST_F(CacheViewTest, SwappedOutBlockResolvesToNothing) {
    HostSwapBackend swap(4);
    alloc_.set_swap_backend(&swap);
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));
    ASSERT_EQ(cache_.swap_out_sequence(1), 1u);
    const auto v = cache_.cache_view(1);
    EXPECT_EQ(v->block_bytes(0), nullptr);
    EXPECT_EQ(v->slot<float>(KVStream::Value, 0, 0, 0), nullptr);
    ASSERT_TRUE(cache_.swap_in_sequence(1));
    EXPECT_NE(cache_.cache_view(1)->block_bytes(0), nullptr);
}

TEST_F(CacheViewTest, SlotWalksTokensAcrossBlocks) {
    constexpr std::uint32_t kTokens = 3 * kTpb - 1;
    ASSERT_TRUE(cache_.reserve_tokens(1, kTokens));
    for (TokenPosition t = 0; t < kTokens; ++t) {
        ASSERT_TRUE(put_vector(cache_, alloc_, 1, KVStream::Key, 1, t, 1, 0.5F + static_cast<float>(t)));
    }
    const auto v = cache_.cache_view(1);
    for (TokenPosition t = 0; t < kTokens; ++t) {
        const float* k = v->slot<float>(KVStream::Key, 1, t, 1);
        ASSERT_NE(k, nullptr) << "token " << t;
        for (std::uint32_t d = 0; d < kDim; ++d) EXPECT_FLOAT_EQ(k[d], 0.5F + static_cast<float>(t));
    }
}

TEST_F(CacheViewTest, StreamsLayersAndHeadsAreSeparate) {
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));
    ASSERT_TRUE(put_vector(cache_, alloc_, 1, KVStream::Key, 0, 2, 0, 1.0F));
    ASSERT_TRUE(put_vector(cache_, alloc_, 1, KVStream::Value, 0, 2, 0, 2.0F));
    ASSERT_TRUE(put_vector(cache_, alloc_, 1, KVStream::Key, 1, 2, 0, 3.0F));
    ASSERT_TRUE(put_vector(cache_, alloc_, 1, KVStream::Key, 0, 2, 1, 4.0F));
    ASSERT_TRUE(put_vector(cache_, alloc_, 1, KVStream::Key, 0, 3, 0, 5.0F));
    const auto v = cache_.cache_view(1);
    EXPECT_FLOAT_EQ(v->slot<float>(KVStream::Key, 0, 2, 0)[0], 1.0F);
    EXPECT_FLOAT_EQ(v->slot<float>(KVStream::Value, 0, 2, 0)[0], 2.0F);
    EXPECT_FLOAT_EQ(v->slot<float>(KVStream::Key, 1, 2, 0)[0], 3.0F);
    EXPECT_FLOAT_EQ(v->slot<float>(KVStream::Key, 0, 2, 1)[0], 4.0F);
    EXPECT_FLOAT_EQ(v->slot<float>(KVStream::Key, 0, 3, 0)[0], 5.0F);
}

TEST_F(CacheViewTest, SlotRefusesAWrongElementSizeAndOutOfRangeCoordinates) {
    ASSERT_TRUE(cache_.reserve_tokens(1, kTpb));
    const auto v = cache_.cache_view(1);
    EXPECT_EQ(v->slot<double>(KVStream::Key, 0, 0, 0), nullptr);
    EXPECT_EQ(v->slot<std::uint16_t>(KVStream::Key, 0, 0, 0), nullptr);
    EXPECT_NE(v->slot<float>(KVStream::Key, 0, 0, 0), nullptr);
    EXPECT_EQ(v->slot<float>(KVStream::Key, kLayers, 0, 0), nullptr);
    EXPECT_EQ(v->slot<float>(KVStream::Key, 0, 0, kHeads), nullptr);
    // Token kTpb lives in logical block 1, which is not mapped.
    EXPECT_EQ(v->slot<float>(KVStream::Key, 0, kTpb, 0), nullptr);
}

TEST_F(CacheViewTest, ForkSharesThenCopyOnWriteSeparates) {
    ASSERT_TRUE(cache_.reserve_tokens(1, 2 * kTpb));
    ASSERT_TRUE(put_vector(cache_, alloc_, 1, KVStream::Key, 0, 0, 0, 7.0F));
    ASSERT_TRUE(put_vector(cache_, alloc_, 1, KVStream::Value, 1, kTpb + 1, 1, 8.0F));
    ASSERT_TRUE(cache_.fork_sequence(1, SequenceMetadata{2, 1, {}, {}}));
    EXPECT_EQ(cache_.cache_view(1)->slot<float>(KVStream::Key, 0, 0, 0),
              cache_.cache_view(2)->slot<float>(KVStream::Key, 0, 0, 0));

    // The child writes token 0: block 0 is copied, block 1 stays shared.
    ASSERT_TRUE(put_vector(cache_, alloc_, 2, KVStream::Key, 0, 0, 0, 9.0F));
    const auto parent = cache_.cache_view(1);
    const auto child = cache_.cache_view(2);
    const float* p0 = parent->slot<float>(KVStream::Key, 0, 0, 0);
    const float* c0 = child->slot<float>(KVStream::Key, 0, 0, 0);
    ASSERT_NE(p0, nullptr);
    ASSERT_NE(c0, nullptr);
    EXPECT_NE(p0, c0);
    EXPECT_FLOAT_EQ(p0[0], 7.0F);
    EXPECT_FLOAT_EQ(c0[0], 9.0F);
    EXPECT_EQ(parent->block_bytes(1), child->block_bytes(1));
    // The copy carried the whole frame, so the other streams came along.
    EXPECT_FLOAT_EQ(child->slot<float>(KVStream::Value, 1, kTpb + 1, 1)[0], 8.0F);
}

// Contract of the core block types (include/qwenvl_paged/Block.h of the
// reference; its suite tests/Block.test.cpp:35-140 states the same properties).
#include "minitest.h"
#include "qwenvl_paged/Block.h"

#include <cstdint>
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

BlockShape small_shape() { return shape_of(4, 2, 2, 8, 2); }

}  // namespace

TEST(BlockShapeTest, ByteSizeIsTheProductOfEveryDimensionTimesTwoStreams) {
    EXPECT_EQ(small_shape().byte_size(), 4u * 2u * 2u * 8u * 2u * 2u);
    // Shapes of the benchmark configurations (single layer): fp32 Hkv2/D64,
    // Qwen2-VL-7B and -72B bf16 with 16 tokens per block.
    EXPECT_EQ(shape_of(16, 1, 2, 64, 4).byte_size(), 16384u);
    EXPECT_EQ(shape_of(16, 1, 4, 128, 2).byte_size(), 32768u);
    EXPECT_EQ(shape_of(16, 1, 8, 128, 2).byte_size(), 65536u);
    EXPECT_EQ(shape_of(16, 28, 4, 128, 2).byte_size(), 917504u);
}

TEST(BlockShapeTest, ByteSizeIsLinearInEachDimension) {
    const std::size_t base = small_shape().byte_size();
    ASSERT_GT(base, 0u);
    for (int dim = 0; dim < 5; ++dim) {
        BlockShape s = small_shape();
        std::uint32_t* fields[] = {&s.tokens_per_block, &s.num_layers, &s.num_kv_heads, &s.head_dim,
                                   &s.bytes_per_element};
        *fields[dim] *= 3;
        EXPECT_EQ(s.byte_size(), base * 3) << "dimension " << dim;
    }
}

TEST(BlockShapeTest, ZeroDimensionGivesZeroBytes) {
    BlockShape s = small_shape();
    s.head_dim = 0;
    EXPECT_EQ(s.byte_size(), 0u);
}

TEST(LogicalBlockTest, EmptyMeansNoCommittedTokens) {
    LogicalBlock block;
    EXPECT_TRUE(block.empty());
    block.token_count = 1;
    EXPECT_FALSE(block.empty());
    block.token_count = 0;
    block.start_token = 64;
    EXPECT_TRUE(block.empty());
}

TEST(PhysicalBlockTest, KeepsItsIdShapeAndOptions) {
    HostMemoryOptions options;
    options.prefer_pinned_memory = true;
    PhysicalBlock block(11, small_shape(), options);
    EXPECT_EQ(block.id(), 11u);
    EXPECT_EQ(block.shape().byte_size(), small_shape().byte_size());
    EXPECT_TRUE(block.pinned_memory_requested());
    EXPECT_EQ(block.placement(), BlockPlacement::Host);
    PhysicalBlock plain(12, small_shape());
    EXPECT_FALSE(plain.pinned_memory_requested());
}

TEST(PhysicalBlockTest, EveryLiveBlockIsAligned) {
    // Many blocks alive at once, so an allocator that ignores the alignment
    // fails with near certainty.
    for (std::size_t alignment : {std::size_t{64}, std::size_t{256}, std::size_t{4096}}) {
        HostMemoryOptions options;
        options.alignment_bytes = alignment;
        std::vector<PhysicalBlock> blocks;
        blocks.reserve(48);
        for (std::uint32_t i = 0; i < 48; ++i) blocks.emplace_back(i, small_shape(), options);
        for (const PhysicalBlock& b : blocks) {
            ASSERT_NE(b.data(), nullptr);
            EXPECT_EQ(b.alignment_bytes(), alignment);
            EXPECT_EQ(reinterpret_cast<std::uintptr_t>(b.data()) % alignment, 0u);
        }
    }
}

TEST(PhysicalBlockTest, SizeIsByteSizeRoundedUpToTheAlignment) {
    HostMemoryOptions options;
    options.alignment_bytes = 256;
    // 4*1*1*8*4*2 = 256 exactly; 3*1*1*8*4*2 = 192 -> 256; 5*... = 320 -> 512.
    EXPECT_EQ(PhysicalBlock(0, shape_of(4, 1, 1, 8, 4), options).size_bytes(), 256u);
    EXPECT_EQ(PhysicalBlock(0, shape_of(3, 1, 1, 8, 4), options).size_bytes(), 256u);
    EXPECT_EQ(PhysicalBlock(0, shape_of(5, 1, 1, 8, 4), options).size_bytes(), 512u);
}

TEST(PhysicalBlockTest, ZeroAlignmentUsesTheDefaultButReportsZero) {
    HostMemoryOptions options;
    options.alignment_bytes = 0;
    PhysicalBlock block(0, shape_of(3, 1, 1, 8, 4), options);
    EXPECT_EQ(block.alignment_bytes(), 0u);
    EXPECT_EQ(block.size_bytes(), kDefaultBlockAlignmentBytes);
    EXPECT_EQ(reinterpret_cast<std::uintptr_t>(block.data()) % kDefaultBlockAlignmentBytes, 0u);
}

TEST(PhysicalBlockTest, ZeroByteShapeStillGetsStorage) {
    BlockShape s = small_shape();
    s.num_layers = 0;
    PhysicalBlock block(0, s);
    EXPECT_NE(block.data(), nullptr);
    EXPECT_GT(block.size_bytes(), 0u);
}

TEST(PhysicalBlockTest, SwapExchangesStorageButNotIds) {
    PhysicalBlock a(1, small_shape());
    PhysicalBlock b(2, small_shape());
    for (std::size_t i = 0; i < a.size_bytes(); ++i) {
        a.data()[i] = static_cast<std::byte>(i * 7 + 1);
        b.data()[i] = static_cast<std::byte>(i * 5 + 3);
    }
    const std::byte* a_storage = a.data();
    a.swap(b);
    EXPECT_EQ(a.id(), 1u);
    EXPECT_EQ(b.id(), 2u);
    EXPECT_EQ(b.data(), a_storage);
    for (std::size_t i = 0; i < a.size_bytes(); ++i) {
        EXPECT_EQ(a.data()[i], static_cast<std::byte>(i * 5 + 3));
        EXPECT_EQ(b.data()[i], static_cast<std::byte>(i * 7 + 1));
    }
}

TEST(PhysicalBlockTest, DeviceFrameViewDoesNotOwnItsFrame) {
    alignas(256) static std::byte frame[512];
    {
        PhysicalBlock view(3, small_shape(), HostMemoryOptions{}, frame, sizeof frame);
        EXPECT_EQ(view.placement(), BlockPlacement::Device);
        EXPECT_EQ(view.data(), frame);
        EXPECT_EQ(view.size_bytes(), sizeof frame);
    }
    // Destroying the view left the static storage alone (a free() of it
    // would have aborted the process).
    frame[0] = std::byte{1};
    EXPECT_EQ(frame[0], std::byte{1});
}

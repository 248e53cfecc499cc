// MRopePositionBatch: M-RoPE position ids from the PositionalEncodingSpan
// metadata a sequence was created with (include/qwenvl_paged/
// KVCacheManager.h:23-78). Expected values are Qwen2-VL's own for the prompt
// "5 text tokens, one 4x6-patch image (2x3 after the 2x2 merge), 4 text
// tokens", as transformers' get_rope_index writes them (the first case of
// tests/golden/mrope_positions.json), and their decode continuation
// p + rope_delta (rope_delta = -3).
#include "device_harness.h"
#include "qwenvl_paged/MRope.h"

#include "qvp.h"

using namespace device_test;

namespace {

PositionalEncodingSpan span(TokenPosition start, std::uint32_t count, PositionEncodingKind kind, std::int64_t at,
                            Position3D grid = {}) {
    PositionalEncodingSpan s;
    s.start_token = start;
    s.token_count = count;
    s.kind = kind;
    s.origin = {at, at, at};
    s.stride = {1, 1, 1};
    s.grid = grid;
    return s;
}

std::vector<std::int64_t> read_back(const void* device, std::size_t n) {
    std::vector<std::int64_t> out(n);
    EXPECT_EQ(qvp_memcpy_dtoh(out.data(), device, n * sizeof(std::int64_t), nullptr), QVP_OK);
    EXPECT_EQ(qvp_device_synchronize(), QVP_OK);
    return out;
}

const std::vector<std::int64_t> kT = {0, 1, 2, 3, 4, 5, 5, 5, 5, 5, 5, 8, 9, 10, 11, 12, 13, 14};
const std::vector<std::int64_t> kH = {0, 1, 2, 3, 4, 5, 5, 5, 6, 6, 6, 8, 9, 10, 11, 12, 13, 14};
const std::vector<std::int64_t> kW = {0, 1, 2, 3, 4, 5, 6, 7, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14};

}  // namespace

TEST(MRopeTest, QwenPromptPositionsAndDecodeContinuation) {
    DeviceHarness dev(shape_of(16, 1, 1, 8), 8);
    ASSERT_TRUE(dev.ready());
    // Sequence 1 spells every run out as get_rope_index does; sequence 2
    // leaves its text runs uncovered (the continuation rule gives the same
    // positions for an image); sequence 3 is a fork of 1 with its own copy of
    // the metadata.
    SequenceMetadata a{1, 1, {}, {}};
    a.positional_encoding.spans = {span(0, 5, PositionEncodingKind::Text1D, 0),
                                   span(5, 6, PositionEncodingKind::Image2D, 5, {1, 2, 3}),
                                   span(11, 4, PositionEncodingKind::Text1D, 8)};
    SequenceMetadata b{2, 2, {}, {}};
    b.positional_encoding.spans = {span(5, 6, PositionEncodingKind::Image2D, 5, {1, 2, 3})};
    ASSERT_TRUE(dev.cache.create_sequence(a));
    ASSERT_TRUE(dev.cache.create_sequence(b));
    SequenceMetadata c = a;
    c.sequence_id = 3;
    ASSERT_TRUE(dev.cache.fork_sequence(1, c));

    void* out = nullptr;
    ASSERT_EQ(qvp_malloc(&out, 3 * 64 * sizeof(std::int64_t)), QVP_OK);
    MRopePositionBatch batch;
    // Whole prompts plus three decode tokens for 1 and 2; the decode token 15
    // alone for the fork.
    ASSERT_TRUE(batch.materialise(dev.cache, {1, 2, 3}, {0, 0, 15}, {18, 18, 16}, static_cast<std::int64_t*>(out),
                                  nullptr))
        << batch.last_error();
    const std::size_t rows = 18 + 18 + 1;
    const auto got = read_back(out, 3 * rows);
    for (std::size_t r = 0; r < rows; ++r) {
        const std::size_t p = r < 36 ? r % 18 : 15;
        EXPECT_EQ(got[r], kT[p]) << "row " << r;
        EXPECT_EQ(got[rows + r], kH[p]) << "row " << r;
        EXPECT_EQ(got[2 * rows + r], kW[p]) << "row " << r;
    }
    ASSERT_EQ(qvp_free(out), QVP_OK);
}

TEST(MRopeTest, RefusalsEnqueueNothing) {
    DeviceHarness dev(shape_of(16, 1, 1, 8), 8);
    ASSERT_TRUE(dev.ready());
    // An Image2D span without a grid (a reference-style span) cannot be placed.
    SequenceMetadata a{1, 1, {}, {}};
    a.positional_encoding.spans = {span(2, 6, PositionEncodingKind::Image2D, 2)};
    SequenceMetadata b{2, 2, {}, {}};
    b.positional_encoding.spans = {span(0, 4, PositionEncodingKind::Text1D, 0),
                                   span(3, 4, PositionEncodingKind::Text1D, 9)};  // overlapping
    SequenceMetadata c{3, 3, {}, {}};
    ASSERT_TRUE(dev.cache.create_sequence(a));
    ASSERT_TRUE(dev.cache.create_sequence(b));
    ASSERT_TRUE(dev.cache.create_sequence(c));
    void* out = nullptr;
    ASSERT_EQ(qvp_malloc(&out, 3 * 16 * sizeof(std::int64_t)), QVP_OK);
    const std::vector<std::uint8_t> fill(3 * 16 * sizeof(std::int64_t), 0x5a);
    ASSERT_EQ(qvp_memcpy_htod(out, fill.data(), fill.size(), nullptr), QVP_OK);
    ASSERT_EQ(qvp_device_synchronize(), QVP_OK);
    auto* o = static_cast<std::int64_t*>(out);
    MRopePositionBatch batch;
    EXPECT_FALSE(batch.materialise(dev.cache, {1}, {0}, {8}, o, nullptr));
    EXPECT_FALSE(batch.materialise(dev.cache, {2}, {0}, {8}, o, nullptr));
    EXPECT_FALSE(batch.materialise(dev.cache, {9}, {0}, {8}, o, nullptr));     // unknown sequence
    EXPECT_FALSE(batch.materialise(dev.cache, {3}, {5}, {4}, o, nullptr));     // begin > end
    EXPECT_FALSE(batch.materialise(dev.cache, {3, 3}, {0}, {4}, o, nullptr));  // sizes differ
    EXPECT_FALSE(batch.last_error().empty());
    std::vector<std::uint8_t> after(fill.size());
    ASSERT_EQ(qvp_memcpy_dtoh(after.data(), out, after.size(), nullptr), QVP_OK);
    ASSERT_EQ(qvp_device_synchronize(), QVP_OK);
    EXPECT_EQ(after, fill);
    // A sequence with no spans numbers its tokens 0, 1, 2, ... on every axis.
    ASSERT_TRUE(batch.materialise(dev.cache, {3}, {4}, {8}, o, nullptr)) << batch.last_error();
    const auto got = read_back(out, 12);
    for (int x = 0; x < 3; ++x)
        for (int r = 0; r < 4; ++r) EXPECT_EQ(got[x * 4 + r], 4 + r);
    ASSERT_EQ(qvp_free(out), QVP_OK);
}

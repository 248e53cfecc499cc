// paged_attention_decode<T> (float, bf16, f16; device frames and host frames)
// and PagedAttentionBatch, held to the reference's contract (include/qwenvl_paged/PagedAttention.h:53-127; its
// suite tests/PagedAttention.test.cpp:255-566 states the same refusals and the
// same closed-form cases). Expected values are float64 textbook attention; the
// fp32 tolerance is 1e-5 absolute, bf16 outputs are checked against the
// float64 result with 2e-3 absolute plus one bf16 rounding step.
#include "device_harness.h"

#include "qvp.h"

#include <random>

using namespace device_test;

namespace {

constexpr float kF32Tol = 1e-5f;

PagedAttentionParams params(std::uint32_t layer, std::uint32_t heads, std::uint32_t ctx, float scale) {
    PagedAttentionParams p;
    p.layer = layer;
    p.num_query_heads = heads;
    p.context_len = ctx;
    p.scale = scale;
    return p;
}

float pat(std::uint32_t layer, KVStream s, std::uint32_t token, std::uint32_t head, std::uint32_t dim) {
    return mix_pattern({layer, s == KVStream::Key ? 0u : 1u, token, head, dim});
}

template <typename Harness>
bool fill_pattern(Harness& h, SequenceId seq, std::uint32_t ctx) {
    const BlockShape& s = h.layout.shape;
    for (std::uint32_t layer = 0; layer < s.num_layers; ++layer) {
        for (KVStream st : {KVStream::Key, KVStream::Value}) {
            for (std::uint32_t t = 0; t < ctx; ++t) {
                for (std::uint32_t hd = 0; hd < s.num_kv_heads; ++hd) {
                    std::vector<float> v(s.head_dim);
                    for (std::uint32_t d = 0; d < s.head_dim; ++d) v[d] = pat(layer, st, t, hd, d);
                    if (!write_head(h, seq, st, layer, t, hd, v)) return false;
                }
            }
        }
    }
    return true;
}

// `blocks` blocks for `seq` interleaved with a spacer sequence that is then
// released, so the frames of `seq` are not one contiguous run.
template <typename Harness>
void reserve_interleaved(Harness& h, SequenceId seq, SequenceId spacer, std::uint32_t blocks) {
    const std::uint32_t tpb = h.layout.shape.tokens_per_block;
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{spacer, spacer, {}, {}}));
    for (std::uint32_t i = 0; i < blocks; ++i) {
        ASSERT_TRUE(h.cache.reserve_tokens(seq, tpb));
        ASSERT_TRUE(h.cache.reserve_tokens(spacer, tpb));
    }
    h.cache.release_sequence(spacer);
}

}  // namespace

TEST(PagedAttentionTest, RefusalsLeaveTheOutputUntouched) {
    DeviceHarness h(shape_of(4, 2, 2, 4), 16);
    ASSERT_TRUE(h.ready());
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(1, 8));
    ASSERT_TRUE(fill_pattern(h, 1, 8));
    const auto view = h.cache.cache_view(1);
    std::vector<float> q(4 * 4, 0.25f);
    std::vector<float> out(q.size(), -1.0f);
    const CacheView invalid;
    EXPECT_FALSE(paged_attention_decode<float>(invalid, q.data(), params(0, 4, 4, 1.0f), out.data()));
    EXPECT_FALSE(paged_attention_decode<float>(*view, nullptr, params(0, 4, 4, 1.0f), out.data()));
    EXPECT_FALSE(paged_attention_decode<float>(*view, q.data(), params(0, 4, 4, 1.0f), nullptr));
    EXPECT_FALSE(paged_attention_decode<float>(*view, q.data(), params(0, 4, 0, 1.0f), out.data()));
    EXPECT_FALSE(paged_attention_decode<float>(*view, q.data(), params(2, 4, 4, 1.0f), out.data()));
    EXPECT_FALSE(paged_attention_decode<float>(*view, q.data(), params(0, 3, 4, 1.0f), out.data()));
    EXPECT_FALSE(paged_attention_decode<float>(*view, q.data(), params(0, 0, 4, 1.0f), out.data()));
    EXPECT_FALSE(paged_attention_decode<float>(*view, q.data(), params(0, 4, 9, 1.0f), out.data()))
        << "context past the mapped blocks";
    std::vector<bf16> qb(16, bf16(0.5f)), ob(16);
    EXPECT_FALSE(paged_attention_decode<bf16>(*view, qb.data(), params(0, 4, 4, 1.0f), ob.data()))
        << "element size differs from the cache";
    ASSERT_EQ(h.cache.swap_out_sequence(1), 2u);
    EXPECT_FALSE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(), params(0, 4, 8, 1.0f), out.data()))
        << "swapped-out context";
    for (float v : out) EXPECT_EQ(v, -1.0f);
    EXPECT_FALSE(paged_attention_last_error().empty());
}

TEST(PagedAttentionTest, HostFramesMatchTextbookAttention) {
    // The reference's own placement: frames in host memory, scattered, two
    // layers, grouped query heads. The layer's slices are staged to the GPU.
    HostHarness h(shape_of(4, 2, 2, 4), 16);
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_NO_FATAL_FAILURE(reserve_interleaved(h, 1, 99, 3));
    ASSERT_TRUE(fill_pattern(h, 1, 10));
    ASSERT_TRUE(scattered(*h.cache.cache_view(1)->block_table));
    for (std::uint32_t heads : {2u, 4u}) {
        for (std::uint32_t layer = 0; layer < 2; ++layer) {
            for (std::uint32_t ctx : {1u, 4u, 5u, 10u}) {
                std::vector<float> q(heads * 4);
                for (std::size_t i = 0; i < q.size(); ++i) q[i] = 0.3f * float(i % 7) - 0.8f;
                std::vector<float> out(q.size(), 0.0f);
                ASSERT_TRUE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(),
                                                          params(layer, heads, ctx, 0.5f), out.data()))
                    << paged_attention_last_error();
                const auto expect = textbook_attention(
                    q, heads, 2, 4, ctx, 0.5f, [&](auto t, auto kh, auto d) { return pat(layer, KVStream::Key, t, kh, d); },
                    [&](auto t, auto kh, auto d) { return pat(layer, KVStream::Value, t, kh, d); });
                for (std::size_t i = 0; i < out.size(); ++i) {
                    EXPECT_NEAR(out[i], expect[i], kF32Tol)
                        << "heads " << heads << " layer " << layer << " ctx " << ctx << " element " << i;
                }
            }
        }
    }
}

TEST(PagedAttentionTest, HostFrameRefusalsLeaveTheOutputUntouched) {
    HostHarness h(shape_of(4, 1, 1, 4), 8);
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(1, 8));
    ASSERT_TRUE(fill_pattern(h, 1, 8));
    std::vector<float> q(4, 1.0f), out(4, -1.0f);
    EXPECT_FALSE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(), params(0, 1, 9, 1.0f), out.data()))
        << "context past the mapped blocks";
    EXPECT_FALSE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(), params(1, 1, 4, 1.0f), out.data()))
        << "layer outside the shape";
    ASSERT_EQ(h.cache.swap_out_sequence(1), 2u);
    EXPECT_FALSE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(), params(0, 1, 8, 1.0f), out.data()))
        << "swapped-out context";
    for (float v : out) EXPECT_EQ(v, -1.0f);
    ASSERT_TRUE(h.cache.swap_in_sequence(1));
    ASSERT_TRUE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(), params(0, 1, 8, 1.0f), out.data()))
        << paged_attention_last_error();
}

TEST(PagedAttentionTest, EqualKeysGiveTheMeanOfTheValues) {
    DeviceHarness h(shape_of(4, 1, 1, 4), 8);
    ASSERT_TRUE(h.ready());
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(1, 8));
    for (std::uint32_t ctx : {1u, 3u, 8u}) {
        float mean = 0.0f;
        for (std::uint32_t t = 0; t < 8; ++t) {
            ASSERT_TRUE(write_head(h, 1, KVStream::Key, 0, t, 0, std::vector<float>(4, 1.0f)));
            ASSERT_TRUE(write_head(h, 1, KVStream::Value, 0, t, 0, std::vector<float>(4, float(t + 1))));
            if (t < ctx) mean += float(t + 1) / float(ctx);
        }
        std::vector<float> q(4, 0.5f), out(4, 0.0f);
        ASSERT_TRUE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(), params(0, 1, ctx, 1.0f),
                                                  out.data()))
            << paged_attention_last_error();
        for (float v : out) EXPECT_NEAR(v, mean, kF32Tol) << "ctx " << ctx;
    }
}

TEST(PagedAttentionTest, OneHotKeysAddressEachLogicalTokenThroughScatteredFrames) {
    DeviceHarness h(shape_of(4, 1, 1, 8), 8);
    ASSERT_TRUE(h.ready());
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_NO_FATAL_FAILURE(reserve_interleaved(h, 1, 99, 2));
    ASSERT_TRUE(scattered(*h.cache.cache_view(1)->block_table));
    for (std::uint32_t t = 0; t < 8; ++t) {
        std::vector<float> k(8, 0.0f);
        k[t] = 1.0f;
        ASSERT_TRUE(write_head(h, 1, KVStream::Key, 0, t, 0, k));
        ASSERT_TRUE(write_head(h, 1, KVStream::Value, 0, t, 0, std::vector<float>(8, float(t + 1) * 10.0f)));
    }
    for (std::uint32_t target = 0; target < 8; ++target) {
        std::vector<float> q(8, 0.0f), out(8, 0.0f);
        q[target] = 1.0f;
        ASSERT_TRUE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(), params(0, 1, 8, 50.0f),
                                                  out.data()));
        for (float v : out) EXPECT_NEAR(v, float(target + 1) * 10.0f, 1e-3f) << "target " << target;
    }
}

TEST(PagedAttentionTest, MatchesTextbookAttentionOnScatteredFrames) {
    DeviceHarness h(shape_of(4, 2, 2, 4), 16);
    ASSERT_TRUE(h.ready());
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_NO_FATAL_FAILURE(reserve_interleaved(h, 1, 99, 3));
    ASSERT_TRUE(fill_pattern(h, 1, 10));
    ASSERT_TRUE(scattered(*h.cache.cache_view(1)->block_table));
    for (std::uint32_t heads : {2u, 4u}) {
        for (std::uint32_t layer = 0; layer < 2; ++layer) {
            for (std::uint32_t ctx : {1u, 5u, 10u}) {
                std::vector<float> q(heads * 4);
                for (std::size_t i = 0; i < q.size(); ++i) q[i] = 0.3f * float(i % 7) - 0.8f;
                std::vector<float> out(q.size(), 0.0f);
                ASSERT_TRUE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(),
                                                          params(layer, heads, ctx, 0.5f), out.data()));
                const auto expect = textbook_attention(
                    q, heads, 2, 4, ctx, 0.5f, [&](auto t, auto kh, auto d) { return pat(layer, KVStream::Key, t, kh, d); },
                    [&](auto t, auto kh, auto d) { return pat(layer, KVStream::Value, t, kh, d); });
                for (std::size_t i = 0; i < out.size(); ++i) {
                    EXPECT_NEAR(out[i], expect[i], kF32Tol)
                        << "heads " << heads << " layer " << layer << " ctx " << ctx << " element " << i;
                }
            }
        }
    }
}

TEST(PagedAttentionTest, EachQueryHeadReadsItsOwnKvHead) {
    DeviceHarness h(shape_of(4, 1, 2, 4), 4);
    ASSERT_TRUE(h.ready());
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(1, 4));
    const float per_head[2] = {100.0f, 200.0f};
    for (std::uint32_t kh = 0; kh < 2; ++kh) {
        for (std::uint32_t t = 0; t < 4; ++t) {
            ASSERT_TRUE(write_head(h, 1, KVStream::Key, 0, t, kh, std::vector<float>(4, 1.0f)));
            ASSERT_TRUE(write_head(h, 1, KVStream::Value, 0, t, kh, std::vector<float>(4, per_head[kh])));
        }
    }
    std::vector<float> q(16, 1.0f), out(16, 0.0f);
    ASSERT_TRUE(paged_attention_decode<float>(*h.cache.cache_view(1), q.data(), params(0, 4, 4, 1.0f), out.data()));
    for (std::uint32_t qh = 0; qh < 4; ++qh) {
        for (std::uint32_t d = 0; d < 4; ++d) EXPECT_NEAR(out[qh * 4 + d], per_head[qh / 2], kF32Tol) << "head " << qh;
    }
}

TEST(PagedAttentionTest, ForkedBranchesReadTheirOwnCopies) {
    DeviceHarness h(shape_of(4, 1, 1, 4), 8);
    ASSERT_TRUE(h.ready());
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(h.cache.reserve_tokens(1, 4));
    for (std::uint32_t t = 0; t < 4; ++t) {
        ASSERT_TRUE(write_head(h, 1, KVStream::Key, 0, t, 0, std::vector<float>(4, 1.0f)));
        ASSERT_TRUE(write_head(h, 1, KVStream::Value, 0, t, 0, std::vector<float>(4, 5.0f)));
    }
    ASSERT_TRUE(h.cache.fork_sequence(1, SequenceMetadata{2, 1, {}, {}}));
    for (std::uint32_t t = 0; t < 4; ++t) {
        ASSERT_TRUE(write_head(h, 2, KVStream::Value, 0, t, 0, std::vector<float>(4, 9.0f)));
    }
    for (auto [seq, expect] : {std::pair<SequenceId, float>{1, 5.0f}, {2, 9.0f}}) {
        std::vector<float> q(4, 0.5f), out(4, 0.0f);
        ASSERT_TRUE(paged_attention_decode<float>(*h.cache.cache_view(seq), q.data(), params(0, 1, 4, 1.0f),
                                                  out.data()));
        for (float v : out) EXPECT_NEAR(v, expect, kF32Tol) << "sequence " << seq;
    }
}

namespace {

// The Qwen2-VL-7B head shape (Hq 28 over Hkv 4, head_dim 128, 16 tokens per
// block) with a two-byte element type T on harness H, against float64
// attention over the same rounded values: tolerance 2e-3 absolute plus one
// rounding step of T (2^-8 relative for bf16, 2^-11 for f16).
template <typename T, typename Harness>
void two_byte_head_dim_128(Harness& h, double rel) {
    ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_NO_FATAL_FAILURE(reserve_interleaved(h, 1, 99, 20));
    const std::uint32_t ctx = 20 * 16 - 7;
    std::mt19937 rng(7);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    std::vector<std::vector<float>> K(ctx * 4), V(ctx * 4);
    for (std::uint32_t t = 0; t < ctx; ++t) {
        for (std::uint32_t kh = 0; kh < 4; ++kh) {
            std::vector<T> kb(128), vb(128);
            K[t * 4 + kh].resize(128);
            V[t * 4 + kh].resize(128);
            for (std::uint32_t d = 0; d < 128; ++d) {
                kb[d] = T(nd(rng));
                vb[d] = T(nd(rng));
                K[t * 4 + kh][d] = float(kb[d]);
                V[t * 4 + kh][d] = float(vb[d]);
            }
            ASSERT_TRUE(write_head(h, 1, KVStream::Key, 0, t, kh, kb));
            ASSERT_TRUE(write_head(h, 1, KVStream::Value, 0, t, kh, vb));
        }
    }
    std::vector<T> qb(28 * 128), out(28 * 128);
    std::vector<float> qf(qb.size());
    for (std::size_t i = 0; i < qb.size(); ++i) {
        qb[i] = T(nd(rng));
        qf[i] = float(qb[i]);
    }
    const float scale = 1.0f / std::sqrt(128.0f);
    ASSERT_TRUE(paged_attention_decode<T>(*h.cache.cache_view(1), qb.data(), params(0, 28, ctx, scale), out.data()))
        << paged_attention_last_error();
    const auto expect = textbook_attention(
        qf, 28, 4, 128, ctx, scale, [&](auto t, auto kh, auto d) { return double(K[t * 4 + kh][d]); },
        [&](auto t, auto kh, auto d) { return double(V[t * 4 + kh][d]); });
    double worst = 0.0;
    for (std::size_t i = 0; i < out.size(); ++i) {
        const double got = float(out[i]);
        const double tol = 2e-3 + std::fabs(expect[i]) * rel;
        worst = std::max(worst, std::fabs(got - expect[i]) - tol);
        ASSERT_NEAR(got, expect[i], tol) << "element " << i;
    }
    EXPECT_LE(worst, 0.0);
}

}  // namespace

TEST(PagedAttentionTest, Bf16HeadDim128MatchesTextbookAttention) {
    // Device frames: the matrix-core kernel over the pool.
    DeviceHarness h(shape_of(16, 1, 4, 128, 2), 64);
    ASSERT_TRUE(h.ready());
    ASSERT_NO_FATAL_FAILURE(two_byte_head_dim_128<bf16>(h, 1.0 / 256.0));
}

TEST(PagedAttentionTest, Bf16HeadDim128OnHostFramesMatchesTextbookAttention) {
    // Host frames: the same kernel over the staged layer slices.
    HostHarness h(shape_of(16, 2, 4, 128, 2), 64);
    ASSERT_NO_FATAL_FAILURE(two_byte_head_dim_128<bf16>(h, 1.0 / 256.0));
}

TEST(PagedAttentionTest, F16HeadDim128MatchesTextbookAttention) {
    // An IEEE half cache read as f16 (the element type names the format).
    DeviceHarness h(shape_of(16, 1, 4, 128, 2), 64);
    ASSERT_TRUE(h.ready());
    ASSERT_NO_FATAL_FAILURE(two_byte_head_dim_128<f16>(h, 1.0 / 2048.0));
}

TEST(PagedAttentionTest, F16HeadDim128OnHostFramesMatchesTextbookAttention) {
    HostHarness h(shape_of(16, 1, 4, 128, 2), 64);
    ASSERT_NO_FATAL_FAILURE(two_byte_head_dim_128<f16>(h, 1.0 / 2048.0));
}

TEST(PagedAttentionBatchTest, OneLaunchDecodesEveryViewLikeTheSingleCalls) {
    // Ragged batch of forked and independent sequences, decoded once through
    // PagedAttentionBatch (device buffers) and once per sequence.
    DeviceHarness h(shape_of(8, 2, 2, 16), 96);
    ASSERT_TRUE(h.ready());
    const std::uint32_t lens[] = {1, 8, 9, 31, 64, 17};
    for (SequenceId s = 1; s <= 6; ++s) {
        ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{s, s, {}, {}}));
        ASSERT_TRUE(h.cache.reserve_tokens(s, lens[s - 1]));
        for (std::uint32_t layer = 0; layer < 2; ++layer) {
            for (KVStream st : {KVStream::Key, KVStream::Value}) {
                for (std::uint32_t t = 0; t < lens[s - 1]; ++t) {
                    for (std::uint32_t kh = 0; kh < 2; ++kh) {
                        std::vector<float> v(16);
                        for (std::uint32_t d = 0; d < 16; ++d) {
                            v[d] = mix_pattern({std::uint32_t(s), layer, st == KVStream::Key ? 0u : 1u, t, kh, d});
                        }
                        ASSERT_TRUE(write_head(h, s, st, layer, t, kh, v));
                    }
                }
            }
        }
    }
    ASSERT_TRUE(h.cache.fork_sequence(5, SequenceMetadata{7, 5, {}, {}}));
    std::vector<CacheView> views;
    std::vector<std::uint32_t> ctx;
    for (SequenceId s = 1; s <= 7; ++s) {
        views.push_back(*h.cache.cache_view(s));
        ctx.push_back(s == 7 ? 40u : lens[s - 1]);
    }
    const std::uint32_t heads = 6;
    std::vector<float> q(views.size() * heads * 16);
    for (std::size_t i = 0; i < q.size(); ++i) q[i] = mix_pattern({77u, std::uint32_t(i)});
    void* dq = nullptr;
    void* dout = nullptr;
    ASSERT_EQ(qvp_malloc(&dq, q.size() * 4), QVP_OK);
    ASSERT_EQ(qvp_malloc(&dout, q.size() * 4), QVP_OK);
    ASSERT_EQ(qvp_memcpy_htod(dq, q.data(), q.size() * 4, h.allocator.stream()), QVP_OK);
    for (std::uint32_t layer = 0; layer < 2; ++layer) {
        PagedAttentionBatch batch;
        ASSERT_TRUE(batch.decode(views, ctx, layer, heads, 0.25f, dq, dout, ElementType::F32)) << batch.last_error();
        std::vector<float> got(q.size());
        ASSERT_EQ(qvp_memcpy_dtoh(got.data(), dout, got.size() * 4, h.allocator.stream()), QVP_OK);
        ASSERT_EQ(qvp_stream_synchronize(h.allocator.stream()), QVP_OK);
        for (std::size_t b = 0; b < views.size(); ++b) {
            std::vector<float> qb(q.begin() + b * heads * 16, q.begin() + (b + 1) * heads * 16);
            std::vector<float> one(qb.size());
            ASSERT_TRUE(paged_attention_decode<float>(views[b], qb.data(), params(layer, heads, ctx[b], 0.25f),
                                                      one.data()));
            for (std::size_t i = 0; i < one.size(); ++i) {
                EXPECT_NEAR(got[b * heads * 16 + i], one[i], kF32Tol) << "layer " << layer << " seq " << b;
            }
        }
    }
    // A context longer than the reserved blocks is refused for the whole batch.
    PagedAttentionBatch batch;
    ctx[2] = 100;
    EXPECT_FALSE(batch.decode(views, ctx, 0, heads, 0.25f, dq, dout, ElementType::F32));
    EXPECT_FALSE(batch.last_error().empty());
    (void)qvp_free(dq);
    (void)qvp_free(dout);
}

TEST(PagedAttentionBatchTest, PackAheadPairsDecodeLikeDecode) {
    // Two objects in turn, each step packed ahead (its upload riding in the
    // previous step's decode launch) and decoded by decode_packed(): every
    // step's output is bit-equal to decode() of the same step. The
    // Qwen2-VL-7B head shape, so the persistent MFMA kernel runs.
    DeviceHarness h(shape_of(16, 1, 4, 128, 2), 256);
    ASSERT_TRUE(h.ready());
    const std::uint32_t base[] = {200, 700, 1100, 333, 900, 64};
    constexpr std::uint32_t kSteps = 5;
    for (SequenceId s = 1; s <= 6; ++s) {
        ASSERT_TRUE(h.cache.create_sequence(SequenceMetadata{s, s, {}, {}}));
        ASSERT_TRUE(h.cache.reserve_tokens(s, base[s - 1] + kSteps));
    }
    // K/V: every frame of the pool gets a pattern (one write per frame).
    std::vector<std::uint16_t> frame(h.allocator.block_stride() / 2);
    for (PhysicalBlockId f = 0; f < 256; ++f) {
        for (std::size_t i = 0; i < frame.size(); ++i) {
            frame[i] = bf16(mix_pattern({f, static_cast<std::uint32_t>(i)})).bits;
        }
        ASSERT_TRUE(h.allocator.write_block_bytes(f, 0, frame.data(), frame.size() * 2));
    }
    std::vector<CacheView> views;
    for (SequenceId s = 1; s <= 6; ++s) views.push_back(*h.cache.cache_view(s));
    const std::size_t qn = views.size() * 28 * 128;
    std::vector<std::uint16_t> q(qn);
    for (std::size_t i = 0; i < qn; ++i) q[i] = bf16(mix_pattern({5u, static_cast<std::uint32_t>(i)})).bits;
    void* dq = nullptr;
    ASSERT_EQ(qvp_malloc(&dq, qn * 2), QVP_OK);
    ASSERT_EQ(qvp_memcpy_htod(dq, q.data(), qn * 2, h.allocator.stream()), QVP_OK);
    std::vector<void*> outs(kSteps, nullptr), refs(kSteps, nullptr);
    for (std::uint32_t r = 0; r < kSteps; ++r) {
        ASSERT_EQ(qvp_malloc(&outs[r], qn * 4), QVP_OK);
        ASSERT_EQ(qvp_malloc(&refs[r], qn * 4), QVP_OK);
    }
    auto lens_of = [&](std::uint32_t r) {
        std::vector<std::uint32_t> l;
        for (std::uint32_t b : base) l.push_back(b + r);
        return l;
    };
    const float scale = 1.0f / std::sqrt(128.0f);
    PagedAttentionBatch a, b;
    EXPECT_FALSE(a.decode_packed());  // nothing packed yet
    EXPECT_FALSE(a.last_error().empty());
    PagedAttentionBatch* cur = &a;
    PagedAttentionBatch* nxt = &b;
    ASSERT_TRUE(cur->pack_ahead(views, lens_of(0), 0, 28, scale, dq, outs[0], ElementType::F32)) << cur->last_error();
    for (std::uint32_t r = 0; r < kSteps; ++r) {
        if (r + 1 < kSteps) {
            ASSERT_TRUE(nxt->pack_ahead(views, lens_of(r + 1), 0, 28, scale, dq, outs[r + 1], ElementType::F32))
                << nxt->last_error();
        }
        ASSERT_TRUE(cur->decode_packed()) << cur->last_error();
        std::swap(cur, nxt);
    }
    EXPECT_FALSE(a.decode_packed());  // each pack is decoded once
    PagedAttentionBatch plain;
    for (std::uint32_t r = 0; r < kSteps; ++r) {
        ASSERT_TRUE(plain.decode(views, lens_of(r), 0, 28, scale, dq, refs[r], ElementType::F32)) << plain.last_error();
    }
    ASSERT_EQ(qvp_stream_synchronize(h.allocator.stream()), QVP_OK);
    for (std::uint32_t r = 0; r < kSteps; ++r) {
        std::vector<std::uint32_t> got(qn), ref(qn);
        ASSERT_EQ(qvp_memcpy_dtoh(got.data(), outs[r], qn * 4, h.allocator.stream()), QVP_OK);
        ASSERT_EQ(qvp_memcpy_dtoh(ref.data(), refs[r], qn * 4, h.allocator.stream()), QVP_OK);
        ASSERT_EQ(qvp_stream_synchronize(h.allocator.stream()), QVP_OK);
        EXPECT_TRUE(got == ref) << "step " << r;
    }
    qvp_decode_plan plan{};
    ASSERT_EQ(qvp_decode_plan_info(a.packed(), &plan), QVP_OK);
    EXPECT_EQ(plan.kernel, QVP_DECODE_MFMA);
    for (void* p : outs) (void)qvp_free(p);
    for (void* p : refs) (void)qvp_free(p);
    (void)qvp_free(dq);
}

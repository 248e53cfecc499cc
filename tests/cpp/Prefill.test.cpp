// PagedAttentionBatch::prefill: causal attention of every new prompt position
// over the paged cache, the reference's decode applied per position p with
// context_len = p + 1 (include/qwenvl_paged/PagedAttention.h:43-44, as its
// end-to-end test runs it: tests/EndToEnd.test.cpp:248-258). Prompts are
// written through KVAppendBatch, then one prefill call must equal float64
// textbook attention of each position over tokens [0, p], for the MFMA shape
// (bf16, head_dim 128) and the decode-kernel shapes.
#include "device_harness.h"
#include "qwenvl_paged/KVAppend.h"

#include "qvp.h"

#include <cmath>
#include <map>

using namespace device_test;

namespace {

struct DeviceBuf {
    void* p{nullptr};
    explicit DeviceBuf(std::size_t bytes) { (void)qvp_malloc(&p, bytes); }
    ~DeviceBuf() { (void)qvp_free(p); }
};

// Element values: bf16-rounded when the cache is bf16, so the float64
// expectation sees exactly what the cache and the query hold.
float element(std::uint32_t bpe, float x) { return bpe == 2 ? static_cast<float>(bf16(x)) : x; }

template <typename T>
std::vector<T> cast_rows(const std::vector<float>& f) {
    std::vector<T> out(f.size());
    for (std::size_t i = 0; i < f.size(); ++i) out[i] = T(f[i]);
    return out;
}

struct Model {
    BlockShape shape;
    std::uint32_t heads;
    float scale;
    float key(SequenceId owner, std::uint32_t l, std::uint32_t t, std::uint32_t h, std::uint32_t d) const {
        return element(shape.bytes_per_element, mix_pattern({std::uint32_t(owner), l, 0u, t, h, d}));
    }
    float value(SequenceId owner, std::uint32_t l, std::uint32_t t, std::uint32_t h, std::uint32_t d) const {
        return element(shape.bytes_per_element, mix_pattern({std::uint32_t(owner), l, 1u, t, h, d}));
    }
    float query(SequenceId seq, std::uint32_t l, std::uint32_t p, std::uint32_t i) const {
        return element(shape.bytes_per_element, 2.0f * mix_pattern({std::uint32_t(seq), l, 7u, p, i}));
    }
};

// Appends tokens [from, to) of `seq` (owner[t] names who wrote token t) for
// every layer in one call.
void append_range(DeviceHarness& dev, KVAppendBatch& batch, const Model& m, SequenceId seq, std::uint32_t from,
                  std::uint32_t to, std::vector<SequenceId>& owner) {
    const BlockShape& s = m.shape;
    std::vector<SequenceId> seqs;
    std::vector<TokenPosition> pos;
    std::vector<float> k, v;
    owner.resize(std::max<std::size_t>(owner.size(), to));
    for (std::uint32_t t = from; t < to; ++t) {
        seqs.push_back(seq);
        pos.push_back(t);
        owner[t] = seq;
        for (std::uint32_t l = 0; l < s.num_layers; ++l)
            for (std::uint32_t h = 0; h < s.num_kv_heads; ++h)
                for (std::uint32_t d = 0; d < s.head_dim; ++d) {
                    k.push_back(m.key(seq, l, t, h, d));
                    v.push_back(m.value(seq, l, t, h, d));
                }
    }
    const std::size_t bytes = k.size() * s.bytes_per_element;
    DeviceBuf dk(bytes), dv(bytes);
    ASSERT_NE(dk.p, nullptr);
    ASSERT_NE(dv.p, nullptr);
    if (s.bytes_per_element == 2) {
        const auto hk = cast_rows<bf16>(k), hv = cast_rows<bf16>(v);
        ASSERT_EQ(qvp_memcpy_htod(dk.p, hk.data(), bytes, nullptr), QVP_OK);
        ASSERT_EQ(qvp_memcpy_htod(dv.p, hv.data(), bytes, nullptr), QVP_OK);
    } else {
        ASSERT_EQ(qvp_memcpy_htod(dk.p, k.data(), bytes, nullptr), QVP_OK);
        ASSERT_EQ(qvp_memcpy_htod(dv.p, v.data(), bytes, nullptr), QVP_OK);
    }
    ASSERT_EQ(qvp_device_synchronize(), QVP_OK);
    ASSERT_TRUE(batch.append(dev.cache, dev.allocator, seqs, pos, 0, s.num_layers, dk.p, dv.p)) << batch.last_error();
    ASSERT_TRUE(dev.allocator.synchronize());
}

// One prefill call over `seqs` (new positions [first[b], ctx[b])) on `layer`,
// checked position by position against float64 attention.
void prefill_and_check(DeviceHarness& dev, const Model& m, const std::vector<SequenceId>& seqs,
                       const std::vector<std::uint32_t>& ctx, const std::vector<std::uint32_t>& first,
                       std::uint32_t layer, std::map<SequenceId, std::vector<SequenceId>>& owner) {
    const BlockShape& s = m.shape;
    const std::uint32_t row = m.heads * s.head_dim;
    std::vector<CacheView> views;
    std::vector<float> q;
    for (std::size_t b = 0; b < seqs.size(); ++b) {
        views.push_back(*dev.cache.cache_view(seqs[b]));
        for (std::uint32_t p = first[b]; p < ctx[b]; ++p)
            for (std::uint32_t i = 0; i < row; ++i) q.push_back(m.query(seqs[b], layer, p, i));
    }
    const std::size_t n = q.size();
    DeviceBuf dq(n * s.bytes_per_element), dout(n * sizeof(float));
    ASSERT_NE(dq.p, nullptr);
    ASSERT_NE(dout.p, nullptr);
    if (s.bytes_per_element == 2) {
        const auto hq = cast_rows<bf16>(q);
        ASSERT_EQ(qvp_memcpy_htod(dq.p, hq.data(), n * 2, nullptr), QVP_OK);
    } else {
        ASSERT_EQ(qvp_memcpy_htod(dq.p, q.data(), n * 4, nullptr), QVP_OK);
    }
    ASSERT_EQ(qvp_device_synchronize(), QVP_OK);
    PagedAttentionBatch batch;
    ASSERT_TRUE(batch.prefill(views, ctx, first, layer, m.heads, m.scale, dq.p, dout.p, ElementType::F32))
        << batch.last_error();
    ASSERT_TRUE(dev.allocator.synchronize());
    std::vector<float> got(n);
    ASSERT_EQ(qvp_memcpy_dtoh(got.data(), dout.p, n * sizeof(float), nullptr), QVP_OK);
    ASSERT_EQ(qvp_device_synchronize(), QVP_OK);

    // bf16 inputs: the kernels round P to bf16 twice (hi + lo); fp32 inputs
    // are exact up to fp32 accumulation.
    const double atol = s.bytes_per_element == 2 ? 2e-3 : 1e-5;
    std::size_t at = 0;
    for (std::size_t b = 0; b < seqs.size(); ++b) {
        const auto& own = owner[seqs[b]];
        for (std::uint32_t p = first[b]; p < ctx[b]; ++p) {
            std::vector<float> qp(q.begin() + static_cast<std::ptrdiff_t>(at),
                                  q.begin() + static_cast<std::ptrdiff_t>(at + row));
            const auto expect = textbook_attention(
                qp, m.heads, s.num_kv_heads, s.head_dim, p + 1, m.scale,
                [&](auto t, auto h, auto d) { return m.key(own[t], layer, t, h, d); },
                [&](auto t, auto h, auto d) { return m.value(own[t], layer, t, h, d); });
            for (std::uint32_t i = 0; i < row; ++i) {
                ASSERT_NEAR(got[at + i], expect[i], atol + 1e-2 * std::fabs(expect[i]) * (s.bytes_per_element == 2))
                    << "seq " << seqs[b] << " position " << p << " element " << i;
            }
            at += row;
        }
    }
}

}  // namespace

TEST(PrefillTest, PromptsAndChunksEqualPerPositionAttention) {
    // (tpb, layers, kv heads, dim, bpe, query heads): the first runs the MFMA
    // prefill kernel, the others the decode kernels per position.
    struct Shape {
        std::uint32_t tpb, layers, kv, dim, bpe, heads;
    };
    for (const Shape sh : {Shape{16, 2, 2, 128, 2, 14}, Shape{16, 2, 2, 64, 4, 8}, Shape{8, 1, 1, 80, 2, 4}}) {
        Model m{shape_of(sh.tpb, sh.layers, sh.kv, sh.dim, sh.bpe), sh.heads, 1.0f / std::sqrt(float(sh.dim))};
        DeviceHarness dev(m.shape, 96);
        ASSERT_TRUE(dev.ready());
        KVAppendBatch append;
        std::map<SequenceId, std::vector<SequenceId>> owner;
        // Two prompts, 150 and 37 tokens, written and prefilled whole.
        const std::vector<std::uint32_t> len{150, 37};
        for (SequenceId id : {1, 2}) {
            ASSERT_TRUE(dev.cache.create_sequence(SequenceMetadata{id, id, {}, {}}));
            ASSERT_TRUE(dev.cache.reserve_tokens(id, 200));
            ASSERT_NO_FATAL_FAILURE(append_range(dev, append, m, id, 0, len[id - 1], owner[id]));
        }
        for (std::uint32_t layer = 0; layer < sh.layers; ++layer) {
            ASSERT_NO_FATAL_FAILURE(prefill_and_check(dev, m, {1, 2}, len, {0, 0}, layer, owner));
        }
        // A second chunk of sequence 1 plus a fork of sequence 2 that shares its
        // prompt blocks and prefills only its own continuation (copy-on-write
        // inside the shared last block).
        ASSERT_TRUE(dev.cache.fork_sequence(2, SequenceMetadata{3, 2, {}, {}}));
        owner[3] = owner[2];
        ASSERT_NO_FATAL_FAILURE(append_range(dev, append, m, 1, 150, 190, owner[1]));
        ASSERT_NO_FATAL_FAILURE(append_range(dev, append, m, 3, 37, 60, owner[3]));
        ASSERT_NO_FATAL_FAILURE(prefill_and_check(dev, m, {1, 3}, {190, 60}, {150, 37}, sh.layers - 1, owner));
        // The parent still sees its own tokens after the fork's writes.
        ASSERT_NO_FATAL_FAILURE(prefill_and_check(dev, m, {2}, {37}, {30}, 0, owner));
    }
}

TEST(PrefillTest, RefusedCallsEnqueueNothing) {
    const BlockShape shape = shape_of(16, 1, 2, 128, 2);
    DeviceHarness dev(shape, 8);
    ASSERT_TRUE(dev.ready());
    ASSERT_TRUE(dev.cache.create_sequence(SequenceMetadata{1, 1, {}, {}}));
    ASSERT_TRUE(dev.cache.reserve_tokens(1, 40));
    const CacheView view = *dev.cache.cache_view(1);
    DeviceBuf dq(40 * 8 * 128 * 2), dout(40 * 8 * 128 * 4);
    const std::vector<std::uint8_t> fill(40 * 8 * 128 * 4, 0x5a);
    ASSERT_EQ(qvp_memcpy_htod(dout.p, fill.data(), fill.size(), nullptr), QVP_OK);
    ASSERT_EQ(qvp_device_synchronize(), QVP_OK);
    PagedAttentionBatch batch;
    EXPECT_FALSE(batch.prefill({view}, {40}, {40}, 0, 8, 0.1f, dq.p, dout.p, ElementType::F32));  // no new position
    EXPECT_FALSE(batch.prefill({view}, {40}, {0, 0}, 0, 8, 0.1f, dq.p, dout.p, ElementType::F32));  // sizes differ
    EXPECT_FALSE(batch.prefill({view}, {40}, {0}, 1, 8, 0.1f, dq.p, dout.p, ElementType::F32));     // layer
    EXPECT_FALSE(batch.prefill({view}, {40}, {0}, 0, 7, 0.1f, dq.p, dout.p, ElementType::F32));     // heads
    EXPECT_FALSE(batch.prefill({view}, {49}, {0}, 0, 8, 0.1f, dq.p, dout.p, ElementType::F32));     // unmapped block
    EXPECT_FALSE(batch.prefill({view}, {40}, {0}, 0, 8, 0.1f, nullptr, dout.p, ElementType::F32));
    EXPECT_FALSE(batch.last_error().empty());
    ASSERT_EQ(qvp_device_synchronize(), QVP_OK);
    std::vector<std::uint8_t> after(fill.size());
    ASSERT_EQ(qvp_memcpy_dtoh(after.data(), dout.p, after.size(), nullptr), QVP_OK);
    ASSERT_EQ(qvp_device_synchronize(), QVP_OK);
    EXPECT_EQ(after, fill);
}

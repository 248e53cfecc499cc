// Long-context multimodal decode through the host API (the third benchmark
// configuration): one Qwen2-VL-72B attention layer (Hq 64 over Hkv 8,
// head_dim 128, 16 tokens per block, bf16 KV), 32 sequences with contexts
// uniform on [8192, 32768]. Every sequence is created with the metadata an
// image prompt carries (include/qwenvl_paged/KVCacheManager.h:23-78): its
// first quarter is one image -- a MultimodalSpan and an Image2D positional
// span over a (1, H, W) patch grid -- and the rest a Text1D span that starts
// after the image's largest position, as Qwen2-VL's get_rope_index lays a
// prompt out. The metadata travels with the sequence and does not change
// attention.
//
// Checks: metadata() returns what create_sequence was given; the M-RoPE
// positions MRopePositionBatch writes for every token (and the decode token)
// equal the closed form; the decode over the tagged sequences is bitwise equal
// to the decode over forks of them created without metadata (same frames);
// sampled heads of four sequences match float64 attention within the bf16
// tolerance. Times (medians of HIP event pairs) the whole step through
// PagedAttentionBatch::decode -- block-table walk, pack and schedule upload,
// decode -- one step at a time (the stream idle while the host works), the
// same steps enqueued back to back as an engine loop runs them (decode() per
// step, and pack_ahead() pairs whose uploads ride in the previous decode;
// pipelined_steps.h), and the decode kernel alone, and reports the schedule.
//
// Output: one JSON line. Usage: config3_bench [--seqs N] [--lo T] [--hi T] [--reps N] [--split T]
// (--split: split-K partition in tokens, 512 by default; 0 lets the decode cut
// its ranges anywhere)
#include "qvp.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MRope.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/PagedAttention.h"

#include "pipelined_steps.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

using namespace qwenvl_paged;

namespace {

struct Rng {
    std::uint64_t s;
    std::uint64_t next() {
        std::uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
};

// bf16 bits of a value uniform on [-a, a): the top bits of a 64-bit draw give
// four elements per draw.
void fill_bf16_uniform(Rng& rng, std::uint16_t* dst, std::size_t n, float a) {
    for (std::size_t i = 0; i < n; i += 4) {
        const std::uint64_t r = rng.next();
        for (std::size_t k = 0; k < 4 && i + k < n; ++k) {
            const float u = static_cast<float>((r >> (16 * k)) & 0xffffu) * (1.0f / 32768.0f) - 1.0f;
            const float v = u * a;
            std::uint32_t b;
            std::memcpy(&b, &v, 4);
            dst[i + k] = static_cast<std::uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
        }
    }
}

float bf16_to_float(std::uint16_t h) {
    const std::uint32_t u = static_cast<std::uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

[[noreturn]] void die(const std::string& what) {
    std::fprintf(stderr, "config3_bench: %s\n", what.c_str());
    std::exit(1);
}

void check(bool ok, const std::string& what) {
    if (!ok) die(what);
}

float elapsed_ms(void* a, void* b) {
    float ms = 0.f;
    check(qvp_event_elapsed_ms(&ms, a, b) == QVP_OK, qvp_last_error());
    return ms;
}

// The (H, W) patch grid of an image of n tokens: the divisor pair of n
// closest to square, H <= W.
std::pair<std::uint32_t, std::uint32_t> image_grid(std::uint32_t n) {
    std::uint32_t h = static_cast<std::uint32_t>(std::sqrt(static_cast<double>(n)));
    while (h > 1 && n % h != 0) --h;
    return {h, n / h};
}

SequenceMetadata image_prompt_metadata(SequenceId id, std::uint32_t ctx, std::uint32_t feature) {
    const std::uint32_t n_img = ctx / 4;
    const auto [gh, gw] = image_grid(n_img);
    SequenceMetadata m{id, id, {}, {}};
    m.multimodal_spans.push_back(MultimodalSpan{0, n_img, feature});
    PositionalEncodingSpan img;
    img.start_token = 0;
    img.token_count = n_img;
    img.kind = PositionEncodingKind::Image2D;
    img.origin = Position3D{0, 0, 0};
    img.stride = Position3D{1, 1, 1};
    img.grid = Position3D{1, gh, gw};
    PositionalEncodingSpan text;
    text.start_token = n_img;
    text.token_count = ctx - n_img;
    text.kind = PositionEncodingKind::Text1D;
    const std::int64_t after = static_cast<std::int64_t>(std::max(gh, gw));
    text.origin = Position3D{after, after, after};
    text.stride = Position3D{1, 1, 1};
    m.positional_encoding.spans = {img, text};
    return m;
}

bool same_metadata(const SequenceMetadata& a, const SequenceMetadata& b) {
    if (a.sequence_id != b.sequence_id || a.request_id != b.request_id ||
        a.multimodal_spans.size() != b.multimodal_spans.size() ||
        a.positional_encoding.spans.size() != b.positional_encoding.spans.size()) {
        return false;
    }
    for (std::size_t i = 0; i < a.multimodal_spans.size(); ++i) {
        const MultimodalSpan &x = a.multimodal_spans[i], &y = b.multimodal_spans[i];
        if (x.start_token != y.start_token || x.token_count != y.token_count || x.feature_index != y.feature_index) {
            return false;
        }
    }
    auto eq3 = [](const Position3D& p, const Position3D& q) {
        return p.temporal == q.temporal && p.height == q.height && p.width == q.width;
    };
    for (std::size_t i = 0; i < a.positional_encoding.spans.size(); ++i) {
        const PositionalEncodingSpan &x = a.positional_encoding.spans[i], &y = b.positional_encoding.spans[i];
        if (x.start_token != y.start_token || x.token_count != y.token_count || x.kind != y.kind ||
            !eq3(x.origin, y.origin) || !eq3(x.stride, y.stride) || !eq3(x.grid, y.grid)) {
            return false;
        }
    }
    return true;
}

}  // namespace

int main(int argc, char** argv) {
    std::uint32_t seqs = 32, lo = 8192, hi = 32768, reps = 20, split = 512;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string k = argv[i];
        const std::uint32_t v = static_cast<std::uint32_t>(std::atoi(argv[i + 1]));
        if (k == "--seqs") seqs = v;
        else if (k == "--lo") lo = v;
        else if (k == "--hi") hi = v;
        else if (k == "--reps") reps = v;
        else if (k == "--split") split = v;
    }
    check(seqs > 0 && lo > 0 && hi >= lo, "bad arguments");
    constexpr std::uint32_t kTpb = 16, kHkv = 8, kHq = 64, kD = 128;
    const BlockShape shape{kTpb, 1, kHkv, kD, 2};
    Rng rng{3};
    std::vector<std::uint32_t> ctx(seqs);
    std::uint64_t need = 0;
    for (auto& c : ctx) {
        c = lo + static_cast<std::uint32_t>(rng.next() % (hi - lo + 1));
        need += (c + kTpb - 1) / kTpb;
    }
    const std::uint32_t pool = static_cast<std::uint32_t>(need + need / 10 + 1);

    AllocatorConfig cfg;
    cfg.block_shape = shape;
    cfg.max_blocks = pool;
    cfg.placement = BlockPlacement::Device;
    MemoryAllocator dev(cfg);
    check(dev.ok(), "device pool: " + dev.last_error());
    KVCacheManager cache(dev);
    const KVBlockLayout layout{shape};
    const std::size_t frame_bytes = shape.byte_size();

    // Tagged sequences, their frames filled with bf16 uniform on [-1, 1);
    // then an untagged fork of each (shares every frame).
    std::vector<SequenceMetadata> given;
    std::vector<std::uint16_t> frame(frame_bytes / 2);
    for (std::uint32_t b = 0; b < seqs; ++b) {
        const SequenceId id = b + 1;
        given.push_back(image_prompt_metadata(id, ctx[b], b));
        check(cache.create_sequence(given.back()), "create sequence");
        check(cache.reserve_tokens(id, ctx[b] + 1), "reserve tokens");
        for (const BlockTableEntry& e : cache.cache_view(id)->block_table->entries()) {
            fill_bf16_uniform(rng, frame.data(), frame.size(), 1.0f);
            check(dev.write_block_bytes(e.physical_id, 0, frame.data(), frame_bytes), "write frame");
        }
    }
    for (std::uint32_t b = 0; b < seqs; ++b) {
        check(cache.fork_sequence(b + 1, SequenceMetadata{1000 + b + 1, b + 1, {}, {}}), "fork");
    }
    check(dev.synchronize(), "sync");

    bool metadata_roundtrip = true;
    std::uint64_t image_tokens = 0;
    for (std::uint32_t b = 0; b < seqs; ++b) {
        const SequenceMetadata* m = cache.metadata(b + 1);
        metadata_roundtrip = metadata_roundtrip && m != nullptr && same_metadata(*m, given[b]);
        image_tokens += given[b].multimodal_spans.front().token_count;
    }

    // M-RoPE positions of every cached token and the decode token.
    void* stream = dev.stream();
    std::vector<SequenceId> ids;
    std::vector<TokenPosition> begin, end;
    std::uint64_t rows = 0;
    for (std::uint32_t b = 0; b < seqs; ++b) {
        ids.push_back(b + 1);
        begin.push_back(0);
        end.push_back(ctx[b] + 1);
        rows += ctx[b] + 1;
    }
    void* dpos = nullptr;
    check(qvp_malloc(&dpos, rows * 3 * sizeof(std::int64_t)) == QVP_OK, "malloc positions");
    MRopePositionBatch rope;
    check(rope.materialise(cache, ids, begin, end, static_cast<std::int64_t*>(dpos), stream), rope.last_error());
    std::vector<std::int64_t> pos(rows * 3);
    check(qvp_memcpy_dtoh(pos.data(), dpos, pos.size() * sizeof(std::int64_t), stream) == QVP_OK, "download");
    check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
    bool positions_ok = true;
    std::uint64_t row = 0;
    for (std::uint32_t b = 0; b < seqs; ++b) {
        const std::uint32_t n_img = ctx[b] / 4;
        const auto [gh, gw] = image_grid(n_img);
        const std::int64_t after = std::max(gh, gw);
        for (std::uint32_t t = 0; t <= ctx[b]; ++t, ++row) {
            std::int64_t want[3];
            if (t < n_img) {
                want[0] = 0;
                want[1] = t / gw;
                want[2] = t % gw;
            } else {
                want[0] = want[1] = want[2] = after + (t - n_img);
            }
            for (int a = 0; a < 3; ++a) positions_ok = positions_ok && pos[a * rows + row] == want[a];
        }
    }

    // Decode: tagged sequences, then their untagged forks.
    std::vector<CacheView> tagged, plain;
    for (std::uint32_t b = 0; b < seqs; ++b) {
        tagged.push_back(*cache.cache_view(b + 1));
        plain.push_back(*cache.cache_view(1000 + b + 1));
    }
    const std::size_t qn = static_cast<std::size_t>(seqs) * kHq * kD;
    std::vector<std::uint16_t> q(qn);
    fill_bf16_uniform(rng, q.data(), q.size(), 1.7f);
    void *dq = nullptr, *dout = nullptr, *dout2 = nullptr;
    check(qvp_malloc(&dq, qn * 2) == QVP_OK && qvp_malloc(&dout, qn * 2) == QVP_OK &&
              qvp_malloc(&dout2, qn * 2) == QVP_OK,
          "malloc");
    check(qvp_memcpy_htod(dq, q.data(), qn * 2, stream) == QVP_OK, "upload q");
    const float scale = 1.0f / std::sqrt(static_cast<float>(kD));
    PagedAttentionBatch attn, attn_plain;
    attn.set_split_tokens(split);
    attn_plain.set_split_tokens(split);
    check(attn.decode(tagged, ctx, 0, kHq, scale, dq, dout, ElementType::BF16), attn.last_error());
    check(attn_plain.decode(plain, ctx, 0, kHq, scale, dq, dout2, ElementType::BF16), attn_plain.last_error());
    check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
    void *e0 = nullptr, *e1 = nullptr;
    check(qvp_event_create(&e0) == QVP_OK && qvp_event_create(&e1) == QVP_OK, "events");
    std::vector<float> times;
    for (std::uint32_t r = 0; r < reps; ++r) {
        check(qvp_event_record(e0, stream) == QVP_OK, "record");
        check(attn.decode(tagged, ctx, 0, kHq, scale, dq, dout, ElementType::BF16), attn.last_error());
        check(qvp_event_record(e1, stream) == QVP_OK, "record");
        check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
        times.push_back(elapsed_ms(e0, e1));
    }
    std::sort(times.begin(), times.end());
    const float step_ms = times.empty() ? 0.f : times[times.size() / 2];
    PagedAttentionBatch ahead_a, ahead_b;
    ahead_a.set_split_tokens(split);
    ahead_b.set_split_tokens(split);
    const pipelined_steps::Forms piped = pipelined_steps::run_forms(
        attn, ahead_a, ahead_b, tagged, ctx, 0, kHq, scale, dq, dout, ElementType::BF16, stream,
        static_cast<int>(std::max<std::uint32_t>(reps, 10)));
    // The decode kernel alone: the packed batch of the last step decoded
    // again (its schedule is cached), as the engine does for every layer of
    // a step after the first.
    qvp_decode_args args{};
    args.query = dq;
    args.out = dout;
    args.kv_base = dev.device_base();
    args.block_stride = dev.block_stride();
    args.batch = attn.packed();
    args.kv_dtype = QVP_DTYPE_BF16;
    args.out_dtype = QVP_DTYPE_BF16;
    args.layer = 0;
    args.num_layers = 1;
    args.num_query_heads = kHq;
    args.num_kv_heads = kHkv;
    args.head_dim = kD;
    args.tokens_per_block = kTpb;
    args.head_stride = layout.head_stride();
    args.token_stride = layout.token_stride();
    args.stream_stride = layout.stream_stride();
    args.layer_stride = layout.layer_stride();
    args.scale = scale;
    times.clear();
    for (std::uint32_t r = 0; r < reps; ++r) {
        check(qvp_event_record(e0, stream) == QVP_OK, "record");
        check(qvp_paged_decode(&args, stream) == QVP_OK, qvp_last_error());
        check(qvp_event_record(e1, stream) == QVP_OK, "record");
        check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
        times.push_back(elapsed_ms(e0, e1));
    }
    std::sort(times.begin(), times.end());
    const float decode_ms = times.empty() ? 0.f : times[times.size() / 2];
    std::vector<std::uint16_t> out(qn), out_plain(qn);
    check(qvp_memcpy_dtoh(out.data(), dout, qn * 2, stream) == QVP_OK, "download");
    check(qvp_memcpy_dtoh(out_plain.data(), dout2, qn * 2, stream) == QVP_OK, "download");
    check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
    const bool tagged_equals_plain = out == out_plain;
    qvp_decode_plan plan{};
    check(qvp_decode_plan_info(attn.packed(), &plan) == QVP_OK, qvp_last_error());

    // float64 attention of eight query heads (one per kv head) of four
    // sequences, from the frames read back.
    double worst = 0.0;
    std::size_t checked = 0;
    for (std::uint32_t b = 0; b < seqs; b += std::max<std::uint32_t>(1, seqs / 4)) {
        const BlockTable& t = *tagged[b].block_table;
        std::vector<std::vector<std::uint16_t>> frames;
        for (std::uint32_t blk = 0; blk * kTpb < ctx[b]; ++blk) {
            std::vector<std::uint16_t> f(frame_bytes / 2);
            check(dev.read_block_bytes(*t.lookup(blk), 0, f.data(), frame_bytes), "read");
            frames.push_back(std::move(f));
        }
        for (std::uint32_t g = 0; g < kHkv; ++g) {
            const std::uint32_t h = g * (kHq / kHkv) + (b + g) % (kHq / kHkv);
            const std::uint16_t* qh = q.data() + (static_cast<std::size_t>(b) * kHq + h) * kD;
            std::vector<double> s(ctx[b]);
            double m = -1e300;
            for (std::uint32_t tok = 0; tok < ctx[b]; ++tok) {
                const std::uint16_t* k =
                    frames[tok / kTpb].data() + *layout.element_offset(0, KVStream::Key, tok % kTpb, g);
                double dot = 0.0;
                for (std::uint32_t d = 0; d < kD; ++d) dot += double(bf16_to_float(qh[d])) * bf16_to_float(k[d]);
                s[tok] = dot * scale;
                m = std::max(m, s[tok]);
            }
            std::vector<double> o(kD, 0.0);
            double l = 0.0;
            for (std::uint32_t tok = 0; tok < ctx[b]; ++tok) {
                const double wgt = std::exp(s[tok] - m);
                l += wgt;
                const std::uint16_t* v =
                    frames[tok / kTpb].data() + *layout.element_offset(0, KVStream::Value, tok % kTpb, g);
                for (std::uint32_t d = 0; d < kD; ++d) o[d] += wgt * bf16_to_float(v[d]);
            }
            for (std::uint32_t d = 0; d < kD; ++d) {
                const double ref = o[d] / l;
                const double got = bf16_to_float(out[(static_cast<std::size_t>(b) * kHq + h) * kD + d]);
                // 2e-3 absolute plus one bf16 rounding of the output.
                worst = std::max(worst, std::fabs(got - ref) - (2e-3 + std::fabs(ref) / 256.0));
                ++checked;
            }
        }
    }

    std::uint64_t tokens = 0;
    for (std::uint32_t c : ctx) tokens += c;
    const double kv_bytes = static_cast<double>(tokens) * kHkv * kD * 2 * 2;
    const double qo = static_cast<double>(qn) * 2 * 2;
    const bool ok = metadata_roundtrip && positions_ok && tagged_equals_plain && worst <= 0.0;
    std::printf(
        "{\"mode\": \"config3_multimodal\", \"sequences\": %u, \"cached_tokens\": %llu, \"image_tokens\": %llu, "
        "\"metadata_roundtrip\": %s, \"position_rows\": %llu, \"positions_match_closed_form\": %s, "
        "\"tagged_equals_untagged_bitwise\": %s, \"step_us_median\": %.3f, \"step_tokens_per_s\": %.1f, "
        "\"pipelined_step_us\": %.3f, \"pack_ahead_step_us\": %.3f, \"host_us_per_step\": %.3f, "
        "\"pack_ahead_host_us_per_step\": %.3f, \"pipelined_over_kernel\": %.4f, \"pack_ahead_over_kernel\": %.4f, "
        "\"pack_ahead_tokens_per_s\": %.1f, "
        "\"decode_us_median\": %.3f, \"decode_GBps\": %.1f, "
        "\"decode_frac_of_8TBps\": %.4f, \"decode_tokens_per_s\": %.1f, \"plan\": {\"kernel\": %u, \"workgroups\": %u, "
        "\"pieces\": %u, \"slots\": %u, \"kv_heads_per_segment\": %u, \"split_tokens\": %u, \"query_group\": %u}, \"checked_elements\": %zu, "
        "\"worst_excess_over_tolerance\": %.3g, \"decode_within_tolerance\": %s}\n",
        seqs, static_cast<unsigned long long>(tokens), static_cast<unsigned long long>(image_tokens),
        metadata_roundtrip ? "true" : "false", static_cast<unsigned long long>(rows), positions_ok ? "true" : "false",
        tagged_equals_plain ? "true" : "false", step_ms * 1e3, seqs / (step_ms * 1e-3), piped.loop.gpu_us_per_step,
        piped.ahead.gpu_us_per_step, piped.loop.host_us_per_step, piped.ahead.host_us_per_step,
        piped.loop.gpu_us_per_step / (decode_ms * 1e3), piped.ahead.gpu_us_per_step / (decode_ms * 1e3),
        seqs / (piped.ahead.gpu_us_per_step * 1e-6), decode_ms * 1e3, (kv_bytes + qo) / (decode_ms * 1e-3) / 1e9,
        (kv_bytes + qo) / (decode_ms * 1e-3) / 8e12, seqs / (decode_ms * 1e-3), plan.kernel, plan.workgroups,
        plan.pieces, plan.slots, plan.kv_heads_per_segment, plan.split_tokens, plan.query_group, checked, worst,
        worst <= 0.0 ? "true" : "false");
    (void)qvp_free(dq);
    (void)qvp_free(dout);
    (void)qvp_free(dout2);
    (void)qvp_free(dpos);
    (void)qvp_event_destroy(e0);
    (void)qvp_event_destroy(e1);
    return ok ? 0 : 2;
}

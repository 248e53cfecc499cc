// Parallel-sampling copy-on-write on device frames (the fourth benchmark
// configuration): 16 prompts of 2048 tokens (Qwen2-VL-7B KV shape, bf16, one
// layer) reserved with 2049 slots, so logical block 128 is a partially filled
// tail shared by the prompt's branches; each prompt forks 8 branches (the
// prompt keeps its reference), every branch's first decode token lands in the
// shared tail, and the step -- the 128 copy-on-write materialisations and the
// 128 tokens' K/V rows -- runs through KVAppendBatch as one launch (each
// destination chunk copied, then overwritten by its rows). Then one paged
// decode over the 128 branches.
//
// Checks: the device allocator takes the same decisions as a host-placement
// allocator replaying the same calls (the reference's memcpy semantics), the
// whole device pool equals the host pool byte for byte, every copied frame
// equals its source with the branch's rows over its slot, and the decode of
// sampled branches matches float64 attention within the bf16 tolerance.
//
// Timing (medians of HIP event pairs): copy_append_us_median is the one
// launch of the step's copies and rows (copy_us_median the copies alone,
// copy_then_append_us_median the two launches); step_us_median is a whole
// PagedAttentionBatch::decode call (block-table walk, pack and schedule upload,
// decode) one step at a time, the stream idle while the host works;
// pipelined_step_us / pack_ahead_step_us the same steps enqueued back to back
// as an engine loop runs them (decode() per step, and pack_ahead() pairs whose
// uploads ride in the previous decode; pipelined_steps.h); decode_us_median
// the decode kernel alone, relaunched on the packed batch.
//
// --layers N stores all N layers of the model in each frame (N = 28: whole
// Qwen2-VL-7B frames of 917,504 B, so each copy-on-write copy moves 28x the
// bytes); the decode reads layer 0.
//
// Output: one JSON line. Usage: cow_bench [--prompts N] [--branches N] [--reps N] [--layers N]
#include "qvp.h"
#include "qwenvl_paged/KVAppend.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/PagedAttention.h"

#include "pipelined_steps.h"

#include <algorithm>
#include <chrono>
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
    // Approximately N(0, sigma^2): sum of four uniforms, rescaled.
    float gauss(float sigma) {
        float acc = 0.f;
        for (int i = 0; i < 4; ++i) acc += static_cast<float>(next() >> 40) * (1.0f / 16777216.0f);
        return (acc - 2.0f) * 1.7320508f * sigma;
    }
};

float bf16_to_float(std::uint16_t h) {
    const std::uint32_t u = static_cast<std::uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

[[noreturn]] void die(const std::string& what) {
    std::fprintf(stderr, "cow_bench: %s\n", what.c_str());
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

}  // namespace

int main(int argc, char** argv) {
    std::uint32_t prompts = 16, branches = 8, reps = 20, layers = 1;
    for (int i = 1; i + 1 < argc; i += 2) {
        const std::string k = argv[i];
        const std::uint32_t v = static_cast<std::uint32_t>(std::atoi(argv[i + 1]));
        if (k == "--prompts") prompts = v;
        else if (k == "--branches") branches = v;
        else if (k == "--reps") reps = v;
        else if (k == "--layers") layers = std::max<std::uint32_t>(1, v);
    }
    constexpr std::uint32_t kTpb = 16, kHkv = 4, kHq = 28, kD = 128, kPrompt = 2048;
    const BlockShape shape{kTpb, layers, kHkv, kD, 2};
    const std::uint32_t blocks_per_prompt = (kPrompt + 1 + kTpb - 1) / kTpb;  // 129
    const std::uint32_t pool = prompts * blocks_per_prompt + prompts * branches + 64;

    AllocatorConfig dev_cfg;
    dev_cfg.block_shape = shape;
    dev_cfg.max_blocks = pool;
    dev_cfg.placement = BlockPlacement::Device;
    MemoryAllocator dev(dev_cfg);
    check(dev.ok(), "device pool: " + dev.last_error());
    AllocatorConfig host_cfg = dev_cfg;
    host_cfg.placement = BlockPlacement::Host;
    MemoryAllocator host(host_cfg);
    KVCacheManager dev_cache(dev);
    KVCacheManager host_cache(host);
    const KVBlockLayout layout{shape};
    const std::size_t frame_bytes = shape.byte_size();

    // Prompts: reserve 2049 slots and fill every frame with bf16 N(0, 0.5).
    Rng rng{42};
    std::vector<std::uint16_t> frame(frame_bytes / 2);
    for (std::uint32_t p = 0; p < prompts; ++p) {
        const SequenceId id = p + 1;
        check(dev_cache.create_sequence(SequenceMetadata{id, id, {}, {}}) &&
                  host_cache.create_sequence(SequenceMetadata{id, id, {}, {}}),
              "create prompt");
        check(dev_cache.reserve_tokens(id, kPrompt + 1) && host_cache.reserve_tokens(id, kPrompt + 1),
              "reserve prompt");
        for (const BlockTableEntry& e : dev_cache.cache_view(id)->block_table->entries()) {
            // Random layer 0 (what the decode reads); the other layers repeat it.
            const std::size_t slice = frame.size() / layers;
            for (std::size_t i = 0; i < slice; ++i) {
                const float v = rng.gauss(0.5f);
                std::uint32_t u;
                std::memcpy(&u, &v, 4);
                frame[i] = static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
            }
            for (std::uint32_t l = 1; l < layers; ++l) std::copy_n(frame.begin(), slice, frame.begin() + l * slice);
            check(dev.write_block_bytes(e.physical_id, 0, frame.data(), frame_bytes), "write frame");
            check(host.write_block_bytes(e.physical_id, 0, frame.data(), frame_bytes), "write host frame");
        }
    }
    // Branches share every block of their prompt.
    for (std::uint32_t p = 0; p < prompts; ++p) {
        for (std::uint32_t c = 0; c < branches; ++c) {
            const SequenceId child = 1000 + p * branches + c;
            check(dev_cache.fork_sequence(p + 1, SequenceMetadata{child, p + 1, {}, {}}) &&
                      host_cache.fork_sequence(p + 1, SequenceMetadata{child, p + 1, {}, {}}),
                  "fork");
        }
    }
    check(dev.synchronize(), "sync");

    // The step: each branch's token 2049 lands in the shared tail block, which
    // is copied for it; KVAppendBatch queues the 128 copies and runs them in
    // the launch that stores the tokens' K/V rows (qvp_copy_append_kv). The
    // host-placement allocator replays the same step with memcpy calls.
    void* stream = dev.stream();
    void *e0 = nullptr, *e1 = nullptr;
    check(qvp_event_create(&e0) == QVP_OK && qvp_event_create(&e1) == QVP_OK, "events");
    const std::uint32_t nb = prompts * branches;
    std::vector<SequenceId> children(nb);
    std::vector<TokenPosition> new_pos(nb, kPrompt + 1);
    std::vector<std::pair<PhysicalBlockId, PhysicalBlockId>> copies;
    for (std::uint32_t i = 0; i < nb; ++i) {
        children[i] = 1000 + i;
        copies.emplace_back(*dev_cache.cache_view(children[i])->block_table->lookup(kPrompt / kTpb), 0);
    }
    const std::size_t row_elems = static_cast<std::size_t>(layers) * kHkv * kD;  // per token
    std::vector<std::uint16_t> k_rows(nb * row_elems), v_rows(nb * row_elems);
    for (auto* rows : {&k_rows, &v_rows}) {
        for (auto& x : *rows) {
            const float f = rng.gauss(0.5f);
            std::uint32_t u;
            std::memcpy(&u, &f, 4);
            x = static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        }
    }
    void *dk = nullptr, *dv = nullptr;
    check(qvp_malloc(&dk, k_rows.size() * 2) == QVP_OK && qvp_malloc(&dv, v_rows.size() * 2) == QVP_OK, "rows");
    check(qvp_memcpy_htod(dk, k_rows.data(), k_rows.size() * 2, stream) == QVP_OK &&
              qvp_memcpy_htod(dv, v_rows.data(), v_rows.size() * 2, stream) == QVP_OK,
          "upload rows");
    const std::uint64_t launches_before = dev.copy_launches();
    KVAppendBatch dev_append, host_append;
    check(dev_append.append(dev_cache, dev, children, new_pos, 0, layers, dk, dv), dev_append.last_error());
    check(host_append.append(host_cache, host, children, new_pos, 0, layers, k_rows.data(), v_rows.data()),
          host_append.last_error());
    const std::size_t pending = dev.pending_operations();
    check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
    const std::uint64_t copy_launches = dev.copy_launches() - launches_before;
    for (std::uint32_t i = 0; i < nb; ++i) {
        copies[i].second = *dev_cache.cache_view(children[i])->block_table->lookup(kPrompt / kTpb);
        const PhysicalBlockId h = *host_cache.cache_view(children[i])->block_table->lookup(kPrompt / kTpb);
        check(copies[i].second == h && copies[i].second != copies[i].first, "copy-on-write decisions differ");
    }
    // Time the same launch again (the first launch of a kernel in a process
    // also loads its code object): copying each source onto its destination
    // and storing the same rows once more changes nothing. Beside it, the
    // step as two launches (qvp_copy_blocks, then qvp_append_kv).
    std::vector<std::uint32_t> src_ids, dst_ids, slots(nb, (kPrompt + 1) % kTpb);
    for (auto [src, dst] : copies) {
        src_ids.push_back(src);
        dst_ids.push_back(dst);
    }
    qvp_append_args ap{};
    ap.kv_base = dev.device_base();
    ap.block_stride = dev.block_stride();
    ap.num_blocks = pool;
    ap.kv_dtype = QVP_DTYPE_BF16;
    ap.num_layers = layers;
    ap.first_layer = 0;
    ap.layer_count = layers;
    ap.num_kv_heads = kHkv;
    ap.head_dim = kD;
    ap.tokens_per_block = kTpb;
    ap.head_stride = layout.head_stride();
    ap.token_stride = layout.token_stride();
    ap.stream_stride = layout.stream_stride();
    ap.layer_stride = layout.layer_stride();
    ap.k = dk;
    ap.v = dv;
    auto median_us = [&](auto&& step) {
        std::vector<float> t;
        for (std::uint32_t r = 0; r < std::max<std::uint32_t>(reps, 1); ++r) {
            check(qvp_event_record(e0, stream) == QVP_OK, "record");
            step();
            check(qvp_event_record(e1, stream) == QVP_OK, "record");
            check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
            t.push_back(elapsed_ms(e0, e1));
        }
        std::sort(t.begin(), t.end());
        return 1e3 * t[t.size() / 2];
    };
    const double fused_us = median_us([&] {
        check(qvp_copy_append_kv(&ap, src_ids.data(), dst_ids.data(), nb, dev.block_stride(), dst_ids.data(),
                                 slots.data(), nb, stream) == QVP_OK,
              qvp_last_error());
    });
    const double copy_us = median_us([&] {
        check(qvp_copy_blocks(dev.device_base(), dev.block_stride(), pool, src_ids.data(), dst_ids.data(), nb,
                              dev.block_stride(), stream) == QVP_OK,
              qvp_last_error());
    });
    const double two_launch_us = median_us([&] {
        check(qvp_copy_blocks(dev.device_base(), dev.block_stride(), pool, src_ids.data(), dst_ids.data(), nb,
                              dev.block_stride(), stream) == QVP_OK &&
                  qvp_append_kv(&ap, dst_ids.data(), slots.data(), nb, stream) == QVP_OK,
              qvp_last_error());
    });

    // Bit-exact: every frame of the device pool equals the host pool's.
    bool frames_equal = true;
    std::vector<std::uint8_t> a(frame_bytes), b(frame_bytes);
    for (PhysicalBlockId f = 0; f < pool && frames_equal; ++f) {
        if (host.info(f)->ref_count == 0) continue;
        check(dev.read_block_bytes(f, 0, a.data(), frame_bytes), "read");
        check(host.read_block_bytes(f, 0, b.data(), frame_bytes), "read host");
        frames_equal = a == b;
    }
    // Each copy equals its source with the branch's rows stored over slot 1.
    bool copies_equal = true;
    for (std::uint32_t i = 0; i < nb; ++i) {
        check(dev.read_block_bytes(copies[i].first, 0, a.data(), frame_bytes), "read");
        check(dev.read_block_bytes(copies[i].second, 0, b.data(), frame_bytes), "read");
        for (std::uint32_t l = 0; l < layers; ++l) {
            for (const KVStream st : {KVStream::Key, KVStream::Value}) {
                const std::uint16_t* rows = (st == KVStream::Key ? k_rows : v_rows).data() + i * row_elems;
                for (std::uint32_t h = 0; h < kHkv; ++h) {
                    const std::size_t off = *layout.element_offset(l, st, slots[i], h) * 2;
                    std::memcpy(a.data() + off, rows + (static_cast<std::size_t>(l) * kHkv + h) * kD, kD * 2);
                }
            }
        }
        copies_equal = copies_equal && a == b;
    }

    // Decode over every branch: context 2050 (the prompt, the shared tail
    // token and the branch's own token, all in frames read back below).
    const std::uint32_t ctx = kPrompt + 2;
    std::vector<CacheView> views;
    std::vector<std::uint32_t> lens(nb, ctx);
    for (std::uint32_t i = 0; i < nb; ++i) views.push_back(*dev_cache.cache_view(1000 + i));
    std::vector<std::uint16_t> q(static_cast<std::size_t>(nb) * kHq * kD);
    for (auto& x : q) {
        const float v = rng.gauss(1.0f);
        std::uint32_t u;
        std::memcpy(&u, &v, 4);
        x = static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
    void *dq = nullptr, *dout = nullptr;
    check(qvp_malloc(&dq, q.size() * 2) == QVP_OK && qvp_malloc(&dout, q.size() * 2) == QVP_OK, "malloc");
    check(qvp_memcpy_htod(dq, q.data(), q.size() * 2, stream) == QVP_OK, "upload q");
    const float scale = 1.0f / std::sqrt(static_cast<float>(kD));
    PagedAttentionBatch attn;
    check(attn.decode(views, lens, 0, kHq, scale, dq, dout, ElementType::BF16), attn.last_error());
    check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
    std::vector<float> times;
    for (std::uint32_t r = 0; r < reps; ++r) {
        check(qvp_event_record(e0, stream) == QVP_OK, "record");
        check(attn.decode(views, lens, 0, kHq, scale, dq, dout, ElementType::BF16), attn.last_error());
        check(qvp_event_record(e1, stream) == QVP_OK, "record");
        check(qvp_stream_synchronize(stream) == QVP_OK, "sync");
        times.push_back(elapsed_ms(e0, e1));
    }
    std::sort(times.begin(), times.end());
    const float step_ms = times[times.size() / 2];
    PagedAttentionBatch ahead_a, ahead_b;
    const pipelined_steps::Forms piped =
        pipelined_steps::run_forms(attn, ahead_a, ahead_b, views, lens, 0, kHq, scale, dq, dout, ElementType::BF16,
                                   stream, static_cast<int>(std::max<std::uint32_t>(reps, 20)));
    // The decode kernel alone: the last step's packed batch decoded again (its
    // work schedule is cached), as an engine decodes the other layers of a
    // step.
    const KVBlockLayout lay{shape};
    qvp_decode_args args{};
    args.query = dq;
    args.out = dout;
    args.kv_base = dev.device_base();
    args.block_stride = dev.block_stride();
    args.batch = attn.packed();
    args.kv_dtype = QVP_DTYPE_BF16;
    args.out_dtype = QVP_DTYPE_BF16;
    args.num_layers = layers;
    args.num_query_heads = kHq;
    args.num_kv_heads = kHkv;
    args.head_dim = kD;
    args.tokens_per_block = kTpb;
    args.head_stride = lay.head_stride();
    args.token_stride = lay.token_stride();
    args.stream_stride = lay.stream_stride();
    args.layer_stride = lay.layer_stride();
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
    const float decode_ms = times[times.size() / 2];
    std::vector<std::uint16_t> out(q.size());
    check(qvp_memcpy_dtoh(out.data(), dout, out.size() * 2, stream) == QVP_OK, "download");
    check(qvp_stream_synchronize(stream) == QVP_OK, "sync");

    // float64 attention of eight sampled branches from the frames read back.
    double worst = 0.0;
    std::size_t checked = 0;
    for (std::uint32_t i = 0; i < nb; i += std::max<std::uint32_t>(1, nb / 8)) {
        const BlockTable& t = *views[i].block_table;
        std::vector<std::vector<std::uint16_t>> frames;
        for (std::uint32_t blk = 0; blk * kTpb < ctx; ++blk) {
            std::vector<std::uint16_t> f(frame_bytes / 2);
            check(dev.read_block_bytes(*t.lookup(blk), 0, f.data(), frame_bytes), "read");
            frames.push_back(std::move(f));
        }
        for (std::uint32_t h = 0; h < kHq; ++h) {
            const std::uint32_t g = h / (kHq / kHkv);
            const std::uint16_t* qh = q.data() + (static_cast<std::size_t>(i) * kHq + h) * kD;
            std::vector<double> s(ctx);
            double m = -1e300;
            for (std::uint32_t tok = 0; tok < ctx; ++tok) {
                const std::uint16_t* k =
                    frames[tok / kTpb].data() + *layout.element_offset(0, KVStream::Key, tok % kTpb, g);
                double dot = 0.0;
                for (std::uint32_t d = 0; d < kD; ++d) dot += double(bf16_to_float(qh[d])) * bf16_to_float(k[d]);
                s[tok] = dot * scale;
                m = std::max(m, s[tok]);
            }
            std::vector<double> o(kD, 0.0);
            double l = 0.0;
            for (std::uint32_t tok = 0; tok < ctx; ++tok) {
                const double wgt = std::exp(s[tok] - m);
                l += wgt;
                const std::uint16_t* v =
                    frames[tok / kTpb].data() + *layout.element_offset(0, KVStream::Value, tok % kTpb, g);
                for (std::uint32_t d = 0; d < kD; ++d) o[d] += wgt * bf16_to_float(v[d]);
            }
            for (std::uint32_t d = 0; d < kD; ++d) {
                const double ref = o[d] / l;
                const double got = bf16_to_float(out[(static_cast<std::size_t>(i) * kHq + h) * kD + d]);
                // 2e-3 absolute plus one bf16 rounding of the output.
                worst = std::max(worst, std::fabs(got - ref) - (2e-3 + std::fabs(ref) / 256.0));
                ++checked;
            }
        }
    }

    const double copy_bytes = 2.0 * static_cast<double>(copies.size()) * dev.block_stride();
    const double row_bytes = 2.0 * 2.0 * static_cast<double>(nb) * row_elems * 2;  // read + write, K and V
    const double per_token = static_cast<double>(kHkv) * kD * 2 * 2;
    const double logical = static_cast<double>(nb) * ctx * per_token;
    // Distinct cached tokens: each prompt's 2048 shared ones, and per branch
    // the two in its private tail frame.
    const double unique = (static_cast<double>(prompts) * kPrompt + 2.0 * nb) * per_token;
    const double qo = static_cast<double>(nb) * kHq * kD * 2 * 2;
    std::printf(
        "{\"mode\": \"config4_cow\", \"layers\": %u, \"prompts\": %u, \"branches_per_prompt\": %u, \"cow_pairs\": %zu, "
        "\"pending_after_append\": %zu, \"copy_launches\": %llu, \"copy_append_us_median\": %.3f, "
        "\"copy_append_read_plus_write_GBps\": %.1f, \"copy_us_median\": %.3f, \"copy_then_append_us_median\": %.3f, "
        "\"frames_equal_host_allocator\": %s, \"copies_equal_source_plus_rows\": %s, \"decode_branches\": %u, "
        "\"decode_ctx\": %u, \"step_us_median\": %.3f, \"pipelined_step_us\": %.3f, \"pack_ahead_step_us\": %.3f, "
        "\"host_us_per_step\": %.3f, \"pack_ahead_host_us_per_step\": %.3f, \"pipelined_over_kernel\": %.4f, "
        "\"pack_ahead_over_kernel\": %.4f, \"decode_us_median\": %.3f, \"decode_logical_GBps\": %.1f, \"decode_unique_GBps\": "
        "%.1f, \"decode_tokens_per_s\": %.1f, \"checked_elements\": %zu, \"worst_excess_over_tolerance\": %.3g, "
        "\"decode_within_tolerance\": %s}\n",
        layers, prompts, branches, copies.size(), pending, static_cast<unsigned long long>(copy_launches), fused_us,
        (copy_bytes + row_bytes) / (fused_us * 1e-6) / 1e9, copy_us, two_launch_us, frames_equal ? "true" : "false", copies_equal ? "true" : "false", nb,
        ctx, step_ms * 1e3, piped.loop.gpu_us_per_step, piped.ahead.gpu_us_per_step, piped.loop.host_us_per_step,
        piped.ahead.host_us_per_step, piped.loop.gpu_us_per_step / (decode_ms * 1e3),
        piped.ahead.gpu_us_per_step / (decode_ms * 1e3), decode_ms * 1e3, (logical + qo) / (decode_ms * 1e-3) / 1e9,
        (unique + qo) / (decode_ms * 1e-3) / 1e9,
        nb / (decode_ms * 1e-3), checked, worst, worst <= 0.0 ? "true" : "false");
    (void)qvp_free(dq);
    (void)qvp_free(dout);
    (void)qvp_free(dk);
    (void)qvp_free(dv);
    (void)qvp_event_destroy(e0);
    (void)qvp_event_destroy(e1);
    return (frames_equal && copies_equal && worst <= 0.0) ? 0 : 2;
}

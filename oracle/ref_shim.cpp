// ref_shim.cpp - C entry points over the REFERENCE implementation itself.
//
// TEST INFRASTRUCTURE. oracle/Makefile compiles this file together with the
// reference's own sources (src/*.cpp under the QwenVL-Paged tree, headers from
// its include/) into oracle/_ref/libqvp_ref.so, which is not committed. It lets
// the tests pin oracle/oracle.c against the real paged_attention_decode<T>
// (include/qwenvl_paged/PagedAttention.h:53-127) and lets bench.py time the
// reference CPU path on the GPU box's host cores.
//
// Nothing here re-implements the reference: it only constructs the reference's
// public objects (MemoryAllocator, BlockTable, CacheView) and calls them.
#include "qwenvl_paged/Block.h"
#include "qwenvl_paged/BlockTable.h"
#include "qwenvl_paged/CacheLayout.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/PagedAttention.h"
#include "qwenvl_paged/Scheduler.h"
#include "qwenvl_paged/SwapBackend.h"
#include "trace_driver.h"

#include <immintrin.h>

#include <atomic>
#include <chrono>
#include <thread>
#include <cstring>
#include <memory>
#include <vector>

namespace {

using namespace qwenvl_paged;

// Element type the reference template is instantiated with for bf16 caches:
// two bytes, explicit conversions to and from float (the template only needs
// sizeof(T) == bytes_per_element and static_cast in both directions,
// PagedAttention.h:64,103,116,122). Narrowing rounds to nearest even.
struct Bf16 {
    std::uint16_t bits;
    Bf16() = default;
    explicit Bf16(float f) {
        std::uint32_t u;
        std::memcpy(&u, &f, 4);
        if ((u & 0x7fffffffu) > 0x7f800000u) {
            bits = static_cast<std::uint16_t>((u >> 16) | 0x40u);
        } else {
            bits = static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
        }
    }
    explicit operator float() const {
        const std::uint32_t u = static_cast<std::uint32_t>(bits) << 16;
        float f;
        std::memcpy(&f, &u, 4);
        return f;
    }
};
static_assert(sizeof(Bf16) == 2, "bf16 must be two bytes");

// IEEE binary16 element type for fp16 caches. The conversions are the x86
// F16C instructions (vcvtps2ph with round-to-nearest-even, vcvtph2ps): a
// hardware implementation independent of oracle.c's bit manipulation, so
// the decode check below pins the oracle's fp16 arithmetic and conversions.
__attribute__((target("f16c"))) std::uint16_t half_from_float(float f) {
    return static_cast<std::uint16_t>(_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT));
}
__attribute__((target("f16c"))) float float_from_half(std::uint16_t h) { return _cvtsh_ss(h); }

struct Half {
    std::uint16_t bits;
    Half() = default;
    explicit Half(float f) : bits(half_from_float(f)) {}
    explicit operator float() const { return float_from_half(bits); }
};
static_assert(sizeof(Half) == 2, "half must be two bytes");

struct Session {
    BlockShape shape{};
    std::unique_ptr<MemoryAllocator> allocator;
};

// Decodes every sequence with the reference's paged_attention_decode<T>,
// one call per sequence; with threads > 1 the sequences are dealt
// round-robin to that many threads (the calls only read the allocator and
// their own tables).
template <typename T>
int decode_all(Session& s, std::uint32_t num_seqs, const std::uint32_t* ids, const std::uint32_t* cu_blocks,
               const std::uint32_t* ctx_lens, const void* query, std::uint32_t layer, std::uint32_t hq,
               float scale, void* out, double* seconds, std::uint32_t threads = 1) {
    const std::size_t per_seq = static_cast<std::size_t>(hq) * s.shape.head_dim;
    std::vector<BlockTable> tables;
    tables.reserve(num_seqs);
    for (std::uint32_t b = 0; b < num_seqs; ++b) {
        BlockTable table(b + 1);
        for (std::uint32_t j = cu_blocks[b]; j < cu_blocks[b + 1]; ++j) {
            const std::uint32_t index = j - cu_blocks[b];
            LogicalBlock logical;
            logical.sequence_id = b + 1;
            logical.index = index;
            logical.start_token = index * s.shape.tokens_per_block;
            logical.token_count = s.shape.tokens_per_block;
            if (ids[j] != 0xFFFFFFFFu) table.map(logical, ids[j], true);
        }
        tables.push_back(std::move(table));
    }
    std::atomic<int> refused{0};
    auto run = [&](std::uint32_t first, std::uint32_t step) {
        for (std::uint32_t b = first; b < num_seqs; b += step) {
        CacheView view;
        view.sequence_id = b + 1;
        view.block_table = &tables[b];
        view.allocator = s.allocator.get();
        view.layout.shape = s.shape;
        PagedAttentionParams params;
        params.layer = layer;
        params.num_query_heads = hq;
        params.context_len = ctx_lens[b];
        params.scale = scale;
        const T* q = static_cast<const T*>(query) + b * per_seq;
        T* o = static_cast<T*>(out) + b * per_seq;
        if (!paged_attention_decode<T>(view, q, params, o)) ++refused;
        }
    };
    const auto t0 = std::chrono::steady_clock::now();
    if (threads <= 1) {
        run(0, 1);
    } else {
        std::vector<std::thread> pool;
        for (std::uint32_t t = 0; t < threads; ++t) pool.emplace_back(run, t, threads);
        for (std::thread& th : pool) th.join();
    }
    const auto t1 = std::chrono::steady_clock::now();
    if (seconds != nullptr) *seconds = std::chrono::duration<double>(t1 - t0).count();
    return refused.load();
}

}  // namespace

extern "C" {

// Builds a reference MemoryAllocator of num_blocks frames and copies frame i of
// the flat pool (stride bytes apart) into block(i)->data().
void* ref_session_create(const std::uint8_t* pool, std::uint64_t stride, std::uint32_t num_blocks,
                         std::uint32_t tpb, std::uint32_t num_layers, std::uint32_t num_kv_heads,
                         std::uint32_t head_dim, std::uint32_t bytes_per_element) {
    auto* s = new Session();
    s->shape.tokens_per_block = tpb;
    s->shape.num_layers = num_layers;
    s->shape.num_kv_heads = num_kv_heads;
    s->shape.head_dim = head_dim;
    s->shape.bytes_per_element = bytes_per_element;
    AllocatorConfig config;
    config.block_shape = s->shape;
    config.max_blocks = num_blocks;
    s->allocator = std::make_unique<MemoryAllocator>(config);
    for (std::uint32_t i = 0; i < num_blocks; ++i) {
        PhysicalBlock* blk = s->allocator->block(i);
        const std::size_t n = blk->size_bytes() < stride ? blk->size_bytes() : stride;
        std::memcpy(blk->data(), pool + static_cast<std::uint64_t>(i) * stride, n);
    }
    return s;
}

void ref_session_destroy(void* session) { delete static_cast<Session*>(session); }

// Runs paged_attention_decode<T> for every sequence; dtype 0 = float, 1 =
// bf16, 2 = fp16. Returns the number of refused sequences, or -1 for an
// unsupported dtype.
int ref_session_decode(void* session, std::uint32_t num_seqs, const std::uint32_t* ids,
                       const std::uint32_t* cu_blocks, const std::uint32_t* ctx_lens, int dtype,
                       const void* query, std::uint32_t layer, std::uint32_t hq, float scale, void* out,
                       double* seconds) {
    Session& s = *static_cast<Session*>(session);
    if (dtype == 0) return decode_all<float>(s, num_seqs, ids, cu_blocks, ctx_lens, query, layer, hq, scale, out, seconds);
    if (dtype == 1) return decode_all<Bf16>(s, num_seqs, ids, cu_blocks, ctx_lens, query, layer, hq, scale, out, seconds);
    if (dtype == 2) return decode_all<Half>(s, num_seqs, ids, cu_blocks, ctx_lens, query, layer, hq, scale, out, seconds);
    return -1;
}

// ref_session_decode with the sequences spread over `threads` threads.
int ref_session_decode_threads(void* session, std::uint32_t num_seqs, const std::uint32_t* ids,
                               const std::uint32_t* cu_blocks, const std::uint32_t* ctx_lens, int dtype,
                               const void* query, std::uint32_t layer, std::uint32_t hq, float scale, void* out,
                               double* seconds, std::uint32_t threads) {
    Session& s = *static_cast<Session*>(session);
    if (dtype == 0) {
        return decode_all<float>(s, num_seqs, ids, cu_blocks, ctx_lens, query, layer, hq, scale, out, seconds, threads);
    }
    if (dtype == 1) {
        return decode_all<Bf16>(s, num_seqs, ids, cu_blocks, ctx_lens, query, layer, hq, scale, out, seconds, threads);
    }
    if (dtype == 2) {
        return decode_all<Half>(s, num_seqs, ids, cu_blocks, ctx_lens, query, layer, hq, scale, out, seconds, threads);
    }
    return -1;
}

// The shim's fp16 conversions, for the tests that check them against numpy.
std::uint16_t ref_half_from_float(float f) { return half_from_float(f); }
float ref_float_from_half(std::uint16_t h) { return float_from_half(h); }

std::uint64_t ref_block_byte_size(std::uint32_t tpb, std::uint32_t layers, std::uint32_t heads,
                                  std::uint32_t dim, std::uint32_t bpe) {
    BlockShape shape;
    shape.tokens_per_block = tpb;
    shape.num_layers = layers;
    shape.num_kv_heads = heads;
    shape.head_dim = dim;
    shape.bytes_per_element = bpe;
    return shape.byte_size();
}

std::uint64_t ref_block_size_bytes(std::uint32_t tpb, std::uint32_t layers, std::uint32_t heads,
                                   std::uint32_t dim, std::uint32_t bpe, std::uint64_t alignment) {
    BlockShape shape;
    shape.tokens_per_block = tpb;
    shape.num_layers = layers;
    shape.num_kv_heads = heads;
    shape.head_dim = dim;
    shape.bytes_per_element = bpe;
    HostMemoryOptions options;
    options.alignment_bytes = alignment;
    PhysicalBlock block(0, shape, options);
    return block.size_bytes();
}

std::int64_t ref_element_offset(std::uint32_t tpb, std::uint32_t layers, std::uint32_t heads,
                                std::uint32_t dim, std::uint32_t layer, std::uint32_t stream,
                                std::uint32_t token, std::uint32_t head) {
    KVBlockLayout layout;
    layout.shape.tokens_per_block = tpb;
    layout.shape.num_layers = layers;
    layout.shape.num_kv_heads = heads;
    layout.shape.head_dim = dim;
    layout.shape.bytes_per_element = 4;
    const auto off = layout.element_offset(layer, stream == 0 ? KVStream::Key : KVStream::Value, token, head);
    return off.has_value() ? static_cast<std::int64_t>(*off) : -1;
}

namespace {

std::uint64_t run_reference_trace(const trace::Config& c, char* out, std::uint64_t cap) {
    AllocatorConfig config;
    config.block_shape.tokens_per_block = c.tokens_per_block;
    config.block_shape.num_layers = 1;
    config.block_shape.num_kv_heads = 1;
    config.block_shape.head_dim = 8;
    config.block_shape.bytes_per_element = 4;
    config.max_blocks = trace::pool_blocks(c);
    MemoryAllocator allocator(config);
    HostSwapBackend swap(1u << 20);
    allocator.set_swap_backend(&swap);
    const std::string log =
        trace::run<MemoryAllocator, KVCacheManager, Scheduler, SchedulerConfig, Request, RequestState>(c, allocator);
    if (cap > 0) {
        const std::size_t n = log.size() < cap - 1 ? log.size() : cap - 1;
        std::memcpy(out, log.data(), n);
        out[n] = '\0';
    }
    return log.size();
}

}  // namespace

// The trace with every parameter given: cfg = {requests, prompt_lo,
// prompt_hi, output_lo, output_hi, arrivals_per_step, tokens_per_block,
// pool_percent, watermark_blocks, max_active, max_batch_tokens, max_steps,
// cancel_after_decodes}.
std::uint64_t ref_scheduler_trace_config(const std::uint32_t* cfg, std::uint64_t seed, char* out, std::uint64_t cap) {
    trace::Config c;
    c.requests = cfg[0];
    c.prompt_lo = cfg[1];
    c.prompt_hi = cfg[2];
    c.output_lo = cfg[3];
    c.output_hi = cfg[4];
    c.arrivals_per_step = cfg[5];
    c.tokens_per_block = cfg[6];
    c.pool_percent = cfg[7];
    c.watermark_blocks = cfg[8];
    c.max_active = cfg[9];
    c.max_batch_tokens = cfg[10];
    c.max_steps = cfg[11];
    c.cancel_after_decodes = cfg[12] != 0;
    c.seed = seed;
    return run_reference_trace(c, out, cap);
}

// Runs the continuous-batching trace of trace_driver.h on the reference's own
// Scheduler / KVCacheManager / MemoryAllocator / HostSwapBackend and copies the
// event log into `out` (NUL-terminated, truncated to `cap`). Returns the full
// log length.
std::uint64_t ref_scheduler_trace(std::uint32_t requests, std::uint64_t seed, std::uint32_t pool_percent,
                                  std::uint32_t watermark_blocks, char* out, std::uint64_t cap) {
    trace::Config c;
    c.requests = requests;
    c.seed = seed;
    c.pool_percent = pool_percent;
    c.watermark_blocks = watermark_blocks;
    return run_reference_trace(c, out, cap);
}

}  // extern "C"

// Shared set-up of the device-placement suites: an HBM block pool, a pinned
// swap arena and a cache manager, plus host-side writers that go through the
// copy-on-write point exactly like an attention backend's K/V append, and a
// float64 textbook attention used as the expected result.
#pragma once

#include "minitest.h"
#include "qwenvl_paged/CacheLayout.h"
#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"
#include "qwenvl_paged/PagedAttention.h"
#include "qwenvl_paged/Scheduler.h"
#include "qwenvl_paged/SwapBackend.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

namespace device_test {

using namespace qwenvl_paged;

inline BlockShape shape_of(std::uint32_t tpb, std::uint32_t layers, std::uint32_t kv_heads, std::uint32_t dim,
                           std::uint32_t bpe = 4) {
    BlockShape s;
    s.tokens_per_block = tpb;
    s.num_layers = layers;
    s.num_kv_heads = kv_heads;
    s.head_dim = dim;
    s.bytes_per_element = bpe;
    return s;
}

inline AllocatorConfig device_config(BlockShape shape, std::uint32_t blocks) {
    AllocatorConfig c;
    c.block_shape = shape;
    c.max_blocks = blocks;
    c.placement = BlockPlacement::Device;
    return c;
}

// Member order matters: the pinned backend is destroyed before the allocator.
struct DeviceHarness {
    DeviceHarness(BlockShape shape, std::uint32_t blocks, std::size_t swap_slots = 64)
        : allocator(device_config(shape, blocks)), swap(allocator, swap_slots), cache(allocator) {
        allocator.set_swap_backend(&swap);
        layout.shape = shape;
    }

    [[nodiscard]] bool ready() const { return allocator.ok() && swap.ok(); }

    MemoryAllocator allocator;
    PinnedSwapBackend swap;
    KVCacheManager cache;
    KVBlockLayout layout{};
};

// Same wiring over host frames: the reference's own placement, used as the
// expected state when device and host engines replay the same operations.
struct HostHarness {
    HostHarness(BlockShape shape, std::uint32_t blocks, std::size_t swap_slots = 64)
        : allocator(host_config(shape, blocks)), swap(swap_slots), cache(allocator) {
        allocator.set_swap_backend(&swap);
        layout.shape = shape;
    }
    static AllocatorConfig host_config(BlockShape shape, std::uint32_t blocks) {
        AllocatorConfig c;
        c.block_shape = shape;
        c.max_blocks = blocks;
        return c;
    }
    MemoryAllocator allocator;
    HostSwapBackend swap;
    KVCacheManager cache;
    KVBlockLayout layout{};
};

// Writes one head vector of element type T through ensure_token_writable.
template <typename Harness, typename T>
bool write_head(Harness& h, SequenceId seq, KVStream stream, std::uint32_t layer, TokenPosition token,
                std::uint32_t kv_head, const std::vector<T>& v) {
    const auto frame = h.cache.ensure_token_writable(seq, token);
    if (!frame) return false;
    const auto off = h.layout.element_offset(layer, stream, token % h.layout.shape.tokens_per_block, kv_head);
    if (!off || v.size() != h.layout.shape.head_dim || sizeof(T) != h.layout.shape.bytes_per_element) return false;
    return h.allocator.write_block_bytes(*frame, *off * sizeof(T), v.data(), v.size() * sizeof(T));
}

// Deterministic contents in [-1, 1) from an FNV-1a mix of the coordinates.
inline float mix_pattern(std::initializer_list<std::uint32_t> parts) {
    std::uint32_t x = 2166136261u;
    for (std::uint32_t p : parts) x = (x ^ p) * 16777619u;
    return static_cast<float>(x % 2000u) / 1000.0f - 1.0f;
}

// Softmax attention of one query over `ctx` tokens, in float64.
// key(t, h, d) / value(t, h, d) give the cached vectors of kv head h.
template <typename KeyFn, typename ValueFn>
std::vector<double> textbook_attention(const std::vector<float>& query, std::uint32_t num_q_heads,
                                       std::uint32_t num_kv_heads, std::uint32_t dim, std::uint32_t ctx, float scale,
                                       KeyFn key, ValueFn value) {
    const std::uint32_t group = num_q_heads / num_kv_heads;
    std::vector<double> out(static_cast<std::size_t>(num_q_heads) * dim, 0.0);
    std::vector<double> s(ctx);
    for (std::uint32_t qh = 0; qh < num_q_heads; ++qh) {
        const std::uint32_t kh = qh / group;
        double m = -std::numeric_limits<double>::infinity();
        for (std::uint32_t t = 0; t < ctx; ++t) {
            double dot = 0.0;
            for (std::uint32_t d = 0; d < dim; ++d) dot += static_cast<double>(query[qh * dim + d]) * key(t, kh, d);
            s[t] = dot * scale;
            m = std::max(m, s[t]);
        }
        double l = 0.0;
        for (std::uint32_t t = 0; t < ctx; ++t) {
            const double w = std::exp(s[t] - m);
            l += w;
            for (std::uint32_t d = 0; d < dim; ++d) out[qh * dim + d] += w * value(t, kh, d);
        }
        for (std::uint32_t d = 0; d < dim; ++d) out[qh * dim + d] /= l;
    }
    return out;
}

inline bool scattered(const BlockTable& t) {
    const auto& e = t.entries();
    if (e.size() < 2) return false;
    PhysicalBlockId lo = e.front().physical_id, hi = lo;
    for (const BlockTableEntry& x : e) {
        lo = std::min(lo, x.physical_id);
        hi = std::max(hi, x.physical_id);
    }
    return hi - lo + 1 != e.size();
}

}  // namespace device_test

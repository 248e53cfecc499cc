// KV append: writes the new tokens' K and V rows into their paged frames.
//
// In the reference a model (its test harnesses, tests/PagedAttention.test.cpp:97-127
// and tests/EndToEnd.test.cpp:157-179) asks KVCacheManager::ensure_token_writable
// for the frame of token position p (copying a shared block first,
// src/KVCacheManager.cpp:104-151) and then stores head_dim elements per
// (layer, stream, kv head) at KVBlockLayout::element_offset(layer, stream,
// p % tokens_per_block, head) (src/CacheLayout.cpp:25-38) of that frame. Here
// one launch does those stores for a whole step: the host turns each token's
// (frame, slot) into the byte offset of its token row, validates everything
// before anything is enqueued, and passes the offsets in the kernel arguments
// (up to 128 tokens a launch: a decode step) or, for longer lists such as a
// prompt, uploads them once through pinned staging and covers every token in
// one launch; one wave per (token, layer, stream) copies the kv heads' rows
// with 16-byte accesses. The source is the step's K (and V) tensor,
// [count][layer_count][num_kv_heads][head_dim], already on the device.
#include "common.h"

#include <algorithm>
#include <mutex>
#include <utility>
#include <vector>

namespace {

using qvp::fail;

constexpr int kAppendTokensPerLaunch = 128;
constexpr int kAppendThreads = 64;
constexpr uint32_t kAppendMaxTokens = 1u << 24;

struct AppendRows {
    uint64_t offset[kAppendTokensPerLaunch];  // byte offset of the token's row in the pool
};

struct AppendGeometry {
    uint8_t* base;
    const uint8_t* k;
    const uint8_t* v;
    uint64_t head_stride;    // bytes
    uint64_t stream_stride;  // bytes
    uint64_t layer_stride;   // bytes
    uint32_t first_token;    // index of this launch's first token in k / v
    uint32_t first_layer;
    uint32_t layer_count;
    uint32_t num_kv_heads;
    uint32_t row_bytes;  // head_dim * element size
    uint32_t vec;        // 16-byte path usable
};

// Block (token, l, s) of a launch: copies the kv heads' rows of source token
// `token`, layer l, stream s to the token row at byte `offset` of the pool.
__device__ inline void copy_token(const AppendGeometry& g, uint32_t token, uint64_t offset) {
    const uint32_t l = blockIdx.y;
    const uint32_t s = blockIdx.z;
    const uint64_t src_row = (static_cast<uint64_t>(token) * g.layer_count + l) * g.num_kv_heads;
    const uint8_t* src = (s == 0 ? g.k : g.v) + src_row * g.row_bytes;
    uint8_t* dst = g.base + offset + static_cast<uint64_t>(g.first_layer + l) * g.layer_stride +
                   static_cast<uint64_t>(s) * g.stream_stride;
    if (g.vec != 0) {
        const uint32_t chunks = g.row_bytes / 16;
        const uint32_t total = chunks * g.num_kv_heads;
        for (uint32_t e = threadIdx.x; e < total; e += kAppendThreads) {
            const uint32_t h = e / chunks;
            const uint32_t c = e - h * chunks;
            *reinterpret_cast<uint4*>(dst + h * g.head_stride + 16u * c) =
                *reinterpret_cast<const uint4*>(src + static_cast<uint64_t>(h) * g.row_bytes + 16u * c);
        }
        return;
    }
    const uint32_t total = g.row_bytes * g.num_kv_heads;
    for (uint32_t e = threadIdx.x; e < total; e += kAppendThreads) {
        const uint32_t h = e / g.row_bytes;
        const uint32_t c = e - h * g.row_bytes;
        dst[h * g.head_stride + c] = src[static_cast<uint64_t>(h) * g.row_bytes + c];
    }
}

// Offsets in the kernel arguments: block i copies token first_token + i.
__global__ __launch_bounds__(kAppendThreads) void append_rows(AppendGeometry g, AppendRows rows) {
    copy_token(g, g.first_token + blockIdx.x, rows.offset[blockIdx.x]);
}

// Offsets uploaded to device memory: block i copies token i of the list.
__global__ __launch_bounds__(kAppendThreads) void append_rows_list(AppendGeometry g,
                                                                   const uint64_t* __restrict__ offsets) {
    copy_token(g, blockIdx.x, offsets[blockIdx.x]);
}

// Row-offset staging of the list path, shared by all calls of the process
// (one engine thread per pool): two pinned buffers, each with the event of
// its last host-to-device copy, and two device buffers, each with the event
// of the last kernel that read it. A call refills slot `parity` after its
// previous copy has left the host buffer, and its stream waits for the
// slot's previous kernel before the new copy overwrites the device buffer.
struct AppendStaging {
    std::mutex mu;
    uint64_t* host[2]{nullptr, nullptr};
    uint64_t* device[2]{nullptr, nullptr};
    size_t cap[2]{0, 0};
    hipEvent_t copied[2]{nullptr, nullptr};
    hipEvent_t consumed[2]{nullptr, nullptr};
    bool copy_pending[2]{false, false};
    bool kernel_pending[2]{false, false};
    int parity{0};
};

AppendStaging& staging() {
    static AppendStaging s;
    return s;
}

int launch_list(const AppendGeometry& g, const uint32_t* frames, const uint32_t* slots, uint32_t count,
                uint64_t block_stride, uint64_t token_stride, uint32_t layer_count, hipStream_t st) {
    AppendStaging& sg = staging();
    std::lock_guard<std::mutex> lock(sg.mu);
    const int k = sg.parity;
    if (sg.copied[k] == nullptr) QVP_HIP(hipEventCreateWithFlags(&sg.copied[k], hipEventDisableTiming));
    if (sg.consumed[k] == nullptr) QVP_HIP(hipEventCreateWithFlags(&sg.consumed[k], hipEventDisableTiming));
    if (sg.copy_pending[k]) {
        QVP_HIP(hipEventSynchronize(sg.copied[k]));
        sg.copy_pending[k] = false;
    }
    if (sg.cap[k] < count) {
        // Growing: the old buffers may still be read by an earlier kernel.
        if (sg.kernel_pending[k]) QVP_HIP(hipEventSynchronize(sg.consumed[k]));
        sg.kernel_pending[k] = false;
        if (sg.host[k] != nullptr) QVP_HIP(hipHostFree(sg.host[k]));
        if (sg.device[k] != nullptr) QVP_HIP(hipFree(sg.device[k]));
        sg.host[k] = nullptr;
        sg.device[k] = nullptr;
        sg.cap[k] = 0;
        const size_t cap = std::max<size_t>(count, 4096);
        QVP_HIP(hipHostMalloc(reinterpret_cast<void**>(&sg.host[k]), cap * sizeof(uint64_t), hipHostMallocCoherent));
        QVP_HIP(hipMalloc(reinterpret_cast<void**>(&sg.device[k]), cap * sizeof(uint64_t)));
        sg.cap[k] = cap;
    }
    for (uint32_t i = 0; i < count; ++i) {
        sg.host[k][i] = static_cast<uint64_t>(frames[i]) * block_stride + static_cast<uint64_t>(slots[i]) * token_stride;
    }
    if (sg.kernel_pending[k]) QVP_HIP(hipStreamWaitEvent(st, sg.consumed[k], 0));
    QVP_TRY(qvp::pull_from_pinned(sg.device[k], sg.host[k], count * sizeof(uint64_t), st));
    QVP_HIP(hipEventRecord(sg.copied[k], st));
    sg.copy_pending[k] = true;
    hipLaunchKernelGGL(append_rows_list, dim3(count, layer_count, 2), dim3(kAppendThreads), 0, st, g, sg.device[k]);
    QVP_HIP(hipGetLastError());
    QVP_HIP(hipEventRecord(sg.consumed[k], st));
    sg.kernel_pending[k] = true;
    sg.parity ^= 1;
    return QVP_OK;
}

}  // namespace

extern "C" int qvp_append_kv(const qvp_append_args* a, const uint32_t* frames, const uint32_t* slots,
                             uint32_t count, void* stream) {
    if (a == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "args is NULL");
    if (count == 0) return QVP_OK;
    if (frames == nullptr || slots == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "frames or slots is NULL");
    // One launch's grid holds every token (a dispatch counts work-items in 32 bits).
    if (count > kAppendMaxTokens) return fail(QVP_ERR_INVALID_ARGUMENT, "%u tokens in one call, limit %u", count, kAppendMaxTokens);
    if (a->kv_base == nullptr || a->k == nullptr || a->v == nullptr) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "kv_base, k or v is NULL");
    }
    const uint64_t bpe = qvp::dtype_size(a->kv_dtype);
    if (bpe == 0) return fail(QVP_ERR_INVALID_ARGUMENT, "unknown kv_dtype %u", a->kv_dtype);
    if (a->num_blocks == 0 || a->tokens_per_block == 0 || a->num_kv_heads == 0 || a->head_dim == 0 ||
        a->num_layers == 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "zero pool size, tokens_per_block, num_kv_heads, head_dim or num_layers");
    }
    if (a->layer_count == 0 || a->layer_count > 65535 ||
        static_cast<uint64_t>(a->first_layer) + a->layer_count > a->num_layers) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "layers [%u, +%u) outside %u layers", a->first_layer, a->layer_count,
                    a->num_layers);
    }
    // Every (layer, stream, slot, head, dim) must name its own element, and the
    // highest one must lie inside the frame (CacheLayout.cpp:25-38 with the
    // reference's strides satisfies both).
    const uint64_t D = a->head_dim;
    const uint64_t head_span = (static_cast<uint64_t>(a->num_kv_heads) - 1) * a->head_stride + D;
    const uint64_t token_span = (static_cast<uint64_t>(a->tokens_per_block) - 1) * a->token_stride + head_span;
    if (a->head_stride < D || a->token_stride < head_span || a->stream_stride < token_span ||
        a->layer_stride < a->stream_stride + token_span) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "strides make rows overlap");
    }
    const uint64_t extent =
        ((static_cast<uint64_t>(a->num_layers) - 1) * a->layer_stride + a->stream_stride + token_span) * bpe;
    if (extent > a->block_stride) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "layout spans %llu bytes, frame stride is %llu",
                    static_cast<unsigned long long>(extent), static_cast<unsigned long long>(a->block_stride));
    }
    std::vector<std::pair<uint32_t, uint32_t>> targets(count);
    for (uint32_t i = 0; i < count; ++i) {
        if (frames[i] >= a->num_blocks) {
            return fail(QVP_ERR_UNMAPPED, "frame %u of token %u outside pool of %u blocks", frames[i], i,
                        a->num_blocks);
        }
        if (slots[i] >= a->tokens_per_block) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "slot %u of token %u >= tokens_per_block %u", slots[i], i,
                        a->tokens_per_block);
        }
        targets[i] = {frames[i], slots[i]};
    }
    std::sort(targets.begin(), targets.end());
    for (uint32_t i = 1; i < count; ++i) {
        if (targets[i] == targets[i - 1]) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "frame %u slot %u written twice", targets[i].first,
                        targets[i].second);
        }
    }

    AppendGeometry g{};
    g.base = static_cast<uint8_t*>(a->kv_base);
    g.k = static_cast<const uint8_t*>(a->k);
    g.v = static_cast<const uint8_t*>(a->v);
    g.head_stride = a->head_stride * bpe;
    g.stream_stride = a->stream_stride * bpe;
    g.layer_stride = a->layer_stride * bpe;
    g.first_layer = a->first_layer;
    g.layer_count = a->layer_count;
    g.num_kv_heads = a->num_kv_heads;
    g.row_bytes = static_cast<uint32_t>(D * bpe);
    const uint64_t token_stride = a->token_stride * bpe;
    const uint64_t align = reinterpret_cast<uintptr_t>(a->kv_base) | reinterpret_cast<uintptr_t>(a->k) |
                           reinterpret_cast<uintptr_t>(a->v) | a->block_stride | g.head_stride | g.stream_stride |
                           g.layer_stride | token_stride | g.row_bytes;
    g.vec = (align % 16 == 0) ? 1u : 0u;
    const hipStream_t st = qvp::as_stream(stream);
    if (count > kAppendTokensPerLaunch) {
        // A graph must not depend on host staging that later calls refill: under
        // capture the offsets stay in the kernel arguments.
        hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
        QVP_HIP(hipStreamIsCapturing(st, &capture));
        if (capture == hipStreamCaptureStatusNone) {
            return launch_list(g, frames, slots, count, a->block_stride, token_stride, a->layer_count, st);
        }
    }
    for (uint32_t first = 0; first < count; first += kAppendTokensPerLaunch) {
        const uint32_t n = std::min<uint32_t>(kAppendTokensPerLaunch, count - first);
        AppendRows rows{};
        for (uint32_t i = 0; i < n; ++i) {
            rows.offset[i] = static_cast<uint64_t>(frames[first + i]) * a->block_stride +
                             static_cast<uint64_t>(slots[first + i]) * token_stride;
        }
        g.first_token = first;
        hipLaunchKernelGGL(append_rows, dim3(n, a->layer_count, 2), dim3(kAppendThreads), 0, st, g, rows);
        QVP_HIP(hipGetLastError());
    }
    return QVP_OK;
}

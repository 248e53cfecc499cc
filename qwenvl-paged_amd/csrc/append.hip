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

// A copy-on-write step in one launch: frame copies (qvp_copy_blocks) and the
// step's K/V rows (qvp_append_kv) together, as one gather-copy. Every 16-byte
// unit of a destination frame is written once, from its final source: the
// K or V row of a token appended into that frame when the unit lies in one of
// its rows, else the same unit of the source frame. So the bytes equal those
// of the copy followed by the append, with no ordering inside the launch, and
// the launch moves what the copy alone moves (plus the rows). A unit's place in
// the layout -- (layer, stream, slot, kv head, byte) -- comes from its frame
// offset by division with the nested strides (magic-number division, exact
// for 32-bit offsets). Rows in frames that no pair copies are items of their
// own. Items are walked grid-stride by at most two workgroups per CU.
constexpr int kFusedThreads = 256;
constexpr int kFusedUnits = 2;  // 16-byte units per thread and item
constexpr uint32_t kFusedChunk = kFusedUnits * 16u * kFusedThreads;
constexpr uint32_t kFusedMaxPairs = 128;
constexpr uint32_t kFusedMaxRows = 128;
constexpr uint32_t kFusedMaxSlots = 64;  // the written-slot mask of a frame is 64 bits
constexpr uint32_t kFusedWgsPerCu = 4;
// Word 3 of a raw (untyped, stride 0) buffer resource on gfx9 parts, and an
// offset past any frame the fused launch takes (frames stay under 2 GiB).
constexpr int kBufferWord3 = 0x00020000;
constexpr uint32_t kDroppedOffset = 0x80000000u;
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// floor(x / d) for every 32-bit x: m = floor(2^32 (2^l - d) / d) + 1,
// l = ceil(log2 d), q = (mulhi(x, m) + x) >> l (Granlund and Montgomery,
// "Division by invariant integers using multiplication", 1994).
struct FastDiv {
    uint32_t m;
    uint32_t l;
};

FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    const uint64_t m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
    return FastDiv{static_cast<uint32_t>(m), l};
}

__device__ inline uint32_t fdiv(uint32_t x, FastDiv f) {
    return static_cast<uint32_t>((static_cast<uint64_t>(__umulhi(x, f.m)) + x) >> f.l);
}

struct FusedGeometry {
    uint8_t* base;
    const uint8_t* k;
    const uint8_t* v;
    uint64_t block_stride;
    uint32_t copy_bytes;     // bytes of each source frame copied
    uint32_t span;           // bytes of a destination frame its items cover: max(copy, row extent)
    uint32_t layer_stride;   // bytes
    uint32_t stream_stride;  // bytes
    uint32_t token_stride;   // bytes
    uint32_t head_stride;    // bytes
    FastDiv div_layer, div_token, div_head, div_words, div_heads;
    uint32_t sh_layer, sh_token, sh_head;  // log2 of the strides when all three are powers of two
    uint32_t first_layer;
    uint32_t layer_count;
    uint32_t num_kv_heads;
    uint32_t tpb;
    uint32_t row_bytes;
    uint32_t row_words;
    uint32_t num_pairs;
    uint32_t chunks_per_frame;
    uint32_t pair_items;     // pairs x chunks_per_frame
    uint32_t multi_row_pairs;  // some pair writes more than one row
    uint32_t tail_first;       // first row in an uncopied frame
    uint32_t total_items;    // pair items + rows in uncopied frames
};

// Pair p copies frame src onto dst and writes the rows row_first ..
// row_first + rows - 1, sorted by slot; slot_mask has bit t set when slot t of
// dst receives a row, `token` is the first row's token index in k / v. One
// entry per pair, read with scalar loads in one round trip. Rows from
// tail_first on are in uncopied frames (row_frame). Row r's token index is
// row_info[r] & 0xffff, its slot row_info[r] >> 16.
struct FusedPair {
    uint32_t src;
    uint32_t dst;
    uint32_t mask_lo;
    uint32_t mask_hi;
    uint32_t info;  // row_first | rows << 8 | token << 16
};

struct FusedList {
    FusedPair pair[kFusedMaxPairs];
    uint32_t row_frame[kFusedMaxRows];
    uint32_t row_info[kFusedMaxRows];
};

static_assert(sizeof(FusedList) + 256 <= 4096, "the lists travel in the kernel arguments");

// Source of the (layer lr, stream s, head h) row of token `token`, byte `byte`
// (the K and V tensors are under 4 GiB, checked).
__device__ inline const uint4* row_source(const FusedGeometry& g, uint32_t token, uint32_t lr, uint32_t s, uint32_t h,
                                          uint32_t byte) {
    const uint32_t row = (token * g.layer_count + lr) * g.num_kv_heads + h;
    return reinterpret_cast<const uint4*>((s == 0 ? g.k : g.v) + (row * g.row_bytes + byte));
}

// floor(x / d) and x - d floor(x / d) for a stride d: a shift and a mask when
// d is a power of two (kPow2; sh = log2 d), else magic-number division.
template <bool kPow2>
__device__ inline uint32_t stride_div(uint32_t x, FastDiv f, uint32_t sh) {
    if constexpr (kPow2) {
        return x >> sh;
    } else {
        return fdiv(x, f);
    }
}

template <bool kPow2, bool kOneRow>
__device__ inline void copy_append_item(const FusedGeometry& g, const FusedPair& e, const uint32_t* sm_token,
                                        uint32_t c0) {
    const uint8_t* src = g.base + static_cast<uint64_t>(e.src) * g.block_stride;
    uint8_t* dst = g.base + static_cast<uint64_t>(e.dst) * g.block_stride;
    const uint64_t mask = (static_cast<uint64_t>(e.mask_hi) << 32) | e.mask_lo;
    const uint32_t rf = e.info & 0xffu;
    const uint32_t token0 = e.info >> 16;
    // Unit off's source; `live` false: the unit is not written, and the
    // pointer is the frame's first unit (in bounds, its value unused).
    // Branch-free, so both loads issue unconditionally before the
    // stores and one wait covers them.
    auto source = [&](uint32_t off, bool& live) -> const uint4* {
        const uint32_t l = stride_div<kPow2>(off, g.div_layer, g.sh_layer);
        uint32_t rem = off - l * g.layer_stride;
        const uint32_t s = rem >= g.stream_stride ? 1u : 0u;
        rem -= s * g.stream_stride;
        const uint32_t t = stride_div<kPow2>(rem, g.div_token, g.sh_token);
        rem -= t * g.token_stride;
        const uint32_t h = stride_div<kPow2>(rem, g.div_head, g.sh_head);
        rem -= h * g.head_stride;
        const uint32_t lr = l - g.first_layer;  // wraps for layers below the range
        const bool row = lr < g.layer_count && t < g.tpb && h < g.num_kv_heads && rem < g.row_bytes &&
                         ((mask >> (t & 63u)) & 1u) != 0;
        uint32_t token = token0;
        if constexpr (!kOneRow) {
            token = sm_token[min(rf + __popcll(mask & ((1ull << (t & 63u)) - 1ull)), kFusedMaxRows - 1)];
        }
        const uint4* from_row = row_source(g, token, lr, s, h, rem);
        live = off < g.span && (row || off < g.copy_bytes);
        const uint4* from = row ? from_row : reinterpret_cast<const uint4*>(src + off);
        return live ? from : reinterpret_cast<const uint4*>(src);
    };
    uint32_t off[kFusedUnits];
    const uint4* from[kFusedUnits];
#pragma unroll
    for (int u = 0; u < kFusedUnits; ++u) {
        bool live;
        off[u] = c0 + 16u * (threadIdx.x + u * kFusedThreads);
        from[u] = source(off[u], live);
        if (!live) off[u] = kDroppedOffset;
    }
    u32x4_t w[kFusedUnits];
#pragma unroll
    for (int u = 0; u < kFusedUnits; ++u) w[u] = *reinterpret_cast<const u32x4_t*>(from[u]);
    // Stores through a buffer resource covering [0, span) of the
    // destination frame: a unit that is not written gets an offset
    // past the range, and the hardware's range check drops the store.
    // No store sits behind a branch, so no wait ends up between them.
    const __amdgpu_buffer_rsrc_t out =
        __builtin_amdgcn_make_buffer_rsrc(dst, 0, static_cast<int>(g.span), kBufferWord3);
#pragma unroll
    for (int u = 0; u < kFusedUnits; ++u) {
        __builtin_amdgcn_raw_buffer_store_b128(w[u], out, static_cast<int>(off[u]), 0, 0);
    }
}

template <bool kPow2>
__global__ __launch_bounds__(kFusedThreads) void copy_append(FusedGeometry g, FusedList L) {
    // Token of each row for pairs that write several rows (per-lane lookups;
    // an LDS read waits for nothing but itself). Staged only when such a pair
    // exists: the staging load and barrier would otherwise delay every item.
    __shared__ uint32_t sm_token[kFusedMaxRows];
    if (g.multi_row_pairs) {
        if (threadIdx.x < kFusedMaxRows) sm_token[threadIdx.x] = L.row_info[threadIdx.x] & 0xffffu;
        __syncthreads();
    }
    for (uint32_t item = blockIdx.x; item < g.total_items; item += gridDim.x) {
        if (item < g.pair_items) {
            const uint32_t p = item / g.chunks_per_frame;
            const uint32_t c0 = (item - p * g.chunks_per_frame) * kFusedChunk;
            const FusedPair e = L.pair[p];
            if (((e.info >> 8) & 0xffu) <= 1) {
                copy_append_item<kPow2, true>(g, e, sm_token, c0);
            } else {
                copy_append_item<kPow2, false>(g, e, sm_token, c0);
            }
            continue;
        }
        const uint32_t r = g.tail_first + (item - g.pair_items);
        const uint32_t info = L.row_info[r];
        uint8_t* frame = g.base + static_cast<uint64_t>(L.row_frame[r]) * g.block_stride +
                         static_cast<uint64_t>(info >> 16) * g.token_stride;
        const uint32_t units = g.layer_count * 2u * g.num_kv_heads * g.row_words;
        for (uint32_t u = threadIdx.x; u < units; u += kFusedThreads) {
            const uint32_t rest = fdiv(u, g.div_words);
            const uint32_t word = u - rest * g.row_words;
            const uint32_t ls = fdiv(rest, g.div_heads);
            const uint32_t h = rest - ls * g.num_kv_heads;
            const uint32_t s = ls & 1u;
            const uint32_t lr = ls >> 1;
            const uint64_t off = static_cast<uint64_t>(g.first_layer + lr) * g.layer_stride +
                                 static_cast<uint64_t>(s) * g.stream_stride + static_cast<uint64_t>(h) * g.head_stride +
                                 16u * word;
            *reinterpret_cast<uint4*>(frame + off) = *row_source(g, info & 0xffffu, lr, s, h, 16u * word);
        }
    }
}

// Compute units of the current device, cached per device ordinal.
std::mutex g_fused_cu_mutex;
std::vector<uint32_t> g_fused_cus;

int device_cus(uint32_t* cus) {
    int dev = 0;
    QVP_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_fused_cu_mutex);
    if (g_fused_cus.size() <= static_cast<size_t>(dev)) g_fused_cus.resize(dev + 1, 0);
    if (g_fused_cus[dev] == 0) {
        int n = 0;
        QVP_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        g_fused_cus[dev] = static_cast<uint32_t>(std::max(n, 1));
    }
    *cus = g_fused_cus[dev];
    return QVP_OK;
}

// The frames one qvp_copy_append_kv call names (at most 128 sources, 128
// destinations and 128 row frames): open addressing on a 1024-entry table.
struct FrameTable {
    struct Entry {
        uint32_t frame;
        uint32_t is_src;
        int32_t pair;   // destination of pair `pair`, or -1
        uint64_t rows;  // slots written by the call's rows
    };
    static constexpr uint32_t kSize = 1024;
    static constexpr uint32_t kEmpty = 0xffffffffu;
    Entry e[kSize];
    FrameTable() {
        for (Entry& x : e) x.frame = kEmpty;
    }
    Entry& find(uint32_t frame) {
        uint32_t h = (frame * 2654435761u) >> 22;  // Knuth's multiplicative hash, 10 bits
        while (e[h].frame != frame && e[h].frame != kEmpty) h = (h + 1) & (kSize - 1);
        if (e[h].frame == kEmpty) e[h] = Entry{frame, 0, -1, 0};
        return e[h];
    }
};

// Checks of qvp_append_kv shared by the fused entry: geometry, frames, slots,
// duplicates. Fills g's layout fields; *vec tells whether 16-byte words work.
// check_duplicates false: the caller finds a (frame, slot) given twice itself.
int check_append(const qvp_append_args* a, const uint32_t* frames, const uint32_t* slots, uint32_t count,
                 uint64_t* bpe_out, uint64_t* token_stride_out, bool* vec_out, bool check_duplicates = true) {
    if (a == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "args is NULL");
    if (count > 0 && (frames == nullptr || slots == nullptr)) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "frames or slots is NULL");
    }
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
    std::vector<std::pair<uint32_t, uint32_t>> targets(check_duplicates ? count : 0);
    for (uint32_t i = 0; i < count; ++i) {
        if (frames[i] >= a->num_blocks) {
            return fail(QVP_ERR_UNMAPPED, "frame %u of token %u outside pool of %u blocks", frames[i], i,
                        a->num_blocks);
        }
        if (slots[i] >= a->tokens_per_block) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "slot %u of token %u >= tokens_per_block %u", slots[i], i,
                        a->tokens_per_block);
        }
        if (check_duplicates) targets[i] = {frames[i], slots[i]};
    }
    if (check_duplicates) {
        std::sort(targets.begin(), targets.end());
        for (uint32_t i = 1; i < count; ++i) {
            if (targets[i] == targets[i - 1]) {
                return fail(QVP_ERR_INVALID_ARGUMENT, "frame %u slot %u written twice", targets[i].first,
                            targets[i].second);
            }
        }
    }
    const uint64_t token_stride = a->token_stride * bpe;
    const uint64_t align = reinterpret_cast<uintptr_t>(a->kv_base) | reinterpret_cast<uintptr_t>(a->k) |
                           reinterpret_cast<uintptr_t>(a->v) | a->block_stride | a->head_stride * bpe |
                           a->stream_stride * bpe | a->layer_stride * bpe | token_stride | D * bpe;
    *bpe_out = bpe;
    *token_stride_out = token_stride;
    *vec_out = align % 16 == 0;
    return QVP_OK;
}

}  // namespace

extern "C" int qvp_append_kv(const qvp_append_args* a, const uint32_t* frames, const uint32_t* slots,
                             uint32_t count, void* stream) {
    if (a == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "args is NULL");
    if (count == 0) return QVP_OK;
    uint64_t bpe = 0, token_stride = 0;
    bool vec = false;
    QVP_TRY(check_append(a, frames, slots, count, &bpe, &token_stride, &vec));
    const uint64_t D = a->head_dim;
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
    g.vec = vec ? 1u : 0u;
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

extern "C" int qvp_copy_append_kv(const qvp_append_args* a, const uint32_t* src_ids, const uint32_t* dst_ids,
                                  uint32_t num_pairs, uint64_t copy_bytes, const uint32_t* frames,
                                  const uint32_t* slots, uint32_t count, void* stream) {
    if (a == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "args is NULL");
    if (num_pairs == 0 && count == 0) return QVP_OK;
    if (num_pairs > kFusedMaxPairs || count > kFusedMaxRows) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "%u copies and %u rows in one call, limits %u and %u", num_pairs, count,
                    kFusedMaxPairs, kFusedMaxRows);
    }
    // Frame offsets, chunk ends included, stay below the dropped-store offset.
    if (a->block_stride > kDroppedOffset - kFusedChunk || a->tokens_per_block > kFusedMaxSlots) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "frames of 2 GiB or more, or more than %u tokens per block",
                    kFusedMaxSlots);
    }
    uint64_t bpe = 0, token_stride = 0;
    bool vec = false;
    QVP_TRY(check_append(a, frames, slots, count, &bpe, &token_stride, &vec, false));
    if (!vec) return fail(QVP_ERR_INVALID_ARGUMENT, "pool, rows and strides must be 16-byte aligned");
    if (static_cast<uint64_t>(count) * a->layer_count * a->num_kv_heads * a->head_dim * bpe > 0xffffffffull) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "K and V tensors of 4 GiB or more");
    }
    if (num_pairs > 0 && (src_ids == nullptr || dst_ids == nullptr)) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "src_ids or dst_ids is NULL");
    }
    if (copy_bytes > a->block_stride || copy_bytes % 16 != 0 || (num_pairs > 0 && copy_bytes == 0)) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "copy of %llu bytes: at most the frame stride %llu, a multiple of 16",
                    static_cast<unsigned long long>(copy_bytes), static_cast<unsigned long long>(a->block_stride));
    }
    // The qvp_copy_blocks rules -- frames inside the pool, distinct
    // destinations, no destination that is another pair's source -- plus no
    // row in a frame a pair reads (it would race the copy) and no (frame,
    // slot) given twice, found through a table of the call's frames (at most
    // 384 distinct ones), in time linear in the lists. A pair with src == dst
    // is a no-op, as in qvp_copy_blocks.
    FrameTable table;
    for (uint32_t i = 0; i < num_pairs; ++i) {
        if (src_ids[i] >= a->num_blocks || dst_ids[i] >= a->num_blocks) {
            return fail(QVP_ERR_UNMAPPED, "copy %u (%u -> %u) outside pool of %u blocks", i, src_ids[i], dst_ids[i],
                        a->num_blocks);
        }
        if (src_ids[i] != dst_ids[i]) table.find(src_ids[i]).is_src = 1;
    }
    FusedList L{};
    uint32_t pairs = 0;
    FrameTable::Entry* pair_entry[kFusedMaxPairs];
    for (uint32_t i = 0; i < num_pairs; ++i) {
        if (src_ids[i] == dst_ids[i]) continue;
        FrameTable::Entry& d = table.find(dst_ids[i]);
        if (d.is_src) return fail(QVP_ERR_INVALID_ARGUMENT, "destination %u is also a source", dst_ids[i]);
        if (d.pair >= 0) return fail(QVP_ERR_INVALID_ARGUMENT, "destination %u repeats", dst_ids[i]);
        d.pair = static_cast<int32_t>(pairs);
        pair_entry[pairs] = &d;
        L.pair[pairs].src = src_ids[i];
        L.pair[pairs].dst = dst_ids[i];
        ++pairs;
    }
    num_pairs = pairs;
    uint32_t rows_of[kFusedMaxPairs + 1] = {};
    int32_t pair_of_row[kFusedMaxRows];
    for (uint32_t i = 0; i < count; ++i) {
        FrameTable::Entry& f = table.find(frames[i]);
        if (f.is_src) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "token %u is written into frame %u, which a copy reads", i, frames[i]);
        }
        const uint64_t bit = 1ull << slots[i];
        if (f.rows & bit) return fail(QVP_ERR_INVALID_ARGUMENT, "frame %u slot %u written twice", frames[i], slots[i]);
        f.rows |= bit;
        pair_of_row[i] = f.pair;
        ++rows_of[f.pair >= 0 ? static_cast<uint32_t>(f.pair) : num_pairs];
    }
    // Pair p's rows start at first[p], in slot order: the row in slot t goes
    // to first[p] + (set bits of the pair's slot mask below t). Rows in
    // uncopied frames follow, in call order.
    uint32_t first[kFusedMaxPairs + 1];
    uint32_t at = 0;
    for (uint32_t p = 0; p <= num_pairs; ++p) {
        first[p] = at;
        at += rows_of[p];
    }
    const uint32_t tail_first = first[num_pairs];
    uint32_t tail = tail_first;
    for (uint32_t i = 0; i < count; ++i) {
        uint32_t r;
        if (pair_of_row[i] >= 0) {
            const uint32_t p = static_cast<uint32_t>(pair_of_row[i]);
            r = first[p] + static_cast<uint32_t>(__builtin_popcountll(pair_entry[p]->rows & ((1ull << slots[i]) - 1)));
        } else {
            r = tail++;
        }
        L.row_frame[r] = frames[i];
        L.row_info[r] = i | (slots[i] << 16);
    }
    bool multi = false;
    for (uint32_t p = 0; p < num_pairs; ++p) {
        const uint64_t mask = pair_entry[p]->rows;
        const uint32_t rows = rows_of[p];
        const uint32_t token = rows > 0 ? L.row_info[first[p]] & 0xffffu : 0u;
        L.pair[p].mask_lo = static_cast<uint32_t>(mask);
        L.pair[p].mask_hi = static_cast<uint32_t>(mask >> 32);
        L.pair[p].info = first[p] | (rows << 8) | (token << 16);
        multi = multi || rows > 1;
    }
    FusedGeometry g{};
    g.base = static_cast<uint8_t*>(a->kv_base);
    g.k = static_cast<const uint8_t*>(a->k);
    g.v = static_cast<const uint8_t*>(a->v);
    g.block_stride = a->block_stride;
    g.copy_bytes = static_cast<uint32_t>(copy_bytes);
    // Offsets inside the frame fit 32 bits (block_stride < 2 GiB, checked).
    g.layer_stride = static_cast<uint32_t>(a->layer_stride * bpe);
    g.stream_stride = static_cast<uint32_t>(a->stream_stride * bpe);
    g.token_stride = static_cast<uint32_t>(token_stride);
    g.head_stride = static_cast<uint32_t>(a->head_stride * bpe);
    g.div_layer = make_fastdiv(g.layer_stride);
    g.div_token = make_fastdiv(g.token_stride);
    g.div_head = make_fastdiv(g.head_stride);
    auto pow2 = [](uint32_t d) { return (d & (d - 1)) == 0; };
    const bool shifts = pow2(g.layer_stride) && pow2(g.token_stride) && pow2(g.head_stride);
    g.sh_layer = g.div_layer.l;
    g.sh_token = g.div_token.l;
    g.sh_head = g.div_head.l;
    g.first_layer = a->first_layer;
    g.layer_count = a->layer_count;
    g.num_kv_heads = a->num_kv_heads;
    g.tpb = a->tokens_per_block;
    g.row_bytes = static_cast<uint32_t>(a->head_dim * bpe);
    g.row_words = g.row_bytes / 16;
    g.div_words = make_fastdiv(g.row_words);
    g.div_heads = make_fastdiv(g.num_kv_heads);
    // Rows reach at most the end of the last written layer's V rows.
    const uint64_t row_end = static_cast<uint64_t>(a->first_layer + a->layer_count - 1) * g.layer_stride +
                             g.stream_stride + static_cast<uint64_t>(a->tokens_per_block - 1) * g.token_stride +
                             static_cast<uint64_t>(a->num_kv_heads - 1) * g.head_stride + g.row_bytes;
    const bool pair_rows = tail_first > 0;
    g.span = static_cast<uint32_t>(pair_rows ? std::max<uint64_t>(copy_bytes, row_end) : copy_bytes);
    g.num_pairs = num_pairs;
    g.chunks_per_frame = (g.span + kFusedChunk - 1) / kFusedChunk;
    const uint64_t pair_items = static_cast<uint64_t>(num_pairs) * g.chunks_per_frame;
    const uint64_t total = pair_items + (count - tail_first);
    if (total == 0) return QVP_OK;
    if (total > 0x7fffffffu) return fail(QVP_ERR_INVALID_ARGUMENT, "launch too large");
    g.pair_items = static_cast<uint32_t>(pair_items);
    g.multi_row_pairs = multi ? 1u : 0u;
    g.tail_first = tail_first;
    g.total_items = static_cast<uint32_t>(total);
    uint32_t cus = 0;
    QVP_TRY(device_cus(&cus));
    const uint64_t grid = std::min<uint64_t>(total, static_cast<uint64_t>(cus) * kFusedWgsPerCu);
    if (shifts) {
        hipLaunchKernelGGL(copy_append<true>, dim3(static_cast<uint32_t>(grid)), dim3(kFusedThreads), 0,
                           qvp::as_stream(stream), g, L);
    } else {
        hipLaunchKernelGGL(copy_append<false>, dim3(static_cast<uint32_t>(grid)), dim3(kFusedThreads), 0,
                           qvp::as_stream(stream), g, L);
    }
    QVP_HIP(hipGetLastError());
    return QVP_OK;
}

// Batched block movement: copy-on-write materialisation and swap gather/scatter.
//
// copy_blocks replaces a loop of MemoryAllocator::copy_block calls, each a
// std::memcpy of the whole padded frame (src/MemoryAllocator.cpp:76-85, caller
// src/KVCacheManager.cpp:141-150), with one launch. Swap gather/scatter replace
// HostSwapBackend::store / load (src/SwapBackend.cpp:10-39): whole frames move
// between HBM and a pinned host arena, the GPU itself driving the host link.
//
// All three share one copy loop: a list of (source, destination) segments of
// equal length travels in the kernel arguments (no staging buffer, no extra
// copy), as 32-bit indices into a base address per side (frame ids times the
// frame stride; arena offsets in 16-byte units), 480 segments per launch; a
// list of full pointers (128 per launch) covers arenas past 64 GiB. The
// segments are cut into 8 KiB chunks numbered across the whole list, and a
// grid of at most two workgroups per CU walks the chunks with a stride of the
// grid: short-lived workgroups (one chunk each) left the copy bound by how
// fast workgroups can be dispatched, about 5.5 TB/s of reads plus writes on
// 128 whole 7B frames against 6.4 TB/s this way. Swaps of one-layer frames
// (32 KiB) cross the host link in launches of up to 15 MiB instead of 4 MiB,
// which halves the per-launch start-up and drain share of the time.
#include "common.h"

#include <algorithm>
#include <mutex>
#include <vector>

namespace {

using qvp::fail;

constexpr int kSegmentsPerLaunch = 128;
constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 2;
constexpr uint64_t kChunkBytes = static_cast<uint64_t>(kCopyThreads) * 16 * kCopyUnroll;
constexpr uint32_t kWgsPerCu = 2;

constexpr int kIndexedPerLaunch = 480;  // 3,840 bytes of indices in the kernel arguments

struct SegmentList {
    const uint8_t* src[kSegmentsPerLaunch];
    uint8_t* dst[kSegmentsPerLaunch];
};

// Segment i: source src_base + src[i] * src_unit, destination dst_base +
// dst[i] * dst_unit.
struct IndexedList {
    uint32_t src[kIndexedPerLaunch];
    uint32_t dst[kIndexedPerLaunch];
};

// Chunk [chunk0, min(chunk0 + kChunkBytes, bytes)) of one segment.
__device__ inline void copy_chunk(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint64_t chunk0,
                                  uint64_t bytes) {
    static_assert(kCopyUnroll == 2, "the full-chunk path moves two 16-byte words per thread");
    const uint64_t chunk_end = min(chunk0 + kChunkBytes, bytes);
    const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0;
    if (vec && chunk_end - chunk0 == kChunkBytes) {
        // Both loads issue before either store (two words in flight per
        // thread); plain registers, so nothing is staged through LDS.
        const uint4* s4 = reinterpret_cast<const uint4*>(src + chunk0);
        uint4* d4 = reinterpret_cast<uint4*>(dst + chunk0);
        const uint4 r0 = s4[threadIdx.x];
        const uint4 r1 = s4[threadIdx.x + kCopyThreads];
        d4[threadIdx.x] = r0;
        d4[threadIdx.x + kCopyThreads] = r1;
    } else if (vec) {
        const uint64_t vec_end = chunk0 + (chunk_end - chunk0) / 16 * 16;
        for (uint64_t off = chunk0 + 16u * threadIdx.x; off < vec_end; off += 16u * kCopyThreads) {
            *reinterpret_cast<uint4*>(dst + off) = *reinterpret_cast<const uint4*>(src + off);
        }
        for (uint64_t off = vec_end + threadIdx.x; off < chunk_end; off += kCopyThreads) dst[off] = src[off];
    } else {
        for (uint64_t off = chunk0 + threadIdx.x; off < chunk_end; off += kCopyThreads) dst[off] = src[off];
    }
}

__global__ __launch_bounds__(kCopyThreads) void copy_segments(SegmentList list, uint64_t bytes,
                                                              uint32_t chunks_per_segment, uint32_t total_chunks) {
    for (uint32_t c = blockIdx.x; c < total_chunks; c += gridDim.x) {
        const uint32_t seg = c / chunks_per_segment;
        const uint8_t* src = list.src[seg];
        uint8_t* dst = list.dst[seg];
        if (src == dst) continue;
        copy_chunk(src, dst, static_cast<uint64_t>(c - seg * chunks_per_segment) * kChunkBytes, bytes);
    }
}

__global__ __launch_bounds__(kCopyThreads) void copy_indexed(const uint8_t* src_base, uint64_t src_unit,
                                                             uint8_t* dst_base, uint64_t dst_unit, IndexedList list,
                                                             uint64_t bytes, uint32_t chunks_per_segment,
                                                             uint32_t total_chunks) {
    for (uint32_t c = blockIdx.x; c < total_chunks; c += gridDim.x) {
        const uint32_t seg = c / chunks_per_segment;
        const uint8_t* src = src_base + static_cast<uint64_t>(list.src[seg]) * src_unit;
        uint8_t* dst = dst_base + static_cast<uint64_t>(list.dst[seg]) * dst_unit;
        if (src == dst) continue;
        copy_chunk(src, dst, static_cast<uint64_t>(c - seg * chunks_per_segment) * kChunkBytes, bytes);
    }
}

// Compute units of the current device, cached per device ordinal.
std::mutex g_cu_mutex;
std::vector<uint32_t> g_cus;

int device_cus(uint32_t* cus) {
    int dev = 0;
    QVP_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_cu_mutex);
    if (g_cus.size() <= static_cast<size_t>(dev)) g_cus.resize(dev + 1, 0);
    if (g_cus[dev] == 0) {
        int n = 0;
        QVP_HIP(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        g_cus[dev] = static_cast<uint32_t>(std::max(n, 1));
    }
    *cus = g_cus[dev];
    return QVP_OK;
}

// Enqueues segments [0, n) in launches of kSegmentsPerLaunch.
int launch_segments(const std::vector<const uint8_t*>& src, const std::vector<uint8_t*>& dst,
                    uint64_t bytes, hipStream_t stream) {
    const size_t n = src.size();
    if (n == 0 || bytes == 0) return QVP_OK;
    uint32_t cus = 0;
    QVP_TRY(device_cus(&cus));
    const uint64_t chunks = (bytes + kChunkBytes - 1) / kChunkBytes;
    if (chunks * kSegmentsPerLaunch > 0xffffffffull) return fail(QVP_ERR_INVALID_ARGUMENT, "segment too large");
    for (size_t first = 0; first < n; first += kSegmentsPerLaunch) {
        const size_t count = std::min<size_t>(kSegmentsPerLaunch, n - first);
        SegmentList list{};
        for (size_t i = 0; i < count; ++i) {
            list.src[i] = src[first + i];
            list.dst[i] = dst[first + i];
        }
        const uint64_t total = chunks * count;
        const uint64_t grid = std::min<uint64_t>(total, static_cast<uint64_t>(cus) * kWgsPerCu);
        hipLaunchKernelGGL(copy_segments, dim3(static_cast<unsigned>(grid)), dim3(kCopyThreads), 0, stream, list,
                           bytes, static_cast<uint32_t>(chunks), static_cast<uint32_t>(total));
        QVP_HIP(hipGetLastError());
    }
    return QVP_OK;
}

// Enqueues segments [0, n) given as indices, in launches of kIndexedPerLaunch.
int launch_indexed(const uint8_t* src_base, uint64_t src_unit, const std::vector<uint32_t>& src, uint8_t* dst_base,
                   uint64_t dst_unit, const std::vector<uint32_t>& dst, uint64_t bytes, hipStream_t stream) {
    const size_t n = src.size();
    if (n == 0 || bytes == 0) return QVP_OK;
    uint32_t cus = 0;
    QVP_TRY(device_cus(&cus));
    const uint64_t chunks = (bytes + kChunkBytes - 1) / kChunkBytes;
    if (chunks * kIndexedPerLaunch > 0xffffffffull) return fail(QVP_ERR_INVALID_ARGUMENT, "segment too large");
    for (size_t first = 0; first < n; first += kIndexedPerLaunch) {
        const size_t count = std::min<size_t>(kIndexedPerLaunch, n - first);
        IndexedList list{};
        std::copy(src.begin() + first, src.begin() + first + count, list.src);
        std::copy(dst.begin() + first, dst.begin() + first + count, list.dst);
        const uint64_t total = chunks * count;
        const uint64_t grid = std::min<uint64_t>(total, static_cast<uint64_t>(cus) * kWgsPerCu);
        hipLaunchKernelGGL(copy_indexed, dim3(static_cast<unsigned>(grid)), dim3(kCopyThreads), 0, stream, src_base,
                           src_unit, dst_base, dst_unit, list, bytes, static_cast<uint32_t>(chunks),
                           static_cast<uint32_t>(total));
        QVP_HIP(hipGetLastError());
    }
    return QVP_OK;
}

// Arena offsets in 16-byte units, when every one fits 32 bits (arenas up to
// 64 GiB); false otherwise.
bool arena_units(const uint64_t* offsets, uint32_t count, std::vector<uint32_t>& units) {
    units.resize(count);
    for (uint32_t i = 0; i < count; ++i) {
        if (offsets[i] / 16 > 0xffffffffull) return false;
        units[i] = static_cast<uint32_t>(offsets[i] / 16);
    }
    return true;
}

int check_frames(const uint32_t* ids, uint32_t count, uint32_t num_blocks, const char* what) {
    if (count > 0 && ids == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "%s ids are NULL", what);
    for (uint32_t i = 0; i < count; ++i) {
        if (ids[i] >= num_blocks) {
            return fail(QVP_ERR_UNMAPPED, "%s id %u at %u outside pool of %u blocks", what, ids[i], i,
                        num_blocks);
        }
    }
    return QVP_OK;
}

// Rejects a repeated id (distinct destinations are required so the result does
// not depend on launch order).
int check_distinct(const uint32_t* ids, uint32_t count, const char* what) {
    std::vector<uint32_t> sorted(ids, ids + count);
    std::sort(sorted.begin(), sorted.end());
    for (uint32_t i = 1; i < count; ++i) {
        if (sorted[i] == sorted[i - 1]) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "%s id %u appears twice", what, sorted[i]);
        }
    }
    return QVP_OK;
}

int check_arena_ranges(const uint64_t* offsets, uint32_t count, uint64_t bytes, uint64_t arena_bytes,
                       bool require_disjoint) {
    if (count > 0 && offsets == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "offsets are NULL");
    for (uint32_t i = 0; i < count; ++i) {
        if (offsets[i] % 16 != 0) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "arena offset %llu is not 16-byte aligned",
                        static_cast<unsigned long long>(offsets[i]));
        }
        if (offsets[i] > arena_bytes || bytes > arena_bytes - offsets[i]) {
            return fail(QVP_ERR_CAPACITY, "arena range [%llu, +%llu) outside %llu bytes",
                        static_cast<unsigned long long>(offsets[i]), static_cast<unsigned long long>(bytes),
                        static_cast<unsigned long long>(arena_bytes));
        }
    }
    if (require_disjoint && count > 1) {
        std::vector<uint64_t> sorted(offsets, offsets + count);
        std::sort(sorted.begin(), sorted.end());
        for (uint32_t i = 1; i < count; ++i) {
            if (sorted[i] - sorted[i - 1] < bytes) {
                return fail(QVP_ERR_INVALID_ARGUMENT, "arena ranges at %llu and %llu overlap",
                            static_cast<unsigned long long>(sorted[i - 1]),
                            static_cast<unsigned long long>(sorted[i]));
            }
        }
    }
    return QVP_OK;
}

}  // namespace

extern "C" {

int qvp_copy_blocks(void* kv_base, uint64_t block_stride, uint32_t num_blocks, const uint32_t* src_ids,
                    const uint32_t* dst_ids, uint32_t num_pairs, uint64_t copy_bytes, void* stream) {
    if (num_pairs == 0) return QVP_OK;
    if (kv_base == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "kv_base is NULL");
    if (copy_bytes > block_stride) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "copy of %llu bytes exceeds frame stride %llu",
                    static_cast<unsigned long long>(copy_bytes), static_cast<unsigned long long>(block_stride));
    }
    QVP_TRY(check_frames(src_ids, num_pairs, num_blocks, "source"));
    QVP_TRY(check_frames(dst_ids, num_pairs, num_blocks, "destination"));
    QVP_TRY(check_distinct(dst_ids, num_pairs, "destination"));
    // A destination that is another pair's source would make the result depend
    // on the order in which workgroups run.
    {
        std::vector<uint32_t> srcs(src_ids, src_ids + num_pairs);
        std::sort(srcs.begin(), srcs.end());
        for (uint32_t i = 0; i < num_pairs; ++i) {
            if (dst_ids[i] == src_ids[i]) continue;
            if (std::binary_search(srcs.begin(), srcs.end(), dst_ids[i])) {
                return fail(QVP_ERR_INVALID_ARGUMENT, "destination %u is also a source", dst_ids[i]);
            }
        }
    }
    uint8_t* base = static_cast<uint8_t*>(kv_base);
    return launch_indexed(base, block_stride, std::vector<uint32_t>(src_ids, src_ids + num_pairs), base, block_stride,
                          std::vector<uint32_t>(dst_ids, dst_ids + num_pairs), copy_bytes, qvp::as_stream(stream));
}

int qvp_swap_gather(const void* kv_base, uint64_t block_stride, uint32_t num_blocks,
                    const uint32_t* frame_ids, const uint64_t* arena_offsets, uint32_t count, void* arena,
                    uint64_t arena_bytes, uint64_t copy_bytes, void* stream) {
    if (count == 0) return QVP_OK;
    if (kv_base == nullptr || arena == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "NULL base or arena");
    if (copy_bytes > block_stride) return fail(QVP_ERR_INVALID_ARGUMENT, "copy exceeds frame stride");
    QVP_TRY(check_frames(frame_ids, count, num_blocks, "frame"));
    QVP_TRY(check_arena_ranges(arena_offsets, count, copy_bytes, arena_bytes, true));
    void* arena_dev = nullptr;
    QVP_HIP(hipHostGetDevicePointer(&arena_dev, arena, 0));
    const uint8_t* base = static_cast<const uint8_t*>(kv_base);
    std::vector<uint32_t> units;
    if (arena_units(arena_offsets, count, units)) {
        return launch_indexed(base, block_stride, std::vector<uint32_t>(frame_ids, frame_ids + count),
                              static_cast<uint8_t*>(arena_dev), 16, units, copy_bytes, qvp::as_stream(stream));
    }
    std::vector<const uint8_t*> src(count);
    std::vector<uint8_t*> dst(count);
    for (uint32_t i = 0; i < count; ++i) {
        src[i] = base + static_cast<uint64_t>(frame_ids[i]) * block_stride;
        dst[i] = static_cast<uint8_t*>(arena_dev) + arena_offsets[i];
    }
    return launch_segments(src, dst, copy_bytes, qvp::as_stream(stream));
}

int qvp_swap_scatter(void* kv_base, uint64_t block_stride, uint32_t num_blocks, const uint32_t* frame_ids,
                     const uint64_t* arena_offsets, uint32_t count, const void* arena, uint64_t arena_bytes,
                     uint64_t copy_bytes, void* stream) {
    if (count == 0) return QVP_OK;
    if (kv_base == nullptr || arena == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "NULL base or arena");
    if (copy_bytes > block_stride) return fail(QVP_ERR_INVALID_ARGUMENT, "copy exceeds frame stride");
    QVP_TRY(check_frames(frame_ids, count, num_blocks, "frame"));
    QVP_TRY(check_distinct(frame_ids, count, "frame"));
    QVP_TRY(check_arena_ranges(arena_offsets, count, copy_bytes, arena_bytes, false));
    void* arena_dev = nullptr;
    QVP_HIP(hipHostGetDevicePointer(&arena_dev, const_cast<void*>(arena), 0));
    uint8_t* base = static_cast<uint8_t*>(kv_base);
    std::vector<uint32_t> units;
    if (arena_units(arena_offsets, count, units)) {
        return launch_indexed(static_cast<const uint8_t*>(arena_dev), 16, units, base, block_stride,
                              std::vector<uint32_t>(frame_ids, frame_ids + count), copy_bytes, qvp::as_stream(stream));
    }
    std::vector<const uint8_t*> src(count);
    std::vector<uint8_t*> dst(count);
    for (uint32_t i = 0; i < count; ++i) {
        src[i] = static_cast<const uint8_t*>(arena_dev) + arena_offsets[i];
        dst[i] = base + static_cast<uint64_t>(frame_ids[i]) * block_stride;
    }
    return launch_segments(src, dst, copy_bytes, qvp::as_stream(stream));
}

}  // extern "C"

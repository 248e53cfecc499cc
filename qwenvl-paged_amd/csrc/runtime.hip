// Error state, runtime plumbing and the HBM block pool.
//
// The pool replaces the reference's one-std::aligned_alloc-per-block storage
// (include/qwenvl_paged/Block.h:99-166, src/Block.cpp:30-44) with a single
// device allocation: frame i starts at base + i * stride, and stride is the
// block's byte size rounded up to the alignment exactly like
// PhysicalBlock::size_bytes() (src/Block.cpp:21-26,32-38).
#include "common.h"

#include <cstring>
#include <new>
#include <string>

namespace qvp {

namespace {
thread_local std::string g_last_error;
}  // namespace

int fail(int status, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error.assign(buf);
    return status;
}

void clear_error() { g_last_error.clear(); }

int hip_fail(hipError_t err, const char* what) {
    const int status = (err == hipErrorOutOfMemory) ? QVP_ERR_OUT_OF_MEMORY : QVP_ERR_DEVICE;
    return fail(status, "%s failed: %s", what, hipGetErrorString(err));
}

}  // namespace qvp

using qvp::fail;

extern "C" {

const char* qvp_last_error(void) { return qvp::g_last_error.c_str(); }

const char* qvp_status_name(int status) {
    switch (status) {
        case QVP_OK: return "QVP_OK";
        case QVP_ERR_INVALID_ARGUMENT: return "QVP_ERR_INVALID_ARGUMENT";
        case QVP_ERR_UNMAPPED: return "QVP_ERR_UNMAPPED";
        case QVP_ERR_OUT_OF_MEMORY: return "QVP_ERR_OUT_OF_MEMORY";
        case QVP_ERR_CAPACITY: return "QVP_ERR_CAPACITY";
        case QVP_ERR_DEVICE: return "QVP_ERR_DEVICE";
        default: return "QVP_ERR_UNKNOWN";
    }
}

int qvp_version(void) { return 100; }

int qvp_device_count(int* count) {
    if (count == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "count is NULL");
    QVP_HIP(hipGetDeviceCount(count));
    return QVP_OK;
}

int qvp_set_device(int device) {
    QVP_HIP(hipSetDevice(device));
    return QVP_OK;
}

int qvp_device_synchronize(void) {
    QVP_HIP(hipDeviceSynchronize());
    return QVP_OK;
}

int qvp_malloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "ptr is NULL");
    *ptr = nullptr;
    if (bytes == 0) return QVP_OK;
    QVP_HIP(hipMalloc(ptr, bytes));
    return QVP_OK;
}

int qvp_free(void* ptr) {
    if (ptr != nullptr) QVP_HIP(hipFree(ptr));
    return QVP_OK;
}

int qvp_host_alloc(void** ptr, size_t bytes) {
    if (ptr == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "ptr is NULL");
    *ptr = nullptr;
    if (bytes == 0) return QVP_OK;
    QVP_HIP(hipHostMalloc(ptr, bytes, hipHostMallocDefault));
    return QVP_OK;
}

int qvp_host_free(void* ptr) {
    if (ptr != nullptr) QVP_HIP(hipHostFree(ptr));
    return QVP_OK;
}

int qvp_host_device_pointer(void** device_ptr, void* host_ptr) {
    if (device_ptr == nullptr || host_ptr == nullptr) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "NULL pointer");
    }
    QVP_HIP(hipHostGetDevicePointer(device_ptr, host_ptr, 0));
    return QVP_OK;
}

int qvp_memcpy_htod(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return QVP_OK;
    QVP_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, qvp::as_stream(stream)));
    return QVP_OK;
}

int qvp_memcpy_dtoh(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return QVP_OK;
    QVP_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, qvp::as_stream(stream)));
    return QVP_OK;
}

int qvp_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream) {
    if (bytes == 0) return QVP_OK;
    QVP_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, qvp::as_stream(stream)));
    return QVP_OK;
}

int qvp_stream_create(void** stream) {
    if (stream == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "stream is NULL");
    hipStream_t s = nullptr;
    // Default priority on purpose: streams of mixed priorities are not used.
    QVP_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return QVP_OK;
}

int qvp_stream_destroy(void* stream) {
    if (stream != nullptr) QVP_HIP(hipStreamDestroy(qvp::as_stream(stream)));
    return QVP_OK;
}

int qvp_stream_synchronize(void* stream) {
    QVP_HIP(hipStreamSynchronize(qvp::as_stream(stream)));
    return QVP_OK;
}

int qvp_event_create(void** event) {
    if (event == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "event is NULL");
    hipEvent_t e = nullptr;
    QVP_HIP(hipEventCreate(&e));
    *event = e;
    return QVP_OK;
}

int qvp_event_destroy(void* event) {
    if (event != nullptr) QVP_HIP(hipEventDestroy(reinterpret_cast<hipEvent_t>(event)));
    return QVP_OK;
}

int qvp_event_record(void* event, void* stream) {
    QVP_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(event), qvp::as_stream(stream)));
    return QVP_OK;
}

int qvp_event_synchronize(void* event) {
    QVP_HIP(hipEventSynchronize(reinterpret_cast<hipEvent_t>(event)));
    return QVP_OK;
}

int qvp_event_query(void* event, int* complete) {
    if (complete == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "complete is NULL");
    const hipError_t err = hipEventQuery(reinterpret_cast<hipEvent_t>(event));
    if (err == hipErrorNotReady) {
        *complete = 0;
        return QVP_OK;
    }
    if (err != hipSuccess) return qvp::hip_fail(err, "hipEventQuery");
    *complete = 1;
    return QVP_OK;
}

int qvp_stream_wait_event(void* stream, void* event) {
    QVP_HIP(hipStreamWaitEvent(qvp::as_stream(stream), reinterpret_cast<hipEvent_t>(event), 0));
    return QVP_OK;
}

int qvp_event_elapsed_ms(float* ms, void* start, void* stop) {
    if (ms == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "ms is NULL");
    QVP_HIP(hipEventElapsedTime(ms, reinterpret_cast<hipEvent_t>(start),
                                reinterpret_cast<hipEvent_t>(stop)));
    return QVP_OK;
}

int qvp_graph_begin_capture(void* stream) {
    if (stream == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "capture needs a created stream, not the default one");
    QVP_HIP(hipStreamBeginCapture(qvp::as_stream(stream), hipStreamCaptureModeThreadLocal));
    return QVP_OK;
}

int qvp_graph_end_capture(void* stream, void** graph_exec) {
    if (stream == nullptr || graph_exec == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "stream or graph_exec is NULL");
    *graph_exec = nullptr;
    hipGraph_t graph = nullptr;
    QVP_HIP(hipStreamEndCapture(qvp::as_stream(stream), &graph));
    hipGraphExec_t exec = nullptr;
    const hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (err != hipSuccess) return qvp::hip_fail(err, "hipGraphInstantiate");
    *graph_exec = exec;
    return QVP_OK;
}

int qvp_graph_launch(void* graph_exec, void* stream) {
    if (graph_exec == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "graph_exec is NULL");
    QVP_HIP(hipGraphLaunch(reinterpret_cast<hipGraphExec_t>(graph_exec), qvp::as_stream(stream)));
    return QVP_OK;
}

int qvp_graph_destroy(void* graph_exec) {
    if (graph_exec == nullptr) return QVP_OK;
    QVP_HIP(hipGraphExecDestroy(reinterpret_cast<hipGraphExec_t>(graph_exec)));
    return QVP_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Fill kernel (used instead of runtime memsets so callers may capture it).
// ---------------------------------------------------------------------------

namespace {

__global__ void fill_bytes_kernel(uint8_t* __restrict__ dst, uint32_t pattern, size_t bytes) {
    const size_t tid = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const size_t nthreads = static_cast<size_t>(gridDim.x) * blockDim.x;
    const uintptr_t addr = reinterpret_cast<uintptr_t>(dst);
    if ((addr & 15u) == 0) {
        const size_t vec = bytes / 16;
        uint4* d4 = reinterpret_cast<uint4*>(dst);
        const uint4 p = make_uint4(pattern, pattern, pattern, pattern);
        for (size_t i = tid; i < vec; i += nthreads) d4[i] = p;
        for (size_t i = vec * 16 + tid; i < bytes; i += nthreads) dst[i] = static_cast<uint8_t>(pattern);
    } else {
        for (size_t i = tid; i < bytes; i += nthreads) dst[i] = static_cast<uint8_t>(pattern);
    }
}

// Staged-upload kernel: one 16-byte host read per thread, spread over as many
// workgroups as the upload needs. Reads of pinned host memory queue per
// wave: with several reads in flight per thread a 152 KB upload took 8.7 us
// per launch (256 threads x 4 reads per workgroup), with one read per thread
// 5.5 us (38 workgroups), back to back on MI355X.
constexpr int kPullThreads = 256;
constexpr size_t kPullMaxBlocks = 2048;

__global__ __launch_bounds__(kPullThreads) void pull_pinned_kernel(const uint4* __restrict__ src,
                                                                   uint4* __restrict__ dst, size_t n16,
                                                                   const uint32_t* __restrict__ src_tail,
                                                                   uint32_t* __restrict__ dst_tail, uint32_t tail) {
    const size_t step = static_cast<size_t>(gridDim.x) * kPullThreads;
    for (size_t i = static_cast<size_t>(blockIdx.x) * kPullThreads + threadIdx.x; i < n16; i += step) dst[i] = src[i];
    if (blockIdx.x == 0 && threadIdx.x < tail) dst_tail[threadIdx.x] = src_tail[threadIdx.x];
}

}  // namespace

namespace qvp {

int pull_from_pinned(void* dst, const void* pinned_host, size_t bytes, hipStream_t stream) {
    if (bytes == 0) return QVP_OK;
    if (bytes % 4 != 0 || (reinterpret_cast<uintptr_t>(dst) & 15u) != 0 ||
        (reinterpret_cast<uintptr_t>(pinned_host) & 15u) != 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "staged upload of %zu bytes is not word-sized or 16-byte aligned",
                    bytes);
    }
    void* src = nullptr;
    QVP_HIP(hipHostGetDevicePointer(&src, const_cast<void*>(pinned_host), 0));
    const size_t n16 = bytes / 16;
    const uint32_t tail = static_cast<uint32_t>((bytes % 16) / 4);
    size_t blocks = (n16 + kPullThreads - 1) / kPullThreads;
    blocks = blocks == 0 ? 1 : (blocks > kPullMaxBlocks ? kPullMaxBlocks : blocks);
    hipLaunchKernelGGL(pull_pinned_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kPullThreads), 0, stream,
                       static_cast<const uint4*>(src), static_cast<uint4*>(dst), n16,
                       reinterpret_cast<const uint32_t*>(static_cast<const uint8_t*>(src) + n16 * 16),
                       reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(dst) + n16 * 16), tail);
    QVP_HIP(hipGetLastError());
    return QVP_OK;
}

}  // namespace qvp

extern "C" int qvp_fill_bytes(void* dst, uint8_t value, size_t bytes, void* stream) {
    if (bytes == 0) return QVP_OK;
    if (dst == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "dst is NULL");
    const uint32_t pattern = 0x01010101u * value;
    const size_t work = (bytes + 15) / 16;
    size_t blocks = (work + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(fill_bytes_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                       qvp::as_stream(stream), static_cast<uint8_t*>(dst), pattern, bytes);
    QVP_HIP(hipGetLastError());
    return QVP_OK;
}

// ---------------------------------------------------------------------------
// Block pool
// ---------------------------------------------------------------------------

struct qvp_pool {
    uint8_t* base{nullptr};
    uint32_t num_blocks{0};
    size_t block_bytes{0};
    size_t stride{0};
};

extern "C" {

int qvp_pool_create(uint32_t num_blocks, size_t block_bytes, size_t alignment, qvp_pool** pool) {
    if (pool == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "pool is NULL");
    *pool = nullptr;
    if (num_blocks == 0) return fail(QVP_ERR_INVALID_ARGUMENT, "num_blocks is 0");
    // Alignment 0 falls back to the 256-byte default, and a zero-byte block
    // still occupies one aligned unit (src/Block.cpp:30-38).
    const size_t align = alignment == 0 ? 256 : alignment;
    if ((align & (align - 1)) != 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "alignment %zu is not a power of two", align);
    }
    size_t stride = qvp::round_up(block_bytes, align);
    if (stride == 0) stride = align;
    const size_t total = stride * static_cast<size_t>(num_blocks);
    if (total / stride != num_blocks) return fail(QVP_ERR_INVALID_ARGUMENT, "pool size overflows");

    qvp_pool* p = new (std::nothrow) qvp_pool();
    if (p == nullptr) return fail(QVP_ERR_OUT_OF_MEMORY, "pool descriptor");
    hipError_t err = hipMalloc(reinterpret_cast<void**>(&p->base), total);
    if (err != hipSuccess) {
        delete p;
        return qvp::hip_fail(err, "hipMalloc(pool)");
    }
    p->num_blocks = num_blocks;
    p->block_bytes = block_bytes;
    p->stride = stride;
    *pool = p;
    return QVP_OK;
}

int qvp_pool_destroy(qvp_pool* pool) {
    if (pool == nullptr) return QVP_OK;
    hipError_t err = hipFree(pool->base);
    delete pool;
    if (err != hipSuccess) return qvp::hip_fail(err, "hipFree(pool)");
    return QVP_OK;
}

void* qvp_pool_base(const qvp_pool* pool) { return pool ? pool->base : nullptr; }
size_t qvp_pool_block_stride(const qvp_pool* pool) { return pool ? pool->stride : 0; }
size_t qvp_pool_block_bytes(const qvp_pool* pool) { return pool ? pool->block_bytes : 0; }
uint32_t qvp_pool_num_blocks(const qvp_pool* pool) { return pool ? pool->num_blocks : 0; }

void* qvp_pool_block_ptr(const qvp_pool* pool, uint32_t block) {
    if (pool == nullptr || block >= pool->num_blocks) return nullptr;
    return pool->base + static_cast<size_t>(block) * pool->stride;
}

static int check_range(const qvp_pool* pool, uint32_t block, size_t offset, size_t bytes) {
    if (pool == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "pool is NULL");
    if (block >= pool->num_blocks) {
        return fail(QVP_ERR_UNMAPPED, "block %u outside pool of %u", block, pool->num_blocks);
    }
    if (offset > pool->stride || bytes > pool->stride - offset) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "range [%zu, +%zu) outside frame of %zu bytes", offset,
                    bytes, pool->stride);
    }
    return QVP_OK;
}

int qvp_pool_write(qvp_pool* pool, uint32_t block, size_t offset, const void* src, size_t bytes,
                   void* stream) {
    QVP_TRY(check_range(pool, block, offset, bytes));
    if (bytes == 0) return QVP_OK;
    if (src == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "src is NULL");
    uint8_t* dst = pool->base + static_cast<size_t>(block) * pool->stride + offset;
    QVP_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, qvp::as_stream(stream)));
    return QVP_OK;
}

int qvp_pool_read(const qvp_pool* pool, uint32_t block, size_t offset, void* dst, size_t bytes,
                  void* stream) {
    QVP_TRY(check_range(pool, block, offset, bytes));
    if (bytes == 0) return QVP_OK;
    if (dst == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "dst is NULL");
    const uint8_t* src = pool->base + static_cast<size_t>(block) * pool->stride + offset;
    QVP_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, qvp::as_stream(stream)));
    return QVP_OK;
}

}  // extern "C"

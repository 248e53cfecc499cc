// HBM read-rate probe for the benchmark (built into libqvp_probe.so, not into
// libqvp.so): streams a buffer once with 16-byte loads and keeps nothing but a
// running XOR, so its duration is what a kernel that only reads those bytes
// takes on this device at this size -- launch ramp and drain included. The
// benchmark runs it over as many bytes as one decode step reads, on buffers it
// rotates (so no pass finds the previous one in the Infinity Cache), and takes
// the fastest of a few launch shapes and both load kinds (plain, and
// non-temporal as the decode kernels read) as the practical ceiling for that
// step.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kThreads = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool kNt>
__device__ inline uint4 load(const uint4* p) {
    if constexpr (kNt) {
        const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
        return make_uint4(v.x, v.y, v.z, v.w);
    }
    return *p;
}

// Each thread takes every gridDim.x * 256-th 16-byte chunk, kUnroll of them
// in flight at a time.
template <int kUnroll, bool kNt>
__global__ __launch_bounds__(kThreads) void read_stream(const uint4* __restrict__ src, uint64_t chunks,
                                                        uint32_t* __restrict__ sink) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (kUnroll - 1) * stride < chunks; i += kUnroll * stride) {
        uint4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) v[u] = load<kNt>(src + i + u * stride);
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < chunks; i += stride) {
        const uint4 v = load<kNt>(src + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    // The store depends on every load, so none of them can be dropped; the
    // sink holds one word per thread.
    sink[static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x] = acc;
}

}  // namespace

namespace {

template <bool kNt>
bool launch(const uint4* p, uint64_t chunks, uint32_t workgroups, uint32_t unroll, uint32_t* sink, hipStream_t st) {
    switch (unroll) {
        case 1:
            hipLaunchKernelGGL((read_stream<1, kNt>), dim3(workgroups), dim3(kThreads), 0, st, p, chunks, sink);
            return true;
        case 2:
            hipLaunchKernelGGL((read_stream<2, kNt>), dim3(workgroups), dim3(kThreads), 0, st, p, chunks, sink);
            return true;
        case 4:
            hipLaunchKernelGGL((read_stream<4, kNt>), dim3(workgroups), dim3(kThreads), 0, st, p, chunks, sink);
            return true;
        case 8:
            hipLaunchKernelGGL((read_stream<8, kNt>), dim3(workgroups), dim3(kThreads), 0, st, p, chunks, sink);
            return true;
        case 16:
            hipLaunchKernelGGL((read_stream<16, kNt>), dim3(workgroups), dim3(kThreads), 0, st, p, chunks, sink);
            return true;
        default:
            return false;
    }
}

}  // namespace

// Enqueues one probe pass over `bytes` (a multiple of 16) at `src`, with
// `workgroups` workgroups of 256 threads, `unroll` (1, 2, 4, 8 or 16) loads in
// flight per thread, plain loads or (nontemporal != 0) non-temporal ones.
// `sink` holds workgroups * 256 uint32. Returns 0, or -1 for arguments it does
// not take.
extern "C" int qvp_probe_read(const void* src, uint64_t bytes, uint32_t workgroups, uint32_t unroll,
                              uint32_t nontemporal, uint32_t* sink, void* stream) {
    if (src == nullptr || sink == nullptr || bytes % 16 != 0 || workgroups == 0 || workgroups > (1u << 20)) {
        return -1;
    }
    const auto* p = static_cast<const uint4*>(src);
    const uint64_t chunks = bytes / 16;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const bool ok = nontemporal != 0 ? launch<true>(p, chunks, workgroups, unroll, sink, st)
                                     : launch<false>(p, chunks, workgroups, unroll, sink, st);
    if (!ok) return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Shared helpers for the qvp HIP library: error state, status plumbing and
// element conversions. gfx950 only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstddef>
#include <cstdint>
#include <cstdio>

#include "qvp.h"

namespace qvp {

// Records `msg` as the calling thread's last error and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Converts a failed HIP call into QVP_ERR_DEVICE (or QVP_ERR_OUT_OF_MEMORY).
int hip_fail(hipError_t err, const char* what);

#define QVP_HIP(call)                                  \
    do {                                               \
        hipError_t qvp_err_ = (call);                  \
        if (qvp_err_ != hipSuccess) {                  \
            return ::qvp::hip_fail(qvp_err_, #call);   \
        }                                              \
    } while (0)

#define QVP_TRY(expr)                  \
    do {                               \
        int qvp_st_ = (expr);          \
        if (qvp_st_ != QVP_OK) {       \
            return qvp_st_;            \
        }                              \
    } while (0)

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Copies `bytes` (a multiple of 4; both pointers 16-byte aligned) from pinned
// host memory allocated by hipHostMalloc with hipHostMallocCoherent (so the
// GPU never holds a stale cached copy of a staging buffer the host refilled)
// into device memory, with a kernel on `stream` that reads the host buffer
// over the bus. A runtime host-to-device copy would go to the DMA engine and
// pay two cross-engine handoffs between the surrounding kernels; the kernel
// stays on the compute queue.
int pull_from_pinned(void* dst, const void* pinned_host, size_t bytes, hipStream_t stream);

inline size_t dtype_size(uint32_t dtype) {
    switch (dtype) {
        case QVP_DTYPE_F32: return 4;
        case QVP_DTYPE_BF16: return 2;
        case QVP_DTYPE_F16: return 2;
        default: return 0;
    }
}

inline uint64_t round_up(uint64_t v, uint64_t a) { return a == 0 ? v : (v + a - 1) / a * a; }

// bfloat16 <-> float. The narrowing conversion rounds to nearest, ties to even,
// and keeps NaNs quiet; the widening one is exact.
__host__ __device__ inline float bf16_bits_to_float(uint16_t h) {
    union { uint32_t u; float f; } v;
    v.u = static_cast<uint32_t>(h) << 16;
    return v.f;
}

__host__ __device__ inline uint16_t float_to_bf16_bits(float f) {
    union { uint32_t u; float f; } v;
    v.f = f;
    if ((v.u & 0x7fffffffu) > 0x7f800000u) {
        return static_cast<uint16_t>((v.u >> 16) | 0x0040u);
    }
    const uint32_t lsb = (v.u >> 16) & 1u;
    return static_cast<uint16_t>((v.u + 0x7fffu + lsb) >> 16);
}

}  // namespace qvp

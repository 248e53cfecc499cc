// Generic paged decode: any element type, head_dim, GQA group and block size.
//
// One workgroup per (split, query head) over the packer's fixed token splits,
// VALU arithmetic. Within a split it runs the reference's two passes
// (include/qwenvl_paged/PagedAttention.h:98-118): scores and their maximum,
// then weights, their sum and the value accumulator; a merge kernel then
// combines the splits of each sequence. It serves fp32/fp16 caches and shapes
// the MFMA kernel does not cover.
#include "decode_common.h"

#include <algorithm>

namespace qvp {
namespace {

constexpr int kGenericThreads = 128;

__device__ inline float block_reduce_max(float v, float* scratch) {
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[wave] = v;
    __syncthreads();
    float r = scratch[0];
    for (int w = 1; w < static_cast<int>(blockDim.x >> 6); ++w) r = fmaxf(r, scratch[w]);
    __syncthreads();
    return r;
}

__device__ inline float block_reduce_sum(float v, float* scratch) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) scratch[wave] = v;
    __syncthreads();
    float r = 0.f;
    for (int w = 0; w < static_cast<int>(blockDim.x >> 6); ++w) r += scratch[w];
    __syncthreads();
    return r;
}

struct SplitArgs {
    const int32_t* split_seq;
    const int32_t* split_start;
    uint32_t split_tokens;
    float* ws_ml;   // [num_splits][Hq][2]
    float* ws_acc;  // [num_splits][Hq][D]
};

template <typename T>
__global__ __launch_bounds__(kGenericThreads) void decode_generic(DecodeGeometry p, SplitArgs sa) {
    extern __shared__ float smem[];
    float* q_s = smem;               // [head_dim]
    float* s_s = smem + p.head_dim;  // [split_tokens]
    __shared__ float red[kGenericThreads / 64];

    const uint32_t split = blockIdx.x / p.num_q_heads;
    const uint32_t h = blockIdx.x - split * p.num_q_heads;
    const uint32_t g = h / p.group;
    const int b = sa.split_seq[split];
    const int start = sa.split_start[split];
    const int ctx = p.seq_lens[b];
    const int len = min(static_cast<int>(sa.split_tokens), ctx - start);
    const int32_t* row = p.tables + static_cast<uint64_t>(b) * p.max_nb;
    const uint32_t D = p.head_dim;

    const T* q = static_cast<const T*>(p.query) + (static_cast<uint64_t>(b) * p.num_q_heads + h) * D;
    for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) q_s[d] = to_float<T>(q[d]);
    __syncthreads();

    const uint64_t head_off = g * p.head_stride;
    float mloc = -INFINITY;
    for (int t = threadIdx.x; t < len; t += blockDim.x) {
        const uint32_t tok = static_cast<uint32_t>(start + t);
        const int32_t blk = row[tok / p.tpb];
        const T* k = reinterpret_cast<const T*>(p.kv_base + static_cast<uint64_t>(blk) * p.block_stride + p.k_off +
                                                (tok % p.tpb) * p.token_stride + head_off);
        float dot = 0.f;
        for (uint32_t d = 0; d < D; ++d) dot += q_s[d] * to_float<T>(k[d]);
        const float sv = dot * p.scale_log2;
        s_s[t] = sv;
        mloc = fmaxf(mloc, sv);
    }
    const float m = block_reduce_max(mloc, red);
    float lloc = 0.f;
    for (int t = threadIdx.x; t < len; t += blockDim.x) {
        const float w = fast_exp2(s_s[t] - m);
        s_s[t] = w;
        lloc += w;
    }
    const float l = block_reduce_sum(lloc, red);  // also orders the s_s writes before the reads below

    float* acc_out = sa.ws_acc + (static_cast<uint64_t>(split) * p.num_q_heads + h) * D;
    for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
        float acc = 0.f;
        for (int t = 0; t < len; ++t) {
            const uint32_t tok = static_cast<uint32_t>(start + t);
            const int32_t blk = row[tok / p.tpb];
            const T* v = reinterpret_cast<const T*>(p.kv_base + static_cast<uint64_t>(blk) * p.block_stride + p.v_off +
                                                    (tok % p.tpb) * p.token_stride + head_off);
            acc += s_s[t] * to_float<T>(v[d]);
        }
        acc_out[d] = acc;
    }
    if (threadIdx.x == 0) {
        sa.ws_ml[(static_cast<uint64_t>(split) * p.num_q_heads + h) * 2 + 0] = m;
        sa.ws_ml[(static_cast<uint64_t>(split) * p.num_q_heads + h) * 2 + 1] = l;
    }
}

// out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M) per (sequence, head).
// Up to kMergeThreads splits: thread s reads split s's (m, l) once, the
// maximum and the weighted sum are workgroup reductions and the splits'
// factors sit in LDS for the accumulation pass (one round trip for the
// (m, l) pairs instead of two dependent loops over them).
constexpr int kMergeThreads = 128;

template <typename OutT>
__global__ __launch_bounds__(kMergeThreads) void merge_splits(const float* __restrict__ ws_ml,
                                                             const float* __restrict__ ws_acc,
                                                             const int32_t* __restrict__ cu_splits,
                                                             OutT* __restrict__ out, uint32_t num_q_heads,
                                                             uint32_t head_dim) {
    __shared__ float f_s[kMergeThreads];
    __shared__ float red[kMergeThreads / 64];
    const uint32_t b = blockIdx.x / num_q_heads;
    const uint32_t h = blockIdx.x - b * num_q_heads;
    const int s0 = cu_splits[b];
    const int s1 = cu_splits[b + 1];
    const int ns = s1 - s0;
    if (ns <= kMergeThreads) {
        const int t = static_cast<int>(threadIdx.x);
        float m = -INFINITY;
        float l = 0.f;
        if (t < ns) {
            const uint64_t idx = static_cast<uint64_t>(s0 + t) * num_q_heads + h;
            m = ws_ml[idx * 2];
            l = ws_ml[idx * 2 + 1];
        }
        const float mmax = block_reduce_max(m, red);
        const float f = t < ns ? fast_exp2(m - mmax) : 0.f;
        f_s[t] = f;
        const float lsum = block_reduce_sum(l * f, red);  // also orders the f_s writes before the reads below
        OutT* o = out + (static_cast<uint64_t>(b) * num_q_heads + h) * head_dim;
        for (uint32_t d = threadIdx.x; d < head_dim; d += blockDim.x) {
            float acc = 0.f;
            for (int x = 0; x < ns; ++x) {
                acc += ws_acc[(static_cast<uint64_t>(s0 + x) * num_q_heads + h) * head_dim + d] * f_s[x];
            }
            o[d] = from_float<OutT>(acc / lsum);
        }
        return;
    }
    float mmax = -INFINITY;
    for (int s = s0; s < s1; ++s) mmax = fmaxf(mmax, ws_ml[(static_cast<uint64_t>(s) * num_q_heads + h) * 2]);
    float lsum = 0.f;
    for (int s = s0; s < s1; ++s) {
        const uint64_t idx = static_cast<uint64_t>(s) * num_q_heads + h;
        lsum += ws_ml[idx * 2 + 1] * fast_exp2(ws_ml[idx * 2] - mmax);
    }
    OutT* o = out + (static_cast<uint64_t>(b) * num_q_heads + h) * head_dim;
    for (uint32_t d = threadIdx.x; d < head_dim; d += blockDim.x) {
        float acc = 0.f;
        for (int s = s0; s < s1; ++s) {
            const uint64_t idx = static_cast<uint64_t>(s) * num_q_heads + h;
            acc += ws_acc[idx * head_dim + d] * fast_exp2(ws_ml[idx * 2] - mmax);
        }
        o[d] = from_float<OutT>(acc / lsum);
    }
}

constexpr int kGroupedThreads = 256;
constexpr int kGroupedWaves = kGroupedThreads / 64;

// Reduces each of a thread's kG per-head values over the workgroup (every
// thread gets the results): shuffles within each wave, one LDS exchange.
template <int kG, bool kMax>
__device__ inline void reduce_heads(float (&v)[kG], float (*red)[kG]) {
#pragma unroll
    for (int h = 0; h < kG; ++h) {
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(v[h], off);
            v[h] = kMax ? fmaxf(v[h], o) : v[h] + o;
        }
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
#pragma unroll
        for (int h = 0; h < kG; ++h) red[wave][h] = v[h];
    }
    __syncthreads();
#pragma unroll
    for (int h = 0; h < kG; ++h) {
        float r = red[0][h];
#pragma unroll
        for (int w = 1; w < kGroupedWaves; ++w) r = kMax ? fmaxf(r, red[w][h]) : r + red[w][h];
        v[h] = r;
    }
    __syncthreads();
}

// Four consecutive elements of a K or V row as floats (the row offset is a
// multiple of four elements and the address of four elements' bytes).
template <typename T>
__device__ inline float4 load4(const T* ptr);
template <>
__device__ inline float4 load4<float>(const float* ptr) {
    return *reinterpret_cast<const float4*>(ptr);
}
template <>
__device__ inline float4 load4<uint16_t>(const uint16_t* ptr) {
    const uint2 r = *reinterpret_cast<const uint2*>(ptr);
    return float4{bf16_bits_to_float(static_cast<uint16_t>(r.x & 0xffffu)), bf16_bits_to_float(static_cast<uint16_t>(r.x >> 16)),
                  bf16_bits_to_float(static_cast<uint16_t>(r.y & 0xffffu)), bf16_bits_to_float(static_cast<uint16_t>(r.y >> 16))};
}
template <>
__device__ inline float4 load4<_Float16>(const _Float16* ptr) {
    typedef _Float16 h4 __attribute__((ext_vector_type(4)));
    const h4 r = *reinterpret_cast<const h4*>(ptr);
    return float4{static_cast<float>(r[0]), static_cast<float>(r[1]), static_cast<float>(r[2]), static_cast<float>(r[3])};
}

// GQA-folded split decode for any element type and head_dim (a multiple of
// four, rows aligned to four elements): one workgroup per (split, kv head)
// computes the split's (m, l, O) for all G query heads of the kv head, so
// each K/V element is read once per group (the generic kernel reads it once
// per query head). The same two passes as decode_generic
// (PagedAttention.h:98-118): per token the G scores, each a dot product over
// d in order (four elements per load, the query rows read four floats at a
// time from LDS); per head the maximum; then weights, their sum and the value
// accumulator, each thread holding four dims of all heads over a contiguous
// run of tokens (weights read four tokens at a time); the runs' partial sums
// are added in run order and the generic split merge finishes. kG >= G is
// the register width of the per-head arrays: query rows past G are zero, and
// their scores and sums are computed but never stored.
template <typename T, int kG>
__global__ __launch_bounds__(kGroupedThreads) void decode_grouped(DecodeGeometry p, SplitArgs sa) {
    extern __shared__ float smem[];
    __shared__ float red[kGroupedWaves][kG];
    const int G = static_cast<int>(p.group);
    const uint32_t D = p.head_dim;
    const uint32_t S = sa.split_tokens;
    float* q_s = smem;           // [kG][D]
    float* s_s = smem + kG * D;  // [kG][S]: scores, then weights

    const uint32_t split = blockIdx.x / p.num_kv_heads;
    const uint32_t g = blockIdx.x - split * p.num_kv_heads;
    const int b = sa.split_seq[split];
    const int start = sa.split_start[split];
    const int ctx = p.seq_lens[b];
    const int len = min(static_cast<int>(S), ctx - start);
    const int32_t* row = p.tables + static_cast<uint64_t>(b) * p.max_nb;
    const uint64_t head0 = static_cast<uint64_t>(b) * p.num_q_heads + static_cast<uint64_t>(g) * G;

    const T* q = static_cast<const T*>(p.query) + head0 * D;
    for (uint32_t e = threadIdx.x; e < kG * D; e += kGroupedThreads) {
        q_s[e] = e < static_cast<uint32_t>(G) * D ? to_float<T>(q[e]) : 0.f;
    }
    __syncthreads();

    const uint64_t head_off = static_cast<uint64_t>(g) * p.head_stride;
    auto row_of = [&](int t, uint64_t off) {
        const uint32_t tok = static_cast<uint32_t>(start + t);
        const int32_t blk = row[tok / p.tpb];
        return reinterpret_cast<const T*>(p.kv_base + static_cast<uint64_t>(blk) * p.block_stride + off +
                                          (tok % p.tpb) * p.token_stride + head_off);
    };
    float mloc[kG];
#pragma unroll
    for (int h = 0; h < kG; ++h) mloc[h] = -INFINITY;
    for (int t = threadIdx.x; t < len; t += kGroupedThreads) {
        const T* k = row_of(t, p.k_off);
        float dot[kG];
#pragma unroll
        for (int h = 0; h < kG; ++h) dot[h] = 0.f;
        for (uint32_t d = 0; d < D; d += 4) {
            const float4 kv = load4<T>(k + d);
#pragma unroll
            for (int h = 0; h < kG; ++h) {
                const float4 qv = *reinterpret_cast<const float4*>(&q_s[h * D + d]);
                dot[h] = fmaf(qv.x, kv.x, dot[h]);
                dot[h] = fmaf(qv.y, kv.y, dot[h]);
                dot[h] = fmaf(qv.z, kv.z, dot[h]);
                dot[h] = fmaf(qv.w, kv.w, dot[h]);
            }
        }
#pragma unroll
        for (int h = 0; h < kG; ++h) {
            const float sv = dot[h] * p.scale_log2;
            s_s[h * S + t] = sv;
            mloc[h] = fmaxf(mloc[h], sv);
        }
    }
    reduce_heads<kG, true>(mloc, red);
    float lloc[kG];
#pragma unroll
    for (int h = 0; h < kG; ++h) lloc[h] = 0.f;
    for (int t = threadIdx.x; t < len; t += kGroupedThreads) {
#pragma unroll
        for (int h = 0; h < kG; ++h) {
            const float w = fast_exp2(s_s[h * S + t] - mloc[h]);
            s_s[h * S + t] = w;
            lloc[h] += w;
        }
    }
    // Also orders the weight writes before the reads below.
    reduce_heads<kG, false>(lloc, red);

    // Thread (run r, chunk c): dims 4c .. 4c + 3 over tokens [r * run,
    // min(len, (r + 1) * run)), run a multiple of four tokens.
    const int chunks = static_cast<int>(D / 4);
    const int runs = kGroupedThreads / chunks;
    const int r = static_cast<int>(threadIdx.x) / chunks;
    const int c4 = 4 * (static_cast<int>(threadIdx.x) - r * chunks);
    const int run = (((len + runs - 1) / runs) + 3) & ~3;
    float acc[kG][4];
#pragma unroll
    for (int h = 0; h < kG; ++h)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[h][e] = 0.f;
    if (r < runs) {
        const int t0 = r * run;
        const int t1 = min(len, t0 + run);
        int t = t0;
        for (; t + 4 <= t1; t += 4) {
            float4 vv[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) vv[u] = load4<T>(row_of(t + u, p.v_off) + c4);
#pragma unroll
            for (int h = 0; h < kG; ++h) {
                const float4 w = *reinterpret_cast<const float4*>(&s_s[h * S + t]);
                const float wu[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    acc[h][0] = fmaf(wu[u], vv[u].x, acc[h][0]);
                    acc[h][1] = fmaf(wu[u], vv[u].y, acc[h][1]);
                    acc[h][2] = fmaf(wu[u], vv[u].z, acc[h][2]);
                    acc[h][3] = fmaf(wu[u], vv[u].w, acc[h][3]);
                }
            }
        }
        for (; t < t1; ++t) {
            const float4 vv = load4<T>(row_of(t, p.v_off) + c4);
#pragma unroll
            for (int h = 0; h < kG; ++h) {
                const float w = s_s[h * S + t];
                acc[h][0] = fmaf(w, vv.x, acc[h][0]);
                acc[h][1] = fmaf(w, vv.y, acc[h][1]);
                acc[h][2] = fmaf(w, vv.z, acc[h][2]);
                acc[h][3] = fmaf(w, vv.w, acc[h][3]);
            }
        }
    }
    __syncthreads();  // every weight read before the partial sums reuse the LDS
    float* part = smem;  // [runs][kG][D]
    if (r < runs) {
#pragma unroll
        for (int h = 0; h < kG; ++h) {
            *reinterpret_cast<float4*>(&part[(r * kG + h) * D + c4]) = float4{acc[h][0], acc[h][1], acc[h][2], acc[h][3]};
        }
    }
    __syncthreads();
    float* acc_out = sa.ws_acc + static_cast<uint64_t>(split) * p.num_q_heads * D + static_cast<uint64_t>(g) * G * D;
    for (uint32_t e = threadIdx.x; e < static_cast<uint32_t>(G) * D; e += kGroupedThreads) {
        const uint32_t h = e / D;
        const uint32_t dd = e - h * D;
        float o = 0.f;
        for (int x = 0; x < runs; ++x) o += part[(x * kG + h) * D + dd];
        acc_out[e] = o;
    }
    float* ml = sa.ws_ml + (static_cast<uint64_t>(split) * p.num_q_heads + static_cast<uint64_t>(g) * G) * 2;
#pragma unroll
    for (int h = 0; h < kG; ++h) {
        if (h < G && static_cast<int>(threadIdx.x) == h) {
            ml[2 * h] = mloc[h];
            ml[2 * h + 1] = lloc[h];
        }
    }
}

// Register width of the folded kernel's per-head arrays for a group.
int grouped_width(uint32_t group) { return group <= 1 ? 1 : group <= 2 ? 2 : group <= 4 ? 4 : group <= 8 ? 8 : 16; }

// LDS of the folded kernel: query rows and scores, later the runs' partial
// sums ((256 / (D / 4)) runs x kG x D floats).
size_t grouped_shmem(const DecodeGeometry& g, uint32_t split_tokens) {
    const size_t kg = static_cast<size_t>(grouped_width(g.group));
    const size_t d = g.head_dim;
    const size_t runs = d >= 4 ? kGroupedThreads / (d / 4) : 0;
    return std::max(kg * (d + split_tokens), runs * kg * d) * sizeof(float);
}

template <typename T>
void launch_grouped_for(const DecodeGeometry& g, const SplitArgs& sa, dim3 grid, size_t shmem, hipStream_t stream) {
    switch (grouped_width(g.group)) {
        case 1: hipLaunchKernelGGL((decode_grouped<T, 1>), grid, dim3(kGroupedThreads), shmem, stream, g, sa); break;
        case 2: hipLaunchKernelGGL((decode_grouped<T, 2>), grid, dim3(kGroupedThreads), shmem, stream, g, sa); break;
        case 4: hipLaunchKernelGGL((decode_grouped<T, 4>), grid, dim3(kGroupedThreads), shmem, stream, g, sa); break;
        case 8: hipLaunchKernelGGL((decode_grouped<T, 8>), grid, dim3(kGroupedThreads), shmem, stream, g, sa); break;
        default: hipLaunchKernelGGL((decode_grouped<T, 16>), grid, dim3(kGroupedThreads), shmem, stream, g, sa); break;
    }
}

}  // namespace

bool grouped_supported(const DecodeGeometry& g, uint32_t kv_dtype, uint32_t split_tokens) {
    // Four-element K/V loads: rows, frames and the pool aligned to four
    // elements; head_dim a multiple of four with at most 256 four-dim chunks;
    // weights read four tokens at a time (splits of a multiple of four).
    const uint64_t a = 4ull * (kv_dtype == QVP_DTYPE_F32 ? 4 : 2);
    const bool aligned = g.token_stride % a == 0 && g.head_stride % a == 0 && g.block_stride % a == 0 &&
                         g.k_off % a == 0 && g.v_off % a == 0 && reinterpret_cast<uintptr_t>(g.kv_base) % a == 0;
    return g.group >= 1 && g.group <= 16 && g.head_dim % 4 == 0 && g.head_dim >= 4 &&
           g.head_dim <= 4 * kGroupedThreads && split_tokens >= 4 && split_tokens % 4 == 0 && aligned &&
           grouped_shmem(g, split_tokens) <= 64 * 1024;
}

int launch_grouped_decode(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t kv_dtype, uint32_t out_dtype,
                          void* out, void* workspace, hipEvent_t split_event, hipStream_t stream) {
    if (!grouped_supported(g, kv_dtype, v.split_tokens)) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "group %u, head_dim %u, split %u: not a folded-decode shape", g.group,
                    g.head_dim, v.split_tokens);
    }
    const uint64_t heads = static_cast<uint64_t>(v.num_splits) * g.num_q_heads;
    SplitArgs sa{};
    sa.split_seq = v.split_seq;
    sa.split_start = v.split_start;
    sa.split_tokens = v.split_tokens;
    sa.ws_ml = static_cast<float*>(workspace);
    sa.ws_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + round_up(heads * 2 * sizeof(float), 256));
    const size_t shmem = grouped_shmem(g, v.split_tokens);
    const dim3 grid(static_cast<unsigned>(static_cast<uint64_t>(v.num_splits) * g.num_kv_heads));
    switch (kv_dtype) {
        case QVP_DTYPE_F32: launch_grouped_for<float>(g, sa, grid, shmem, stream); break;
        case QVP_DTYPE_BF16: launch_grouped_for<uint16_t>(g, sa, grid, shmem, stream); break;
        default: launch_grouped_for<_Float16>(g, sa, grid, shmem, stream); break;
    }
    QVP_HIP(hipGetLastError());
    if (split_event != nullptr) QVP_HIP(hipEventRecord(split_event, stream));
    return launch_merge_splits(g, v, out_dtype, out, sa.ws_ml, sa.ws_acc, stream);
}

uint64_t generic_workspace_bytes(const qvp_packed_view& v, uint32_t hq, uint32_t d) {
    const uint64_t heads = static_cast<uint64_t>(v.num_splits) * hq;
    return round_up(heads * 2 * sizeof(float), 256) + round_up(heads * d * sizeof(float), 256);
}

int launch_generic_decode(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t kv_dtype, uint32_t out_dtype,
                          void* out, void* workspace, hipEvent_t split_event, hipStream_t stream) {
    const uint64_t heads = static_cast<uint64_t>(v.num_splits) * g.num_q_heads;
    SplitArgs sa{};
    sa.split_seq = v.split_seq;
    sa.split_start = v.split_start;
    sa.split_tokens = v.split_tokens;
    sa.ws_ml = static_cast<float*>(workspace);
    sa.ws_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + round_up(heads * 2 * sizeof(float), 256));
    const size_t shmem = (static_cast<size_t>(g.head_dim) + v.split_tokens) * sizeof(float);
    if (shmem > 64 * 1024) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "head_dim %u with split %u needs %zu bytes of LDS", g.head_dim,
                    v.split_tokens, shmem);
    }
    const dim3 grid(static_cast<unsigned>(heads));
    switch (kv_dtype) {
        case QVP_DTYPE_F32:
            hipLaunchKernelGGL(decode_generic<float>, grid, dim3(kGenericThreads), shmem, stream, g, sa);
            break;
        case QVP_DTYPE_BF16:
            hipLaunchKernelGGL(decode_generic<uint16_t>, grid, dim3(kGenericThreads), shmem, stream, g, sa);
            break;
        default:
            hipLaunchKernelGGL(decode_generic<_Float16>, grid, dim3(kGenericThreads), shmem, stream, g, sa);
            break;
    }
    QVP_HIP(hipGetLastError());
    if (split_event != nullptr) QVP_HIP(hipEventRecord(split_event, stream));

    return launch_merge_splits(g, v, out_dtype, out, sa.ws_ml, sa.ws_acc, stream);
}

int launch_merge_splits(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t out_dtype, void* out,
                        const float* ws_ml, const float* ws_acc, hipStream_t stream) {
    const dim3 mgrid(v.num_seqs * g.num_q_heads);
    switch (out_dtype) {
        case QVP_DTYPE_F32:
            hipLaunchKernelGGL(merge_splits<float>, mgrid, dim3(kMergeThreads), 0, stream, ws_ml, ws_acc, v.cu_splits,
                               static_cast<float*>(out), g.num_q_heads, g.head_dim);
            break;
        case QVP_DTYPE_BF16:
            hipLaunchKernelGGL(merge_splits<uint16_t>, mgrid, dim3(kMergeThreads), 0, stream, ws_ml, ws_acc, v.cu_splits,
                               static_cast<uint16_t*>(out), g.num_q_heads, g.head_dim);
            break;
        default:
            hipLaunchKernelGGL(merge_splits<_Float16>, mgrid, dim3(kMergeThreads), 0, stream, ws_ml, ws_acc, v.cu_splits,
                               static_cast<_Float16*>(out), g.num_q_heads, g.head_dim);
            break;
    }
    QVP_HIP(hipGetLastError());
    return QVP_OK;
}

}  // namespace qvp

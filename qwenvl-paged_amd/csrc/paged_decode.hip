// Split-K (flash-decoding) paged decode over a packed ragged batch, gfx950.
//
// Semantics follow the reference CPU kernel paged_attention_decode<T>
// (include/qwenvl_paged/PagedAttention.h:53-127): for query head h the output is
// softmax(scale * q_h . K_g^T) V_g with g = h / (Hq / Hkv) and fp32 accumulation.
// The reference runs two passes (max, then exp/sum/accumulate) per head; here
// each split of a sequence keeps a running max m, a running sum l and an
// unnormalised accumulator (online softmax), and a second kernel merges the
// splits: out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s.
// Scores are kept in base 2 (scale * log2(e) folded into one multiplier), so
// every exponential is a single v_exp_f32.
//
// Two decode kernels share that split format:
//   decode_mfma_bf16_d128  bf16 cache, head_dim 128, GQA group <= 16. One
//                          workgroup (4 waves) per (split, kv head); the whole
//                          query-head group of that kv head rides in the 16
//                          columns of one MFMA tile, so every K/V byte is read
//                          from HBM once. QK^T and PV both run on
//                          v_mfma_f32_16x16x32_bf16.
//   decode_generic         any dtype / head_dim / group; VALU, one workgroup per
//                          (split, query head). Used for fp32 caches and shapes
//                          the MFMA kernel does not cover.
#include "common.h"

#include <algorithm>
#include <mutex>
#include <vector>

struct qvp_batch;  // defined in pack.hip; only the public view is used here

namespace {

using qvp::fail;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMfmaWaves = 4;
constexpr int kMfmaThreads = kMfmaWaves * 64;
constexpr int kMfmaMaxTableEntries = 512;  // block ids of one split staged in LDS
constexpr int kGenericThreads = 128;

struct DecodeParams {
    const uint8_t* kv_base;
    uint64_t block_stride;  // bytes
    uint64_t k_off;         // bytes from frame start to this layer's K half
    uint64_t v_off;         // bytes from frame start to this layer's V half
    uint64_t token_stride;  // bytes
    uint64_t head_stride;   // bytes
    const int32_t* tables;
    const int32_t* seq_lens;
    const int32_t* split_seq;
    const int32_t* split_start;
    const void* query;
    float* ws_ml;   // [num_splits][Hq][2] : running max (base 2) and sum
    float* ws_acc;  // [num_splits][Hq][D] : unnormalised accumulator
    uint32_t max_nb;
    uint32_t tpb;
    uint32_t tpb_shift;
    uint32_t split_tokens;
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t head_dim;
    float scale_log2;
};

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline u32x4 load_u32x4(const uint8_t* p) {
    return *reinterpret_cast<const u32x4*>(p);
}

// bf16 bits of x with the low 16 mantissa bits dropped (x - hi is exact in fp32).
__device__ inline uint32_t bf16_trunc_bits(float x) { return __float_as_uint(x) >> 16; }

// ---------------------------------------------------------------------------
// MFMA kernel, bf16 cache, head_dim 128.
//
// Lane l of a wave is (c = l % 16, j = l / 16). v_mfma_f32_16x16x32_bf16 takes
// A[row][k] from lane (row, k / 8), B[k][col] from lane (col, k / 8) and
// returns C[4 * j + r][c] in register r of lane (c, j).
//
// Tile = 32 tokens of one split. QK^T is computed transposed, S^T = K Q^T, in
// two 16-token halves u. Row r of half u carries token (r / 4) + 16u + 4 (r % 4)
// of the tile, so the C register r of lane (c, j) holds the score of token
// j + 4 (4u + r) for query head c. The contraction order over head_dim is free;
// the four k-groups of MFMA i cover dims 32i .. 32i + 31.
//
// PV is computed as O^T = V^T P^T. Lane (c, j) holds P for tokens j + 4q,
// q = 0..7, which is exactly the B operand (k slot q <-> token j + 4q). The V
// tile is loaded with 16-byte coalesced loads where lane (c, j) of load q reads
// dims 8c .. 8c + 7 of token 4q + j; row x of PV MFMA n stands for dim 8x + n,
// so lane (c, j) already owns its whole A operand (element n of each of its 8
// loads) and only an in-register 16-bit transpose is needed, no LDS round trip.
// P enters the bf16 MFMA as a hi + lo pair (hi = P truncated to bf16, lo = P - hi
// rounded to bf16), which keeps the weights at ~2^-16 relative error.
// C register r of PV MFMA n in lane (c, j) is O[head c][dim 32j + 8r + n].
// ---------------------------------------------------------------------------

struct KvTile {
    u32x4 k[2][4];  // [half u][mfma i]
    u32x4 v[8];     // [load q]
};

__device__ inline void load_tile(const DecodeParams& p, const int32_t* sm_blk, int first_blk,
                                 int end, int tb, int c, int j, uint64_t k_lane_off,
                                 uint64_t v_lane_off, KvTile& t) {
    const uint32_t tmask = p.tpb - 1;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        int tok = tb + (c >> 2) + 16 * u + 4 * (c & 3);
        tok = min(tok, end - 1);
        const int32_t blk = sm_blk[(tok >> p.tpb_shift) - first_blk];
        const uint8_t* base = p.kv_base + static_cast<uint64_t>(blk) * p.block_stride +
                              static_cast<uint64_t>(tok & tmask) * p.token_stride + k_lane_off;
#pragma unroll
        for (int i = 0; i < 4; ++i) t.k[u][i] = load_u32x4(base + 64 * i);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const int tok_raw = tb + 4 * q + j;
        const int tok = min(tok_raw, end - 1);
        const int32_t blk = sm_blk[(tok >> p.tpb_shift) - first_blk];
        const uint8_t* base = p.kv_base + static_cast<uint64_t>(blk) * p.block_stride +
                              static_cast<uint64_t>(tok & tmask) * p.token_stride + v_lane_off;
        u32x4 v = load_u32x4(base);
        if (tok_raw >= end) v = u32x4{0u, 0u, 0u, 0u};
        t.v[q] = v;
    }
}

__global__ __launch_bounds__(kMfmaThreads, 2) void decode_mfma_bf16_d128(DecodeParams p) {
    constexpr int D = 128;
    constexpr int kRowPad = D + 4;
    __shared__ int32_t sm_blk[kMfmaMaxTableEntries];
    __shared__ float sm_m[kMfmaWaves][16];
    __shared__ float sm_l[kMfmaWaves][16];
    __shared__ float sm_o[kMfmaWaves][16][kRowPad];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int c = lane & 15;
    const int j = lane >> 4;

    const uint32_t split = blockIdx.x / p.num_kv_heads;
    const uint32_t g = blockIdx.x - split * p.num_kv_heads;
    const int b = p.split_seq[split];
    const int start = p.split_start[split];
    const int ctx = p.seq_lens[b];
    const int len = min(static_cast<int>(p.split_tokens), ctx - start);
    const int end = start + len;
    const int n_tiles = (len + 31) >> 5;

    // Stage this split's block ids in LDS.
    const int first_blk = start >> p.tpb_shift;
    {
        const int32_t* row = p.tables + static_cast<uint64_t>(b) * p.max_nb;
        const int count = ((end - 1) >> p.tpb_shift) - first_blk + 1;
        for (int e = threadIdx.x; e < count; e += kMfmaThreads) sm_blk[e] = row[first_blk + e];
    }

    // Query B operand: lane (c, j), MFMA i -> Q[head g*G + c][dims 32i + 8j .. +8].
    u32x4 qop[4];
    {
        const bool live = static_cast<uint32_t>(c) < p.group;
        const uint16_t* q = static_cast<const uint16_t*>(p.query) +
                            (static_cast<uint64_t>(b) * p.num_q_heads + g * p.group +
                             (live ? c : 0)) * D;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            u32x4 v = *reinterpret_cast<const u32x4*>(q + 32 * i + 8 * j);
            qop[i] = live ? v : u32x4{0u, 0u, 0u, 0u};
        }
    }
    __syncthreads();

    const uint64_t k_lane_off = p.k_off + g * p.head_stride + 16u * j;
    const uint64_t v_lane_off = p.v_off + g * p.head_stride + 16u * c;

    floatx4 o[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    float l_run = 0.f;

    KvTile nxt;
    int t = wave;
    if (t < n_tiles) load_tile(p, sm_blk, first_blk, end, start + 32 * t, c, j, k_lane_off, v_lane_off, nxt);
    for (; t < n_tiles; t += kMfmaWaves) {
        const KvTile cur = nxt;
        const int tb = start + 32 * t;
        if (t + kMfmaWaves < n_tiles) {
            load_tile(p, sm_blk, first_blk, end, tb + 32 * kMfmaWaves, c, j, k_lane_off, v_lane_off, nxt);
        }

        // S^T = K Q^T for both halves.
        float s[2][4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    __builtin_bit_cast(bf16x8_t, cur.k[u][i]), __builtin_bit_cast(bf16x8_t, qop[i]),
                    acc, 0, 0, 0);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tok = tb + j + 16 * u + 4 * r;
                s[u][r] = (tok < end) ? acc[r] * p.scale_log2 : -INFINITY;
            }
        }

        // Online softmax: the max is shared by the 4 lanes (c, 0..3) of head c.
        float mt = s[0][0];
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) mt = fmaxf(mt, s[u][r]);
        mt = fmaxf(mt, __shfl_xor(mt, 16));
        mt = fmaxf(mt, __shfl_xor(mt, 32));
        const float m_new = fmaxf(m_run, mt);
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;

        float psum = 0.f;
        uint32_t phi[4], plo[4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int r = 0; r < 4; r += 2) {
                const float p0 = fast_exp2(s[u][r] - m_new);
                const float p1 = fast_exp2(s[u][r + 1] - m_new);
                psum += p0 + p1;
                const uint32_t h0 = bf16_trunc_bits(p0);
                const uint32_t h1 = bf16_trunc_bits(p1);
                const float r0 = p0 - __uint_as_float(h0 << 16);
                const float r1 = p1 - __uint_as_float(h1 << 16);
                const uint32_t l0 = qvp::float_to_bf16_bits(r0);
                const uint32_t l1 = qvp::float_to_bf16_bits(r1);
                phi[2 * u + r / 2] = h0 | (h1 << 16);
                plo[2 * u + r / 2] = l0 | (l1 << 16);
            }
        }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int n = 0; n < 8; ++n) o[n] *= alpha;

        const u32x4 bhi = {phi[0], phi[1], phi[2], phi[3]};
        const u32x4 blo = {plo[0], plo[1], plo[2], plo[3]};
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            // A operand of MFMA n: element n of each of the 8 V loads.
            const int w = n >> 1;
            u32x4 a;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t x = cur.v[2 * k][w];
                const uint32_t y = cur.v[2 * k + 1][w];
                a[k] = (n & 1) ? ((x >> 16) | (y & 0xffff0000u)) : ((x & 0xffffu) | (y << 16));
            }
            const bf16x8_t av = __builtin_bit_cast(bf16x8_t, a);
            o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8_t, bhi),
                                                           o[n], 0, 0, 0);
            o[n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, __builtin_bit_cast(bf16x8_t, blo),
                                                           o[n], 0, 0, 0);
        }
    }

    // Sum l over the 4 lanes of each head, then merge the 4 waves in LDS.
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (j == 0) {
        sm_m[wave][c] = m_run;
        sm_l[wave][c] = l_run;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int n = 0; n < 8; ++n) sm_o[wave][c][32 * j + 8 * r + n] = o[n][r];
    __syncthreads();

    const uint32_t G = p.group;
    const uint64_t head0 = static_cast<uint64_t>(split) * p.num_q_heads + g * G;
    for (uint32_t e = threadIdx.x; e < G * D; e += kMfmaThreads) {
        const uint32_t hc = e / D;
        const uint32_t d = e - hc * D;
        float mmax = sm_m[0][hc];
#pragma unroll
        for (int w = 1; w < kMfmaWaves; ++w) mmax = fmaxf(mmax, sm_m[w][hc]);
        float acc = 0.f;
        float lsum = 0.f;
#pragma unroll
        for (int w = 0; w < kMfmaWaves; ++w) {
            const float f = fast_exp2(sm_m[w][hc] - mmax);
            acc += sm_o[w][hc][d] * f;
            lsum += sm_l[w][hc] * f;
        }
        p.ws_acc[(head0 + hc) * D + d] = acc;
        if (d == 0) {
            p.ws_ml[(head0 + hc) * 2 + 0] = mmax;
            p.ws_ml[(head0 + hc) * 2 + 1] = lsum;
        }
    }
}

// ---------------------------------------------------------------------------
// Generic kernel: any element type, head_dim, group size and block size.
// ---------------------------------------------------------------------------

template <typename T> __device__ inline float to_float(T v);
template <> __device__ inline float to_float<float>(float v) { return v; }
template <> __device__ inline float to_float<uint16_t>(uint16_t v) { return qvp::bf16_bits_to_float(v); }
template <> __device__ inline float to_float<_Float16>(_Float16 v) { return static_cast<float>(v); }

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

template <typename T>
__global__ __launch_bounds__(kGenericThreads) void decode_generic(DecodeParams p) {
    extern __shared__ float smem[];
    float* q_s = smem;                  // [head_dim]
    float* s_s = smem + p.head_dim;     // [split_tokens]
    __shared__ float red[kGenericThreads / 64];

    const uint32_t split = blockIdx.x / p.num_q_heads;
    const uint32_t h = blockIdx.x - split * p.num_q_heads;
    const uint32_t g = h / p.group;
    const int b = p.split_seq[split];
    const int start = p.split_start[split];
    const int ctx = p.seq_lens[b];
    const int len = min(static_cast<int>(p.split_tokens), ctx - start);
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
        const T* k = reinterpret_cast<const T*>(p.kv_base + static_cast<uint64_t>(blk) * p.block_stride +
                                                p.k_off + (tok % p.tpb) * p.token_stride + head_off);
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

    float* acc_out = p.ws_acc + (static_cast<uint64_t>(split) * p.num_q_heads + h) * D;
    for (uint32_t d = threadIdx.x; d < D; d += blockDim.x) {
        float acc = 0.f;
        for (int t = 0; t < len; ++t) {
            const uint32_t tok = static_cast<uint32_t>(start + t);
            const int32_t blk = row[tok / p.tpb];
            const T* v = reinterpret_cast<const T*>(p.kv_base + static_cast<uint64_t>(blk) * p.block_stride +
                                                    p.v_off + (tok % p.tpb) * p.token_stride + head_off);
            acc += s_s[t] * to_float<T>(v[d]);
        }
        acc_out[d] = acc;
    }
    if (threadIdx.x == 0) {
        p.ws_ml[(static_cast<uint64_t>(split) * p.num_q_heads + h) * 2 + 0] = m;
        p.ws_ml[(static_cast<uint64_t>(split) * p.num_q_heads + h) * 2 + 1] = l;
    }
}

// ---------------------------------------------------------------------------
// Split merge: one workgroup per (sequence, query head).
// ---------------------------------------------------------------------------

template <typename OutT> __device__ inline OutT from_float(float v);
template <> __device__ inline float from_float<float>(float v) { return v; }
template <> __device__ inline uint16_t from_float<uint16_t>(float v) { return qvp::float_to_bf16_bits(v); }
template <> __device__ inline _Float16 from_float<_Float16>(float v) { return static_cast<_Float16>(v); }

template <typename OutT>
__global__ __launch_bounds__(128) void merge_splits(const float* __restrict__ ws_ml,
                                                    const float* __restrict__ ws_acc,
                                                    const int32_t* __restrict__ cu_splits,
                                                    OutT* __restrict__ out, uint32_t num_q_heads,
                                                    uint32_t head_dim) {
    const uint32_t b = blockIdx.x / num_q_heads;
    const uint32_t h = blockIdx.x - b * num_q_heads;
    const int s0 = cu_splits[b];
    const int s1 = cu_splits[b + 1];
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

// ---------------------------------------------------------------------------
// Library-managed workspace (one per device, grows on demand).
// ---------------------------------------------------------------------------

struct Workspace {
    void* ptr{nullptr};
    uint64_t bytes{0};
};

std::mutex g_ws_mutex;
std::vector<Workspace> g_ws;

int library_workspace(uint64_t need, void** out) {
    int dev = 0;
    QVP_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if (g_ws.size() <= static_cast<size_t>(dev)) g_ws.resize(dev + 1);
    Workspace& ws = g_ws[dev];
    if (ws.bytes < need) {
        if (ws.ptr != nullptr) {
            // Earlier launches may still read the old buffer.
            QVP_HIP(hipDeviceSynchronize());
            QVP_HIP(hipFree(ws.ptr));
            ws.ptr = nullptr;
            ws.bytes = 0;
        }
        const uint64_t cap = std::max<uint64_t>(need + need / 4, 1u << 20);
        QVP_HIP(hipMalloc(&ws.ptr, cap));
        ws.bytes = cap;
    }
    *out = ws.ptr;
    return QVP_OK;
}

uint64_t workspace_need(const qvp_packed_view& v, uint32_t hq, uint32_t d) {
    const uint64_t heads = static_cast<uint64_t>(v.num_splits) * hq;
    const uint64_t ml = qvp::round_up(heads * 2 * sizeof(float), 256);
    return ml + qvp::round_up(heads * d * sizeof(float), 256);
}

bool is_pow2(uint32_t x) { return x != 0 && (x & (x - 1)) == 0; }

uint32_t log2_u32(uint32_t x) {
    uint32_t r = 0;
    while ((1u << r) < x) ++r;
    return r;
}

}  // namespace

extern "C" {

int qvp_decode_workspace_bytes(const qvp_batch* batch, uint32_t num_query_heads, uint32_t head_dim,
                               uint64_t* bytes) {
    if (bytes == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "bytes is NULL");
    qvp_packed_view v{};
    QVP_TRY(qvp_batch_view(batch, &v));
    *bytes = workspace_need(v, num_query_heads, head_dim);
    return QVP_OK;
}

int qvp_paged_decode(const qvp_decode_args* a, void* stream) {
    if (a == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "args is NULL");
    qvp_packed_view v{};
    QVP_TRY(qvp_batch_view(a->batch, &v));
    if (a->query == nullptr || a->out == nullptr || a->kv_base == nullptr) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "query, out or kv_base is NULL");
    }
    const size_t esz = qvp::dtype_size(a->kv_dtype);
    const size_t osz = qvp::dtype_size(a->out_dtype);
    if (esz == 0 || osz == 0) return fail(QVP_ERR_INVALID_ARGUMENT, "unknown dtype");
    // Argument checks of the reference (PagedAttention.h:63-68).
    if (a->num_query_heads == 0 || a->num_kv_heads == 0 || a->num_query_heads % a->num_kv_heads != 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "%u query heads do not group onto %u kv heads",
                    a->num_query_heads, a->num_kv_heads);
    }
    if (a->layer >= a->num_layers) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "layer %u outside %u layers", a->layer, a->num_layers);
    }
    if (a->head_dim == 0) return fail(QVP_ERR_INVALID_ARGUMENT, "head_dim is 0");
    if (a->tokens_per_block != v.tokens_per_block) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "batch packed for %u tokens per block, args say %u",
                    v.tokens_per_block, a->tokens_per_block);
    }
    // Every element the kernels can address must lie inside one frame.
    const uint64_t last_elem = static_cast<uint64_t>(a->num_layers - 1) * a->layer_stride +
                               a->stream_stride +
                               static_cast<uint64_t>(a->tokens_per_block - 1) * a->token_stride +
                               static_cast<uint64_t>(a->num_kv_heads - 1) * a->head_stride + a->head_dim;
    if (last_elem * esz > a->block_stride) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "layout addresses %llu bytes but frames are %llu bytes",
                    static_cast<unsigned long long>(last_elem * esz),
                    static_cast<unsigned long long>(a->block_stride));
    }
    if (a->head_stride < a->head_dim || a->token_stride == 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "head vectors overlap (head_stride %llu < head_dim %u)",
                    static_cast<unsigned long long>(a->head_stride), a->head_dim);
    }
    if (v.num_seqs == 0) return QVP_OK;

    const uint32_t group = a->num_query_heads / a->num_kv_heads;
    const uint64_t need = workspace_need(v, a->num_query_heads, a->head_dim);
    void* ws = a->workspace;
    if (ws == nullptr) {
        QVP_TRY(library_workspace(need, &ws));
    } else if (a->workspace_bytes < need) {
        return fail(QVP_ERR_CAPACITY, "workspace of %llu bytes, need %llu",
                    static_cast<unsigned long long>(a->workspace_bytes),
                    static_cast<unsigned long long>(need));
    } else if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    }

    DecodeParams p{};
    p.kv_base = static_cast<const uint8_t*>(a->kv_base);
    p.block_stride = a->block_stride;
    p.k_off = static_cast<uint64_t>(a->layer) * a->layer_stride * esz;
    p.v_off = p.k_off + a->stream_stride * esz;
    p.token_stride = a->token_stride * esz;
    p.head_stride = a->head_stride * esz;
    p.tables = v.block_tables;
    p.seq_lens = v.seq_lens;
    p.split_seq = v.split_seq;
    p.split_start = v.split_start;
    p.query = a->query;
    const uint64_t heads = static_cast<uint64_t>(v.num_splits) * a->num_query_heads;
    p.ws_ml = static_cast<float*>(ws);
    p.ws_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) +
                                        qvp::round_up(heads * 2 * sizeof(float), 256));
    p.max_nb = v.max_blocks_per_seq;
    p.tpb = a->tokens_per_block;
    p.tpb_shift = log2_u32(a->tokens_per_block);
    p.split_tokens = v.split_tokens;
    p.num_q_heads = a->num_query_heads;
    p.num_kv_heads = a->num_kv_heads;
    p.group = group;
    p.head_dim = a->head_dim;
    p.scale_log2 = a->scale * kLog2e;

    const uintptr_t qaddr = reinterpret_cast<uintptr_t>(a->query);
    const bool aligned16 = (a->block_stride % 16 == 0) && (p.k_off % 16 == 0) && (p.v_off % 16 == 0) &&
                           (p.token_stride % 16 == 0) && (p.head_stride % 16 == 0) &&
                           (reinterpret_cast<uintptr_t>(a->kv_base) % 16 == 0) && (qaddr % 16 == 0);
    const bool use_mfma = a->kv_dtype == QVP_DTYPE_BF16 && a->head_dim == 128 && group <= 16 &&
                          aligned16 && is_pow2(a->tokens_per_block) &&
                          (v.split_tokens >> p.tpb_shift) + 1 <= static_cast<uint32_t>(kMfmaMaxTableEntries);

    hipStream_t s = qvp::as_stream(stream);
    if (use_mfma) {
        const uint64_t grid = static_cast<uint64_t>(v.num_splits) * a->num_kv_heads;
        hipLaunchKernelGGL(decode_mfma_bf16_d128, dim3(static_cast<unsigned>(grid)), dim3(kMfmaThreads),
                           0, s, p);
    } else {
        const uint64_t grid = heads;
        const size_t shmem = (static_cast<size_t>(a->head_dim) + v.split_tokens) * sizeof(float);
        if (shmem > 64 * 1024) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "head_dim %u with split %u needs %zu bytes of LDS",
                        a->head_dim, v.split_tokens, shmem);
        }
        switch (a->kv_dtype) {
            case QVP_DTYPE_F32:
                hipLaunchKernelGGL(decode_generic<float>, dim3(static_cast<unsigned>(grid)),
                                   dim3(kGenericThreads), shmem, s, p);
                break;
            case QVP_DTYPE_BF16:
                hipLaunchKernelGGL(decode_generic<uint16_t>, dim3(static_cast<unsigned>(grid)),
                                   dim3(kGenericThreads), shmem, s, p);
                break;
            default:
                hipLaunchKernelGGL(decode_generic<_Float16>, dim3(static_cast<unsigned>(grid)),
                                   dim3(kGenericThreads), shmem, s, p);
                break;
        }
    }
    QVP_HIP(hipGetLastError());

    const dim3 mgrid(v.num_seqs * a->num_query_heads);
    switch (a->out_dtype) {
        case QVP_DTYPE_F32:
            hipLaunchKernelGGL(merge_splits<float>, mgrid, dim3(128), 0, s, p.ws_ml, p.ws_acc,
                               v.cu_splits, static_cast<float*>(a->out), a->num_query_heads, a->head_dim);
            break;
        case QVP_DTYPE_BF16:
            hipLaunchKernelGGL(merge_splits<uint16_t>, mgrid, dim3(128), 0, s, p.ws_ml, p.ws_acc,
                               v.cu_splits, static_cast<uint16_t*>(a->out), a->num_query_heads,
                               a->head_dim);
            break;
        default:
            hipLaunchKernelGGL(merge_splits<_Float16>, mgrid, dim3(128), 0, s, p.ws_ml, p.ws_acc,
                               v.cu_splits, static_cast<_Float16*>(a->out), a->num_query_heads,
                               a->head_dim);
            break;
    }
    QVP_HIP(hipGetLastError());
    return QVP_OK;
}

}  // extern "C"

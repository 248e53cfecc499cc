// Matrix-core split decode for bf16 and fp16 caches with head_dim 64 -- the
// reference's paged_attention_decode<T> (include/qwenvl_paged/PagedAttention.h:53-127)
// for T = bf16 or a two-byte half at D = 64, at batch scale.
//
// One workgroup per (split, kv head) over the packer's fixed token splits;
// its four waves take the split's 32-token tiles round-robin, each with the
// next tile's loads in flight while the current one is computed. The tile
// math is the head_dim-128 decode's (mfma_tile.h) at half the dims: S^T =
// K Q^T per 16-token half from two k-groups of 32 dims (C register r of lane
// (c, j) is the score of token j + 4 (4u + r) for query head c), online
// softmax in base 2 with P entering the MFMAs as hi + lo, O^T = V^T P^T.
// Lane (c, j) of V load q holds dims 4c .. 4c + 3 of token 4q + j (8
// contiguous bytes), so PV MFMA n (n < 4) takes element n of each of its
// loads -- row c stands for dim 4c + n -- and C register r of MFMA n in lane
// (c, j) is O[head c][dim 16j + 4r + n]. The GQA group fills the MFMA
// columns, so each K/V byte is read once per group. The four waves merge
// through LDS and write the split's (m, l, O) in the generic workspace
// layout; the generic split merge produces the output.
#include "decode_split16.h"
#include "mfma_tile.h"

namespace qvp {
namespace {

constexpr int kS16Waves = 4;
constexpr int kS16Threads = kS16Waves * 64;
constexpr int kS16D = 64;
constexpr int kS16RowPad = kS16D + 4;  // LDS row of one merged output column (floats)

struct S16Args {
    const int32_t* split_seq;
    const int32_t* split_start;
    uint32_t split_tokens;
    float* ws_ml;   // [num_splits][Hq][2]: running max (base 2), running sum
    float* ws_acc;  // [num_splits][Hq][64]
};

struct S16Tile {
    u32x4 k[2][2];       // [half u][k-group i]: token 16u + (c >> 2) + 4 (c & 3), dims 32i + 8j .. + 7
    uint32_t v[8][2];    // [load q]: token 4q + j, dims 4c .. 4c + 3
};

template <typename T>
__device__ inline const __attribute__((address_space(4))) T* as_const(const T* ptr) {
    return (const __attribute__((address_space(4))) T*)(ptr);
}

template <bool kF16>
__global__ __launch_bounds__(kS16Threads, 2) void decode_split16(DecodeGeometry p, S16Args sa) {
    __shared__ float sm_m[kS16Waves][16];
    __shared__ float sm_l[kS16Waves][16];
    __shared__ float sm_o[kS16Waves][16][kS16RowPad];

    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int c = lane & 15;
    const int j = lane >> 4;
    const int G = static_cast<int>(p.group);
    const int split = static_cast<int>(blockIdx.x / p.num_kv_heads);
    const int g = static_cast<int>(blockIdx.x - split * p.num_kv_heads);
    const int b = as_const(sa.split_seq)[split];
    const int start = as_const(sa.split_start)[split];
    const int ctx = as_const(p.seq_lens)[b];
    const int end = min(start + static_cast<int>(sa.split_tokens), ctx);
    const int ntile = (end - start + kTileTokens - 1) / kTileTokens;
    const auto* row = as_const(p.tables) + static_cast<uint64_t>(b) * p.max_nb;
    const uint32_t tmask = p.tpb - 1;

    // Q operand of lane (c, j): query head g*G + c (columns past the group
    // repeat its last head and are never written), dims 32i + 8j .. + 7.
    u32x4 qop[2];
    {
        const uint16_t* qp = static_cast<const uint16_t*>(p.query) +
                             (static_cast<uint64_t>(b) * p.num_q_heads + g * G + min(c, G - 1)) * kS16D + 8 * j;
#pragma unroll
        for (int i = 0; i < 2; ++i) qop[i] = *reinterpret_cast<const u32x4*>(qp + 32 * i);
    }

    // Tile i holds tokens start + 32i .. + 31; each 16-token half lies in one
    // frame (start is a multiple of 32 and tokens_per_block a power of two >=
    // 16), a half past the split's end reads the last valid token's frame.
    // Tokens past the end read in-frame bytes: their scores are masked and
    // their values zeroed when the tile is computed.
    auto load = [&](int i, S16Tile& t) {
        const int tok0 = start + kTileTokens * i;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int half0 = tok0 + 16 * u;
            const int32_t blk = row[min(half0, end - 1) >> p.tpb_shift];
            const uint8_t* frame = p.kv_base + static_cast<uint64_t>(blk) * p.block_stride +
                                   static_cast<uint64_t>(g) * p.head_stride;
            const int ktok = half0 + (c >> 2) + 4 * (c & 3);
            const uint8_t* kp = frame + p.k_off + static_cast<uint64_t>(ktok & tmask) * p.token_stride + 16u * j;
#pragma unroll
            for (int k = 0; k < 2; ++k) t.k[u][k] = load16(kp + 64 * k);
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
                const int vtok = half0 + 4 * qq + j;
                const uint8_t* vp = frame + p.v_off + static_cast<uint64_t>(vtok & tmask) * p.token_stride + 8u * c;
                const uint2 w = *reinterpret_cast<const uint2*>(vp);
                t.v[4 * u + qq][0] = w.x;
                t.v[4 * u + qq][1] = w.y;
            }
        }
    };

    floatx4 o[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    float l_run = 0.f;

    auto compute = [&](S16Tile& t, int tok0) {
        floatx4 s[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 2; ++k) acc = mfma16<kF16>(t.k[u][k], qop[k], acc);
            s[u] = acc;
        }
        if (tok0 + kTileTokens > end) {
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    if (tok0 + j + 16 * u + 4 * r >= end) s[u][r] = -INFINITY;
                }
        }
        u32x4 bhi, blo;
        float alpha;
        softmax_p<kF16, true>(s, p.scale_log2, m_run, l_run, bhi, blo, alpha);
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int n = 0; n < 4; ++n) o[n] *= alpha;
        }
        // Values of tokens past the split are not data (0 * NaN would poison O).
        if (tok0 + kTileTokens > end) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if (tok0 + 4 * q + j >= end) {
                    t.v[q][0] = 0u;
                    t.v[q][1] = 0u;
                }
            }
        }
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            u32x4 a;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                // Element n of tokens 2k and 2k + 1 of this lane's loads, token
                // 2k in the low half.
                a[k] = __builtin_amdgcn_perm(t.v[2 * k + 1][n >> 1], t.v[2 * k][n >> 1],
                                             (n & 1) ? 0x07060302u : 0x05040100u);
            }
            o[n] = mfma16<kF16>(a, bhi, o[n]);
            o[n] = mfma16<kF16>(a, blo, o[n]);
        }
    };

    S16Tile nxt;
    if (wave < ntile) load(wave, nxt);
    for (int i = wave; i < ntile; i += kS16Waves) {
        S16Tile cur = nxt;
        if (i + kS16Waves < ntile) load(i + kS16Waves, nxt);
        compute(cur, start + kTileTokens * i);
    }

    // Merge the four waves (a wave without tiles has m = -inf, l = 0, O = 0).
    l_run = sum_over_j(l_run);
    if (j == 0) {
        sm_m[wave][c] = m_run;
        sm_l[wave][c] = l_run;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int n = 0; n < 4; ++n) sm_o[wave][c][16 * j + 4 * r + n] = o[n][r];
    __syncthreads();
    const uint64_t head0 = static_cast<uint64_t>(split) * p.num_q_heads + static_cast<uint64_t>(g) * G;
    for (int e = threadIdx.x; e < G * kS16D; e += kS16Threads) {
        const int hc = e >> 6;
        const int dd = e & (kS16D - 1);
        float mmax = sm_m[0][hc];
#pragma unroll
        for (int w = 1; w < kS16Waves; ++w) mmax = fmaxf(mmax, sm_m[w][hc]);
        float acc = 0.f;
        float lsum = 0.f;
#pragma unroll
        for (int w = 0; w < kS16Waves; ++w) {
            const float mw = sm_m[w][hc];
            const float f = mw == -INFINITY ? 0.f : fast_exp2(mw - mmax);
            acc += sm_o[w][hc][dd] * f;
            lsum += sm_l[w][hc] * f;
        }
        sa.ws_acc[(head0 + hc) * kS16D + dd] = acc;
        if (dd == 0) {
            sa.ws_ml[(head0 + hc) * 2 + 0] = mmax;
            sa.ws_ml[(head0 + hc) * 2 + 1] = lsum;
        }
    }
}

}  // namespace

bool split16_supported(const DecodeGeometry& g, uint32_t kv_dtype, uint32_t split_tokens, uintptr_t query_addr) {
    const bool pow2 = g.tpb != 0 && (g.tpb & (g.tpb - 1)) == 0;
    const bool aligned = (g.block_stride % 16 == 0) && (g.k_off % 16 == 0) && (g.v_off % 16 == 0) &&
                         (g.token_stride % 16 == 0) && (g.head_stride % 16 == 0) &&
                         (reinterpret_cast<uintptr_t>(g.kv_base) % 16 == 0) && (query_addr % 16 == 0);
    return (kv_dtype == QVP_DTYPE_BF16 || kv_dtype == QVP_DTYPE_F16) && g.head_dim == kS16D && g.group >= 1 &&
           g.group <= 16 && g.scale_log2 > 0.0f && pow2 && g.tpb >= 16 && split_tokens % kTileTokens == 0 &&
           aligned;
}

int launch_split16_decode(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t kv_dtype, uint32_t out_dtype,
                          void* out, void* workspace, hipEvent_t split_event, hipStream_t stream) {
    const uint64_t heads = static_cast<uint64_t>(v.num_splits) * g.num_q_heads;
    S16Args sa{};
    sa.split_seq = v.split_seq;
    sa.split_start = v.split_start;
    sa.split_tokens = v.split_tokens;
    sa.ws_ml = static_cast<float*>(workspace);
    sa.ws_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + round_up(heads * 2 * sizeof(float), 256));
    const uint64_t groups = static_cast<uint64_t>(v.num_splits) * g.num_kv_heads;
    if (groups > 0x7fffffffu) return fail(QVP_ERR_INVALID_ARGUMENT, "too many (split, kv head) pairs");
    const dim3 grid(static_cast<unsigned>(groups));
    if (kv_dtype == QVP_DTYPE_F16) {
        hipLaunchKernelGGL(decode_split16<true>, grid, dim3(kS16Threads), 0, stream, g, sa);
    } else {
        hipLaunchKernelGGL(decode_split16<false>, grid, dim3(kS16Threads), 0, stream, g, sa);
    }
    QVP_HIP(hipGetLastError());
    if (split_event != nullptr) QVP_HIP(hipEventRecord(split_event, stream));
    return launch_merge_splits(g, v, out_dtype, out, sa.ws_ml, sa.ws_acc, stream);
}

}  // namespace qvp

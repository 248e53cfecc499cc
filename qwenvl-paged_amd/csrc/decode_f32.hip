// fp32 paged decode on the fp32 matrix cores (v_mfma_f32_16x16x4_f32), for
// fp32 caches with head_dim 128 or 64 -- the reference's paged_attention_decode<float>
// (include/qwenvl_paged/PagedAttention.h:53-127) at batch scale.
//
// One workgroup per (split, kv head) over the packer's fixed token splits; its
// four waves take the split's 16-token blocks round-robin, each with the next
// block's loads in flight while the current one is computed. The GQA group
// sits in the MFMA columns (S^T = K Q^T, O^T = V^T P^T), so every K/V byte is
// read once per group, and the contraction index of each MFMA is assigned so
// that every lane reads contiguous bytes: for QK, lane (c, j) contributes dim
// 32j + m of token c at step m (128 contiguous bytes of one K row); for PV,
// lane (c, j) contributes token 4j + s of dims 8c .. 8c + 7 (32 contiguous
// bytes of one V row), and C register s of the QK output of lane (c, j) is
// exactly the weight of token 4j + s, so P feeds PV with no data movement
// (at head_dim 64: dim 16j + m, 64 bytes of K; dims 4c .. 4c + 3, 16 bytes of
// V).
// Weights stay fp32. The four waves merge their online-softmax states through
// LDS and write the split's (m, l, O) in the generic kernel's workspace
// layout; the generic split merge produces the output.
#include "mfma_tile.h"

namespace qvp {
namespace {

constexpr int kF32Waves = 4;
constexpr int kF32Threads = kF32Waves * 64;
constexpr int kF32Block = 16;  // tokens per block (one MFMA row block)

struct F32SplitArgs {
    const int32_t* split_seq;
    const int32_t* split_start;
    uint32_t split_tokens;
    float* ws_ml;   // [num_splits][Hq][2]: running max (base 2), running sum
    float* ws_acc;  // [num_splits][Hq][D]
};

// One 16-token block of K and V for head_dim kD (128 or 64).
template <int kD>
struct F32Tile {
    floatx4 k[kD / 16];     // token c, dims (kD / 4) j + 4m .. +3
    floatx4 v[4][kD / 64];  // token 4j + s, dims (kD / 16) c .. + kD / 16 - 1
};

template <typename T>
__device__ inline const __attribute__((address_space(4))) T* as_const(const T* ptr) {
    return (const __attribute__((address_space(4))) T*)(ptr);
}

// Plain loads: with the non-temporal hint (which speeds up the bf16 decode)
// this kernel ran the config2-shaped fp32 batch in 219 us instead of 136 us.
__device__ inline floatx4 load4f(const uint8_t* ptr) { return *reinterpret_cast<const floatx4*>(ptr); }

// kD = 128: lane (c, j) contributes dim 32j + m of token c at QK step m
// (m < 32) and dims 8c .. 8c + 7 of token 4j + s to PV; kD = 64: dim 16j + m
// (m < 16) and dims 4c .. 4c + 3. PV MFMA n (n < kD / 16) puts dim
// (kD / 16) c + n in row c, so C register r of lane (c, j) is dim
// (kD / 4) j + (kD / 16) r + n of column c.
template <int kD>
__global__ __launch_bounds__(kF32Threads, 2) void decode_f32_grouped(DecodeGeometry p, F32SplitArgs sa) {
    constexpr int kRowPad = kD + 4;  // LDS row of one merged output column (floats)
    constexpr int kK = kD / 16;      // K loads (and query vectors) per lane
    constexpr int kV = kD / 64;      // V loads per lane and token
    __shared__ float sm_m[kF32Waves][16];
    __shared__ float sm_l[kF32Waves][16];
    __shared__ float sm_o[kF32Waves][16][kRowPad];

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
    const int nblk = (end - start + kF32Block - 1) / kF32Block;
    const auto* row = as_const(p.tables) + static_cast<uint64_t>(b) * p.max_nb;
    const uint32_t tmask = p.tpb - 1;

    // Q operand of lane (c, j): query head g*G + c (columns past the group
    // repeat its last head and are never written), dims (kD / 4) j onward.
    floatx4 q[kK];
    {
        const float* qp = static_cast<const float*>(p.query) +
                          (static_cast<uint64_t>(b) * p.num_q_heads + g * G + min(c, G - 1)) * kD + (kD / 4) * j;
#pragma unroll
        for (int m = 0; m < kK; ++m) q[m] = *reinterpret_cast<const floatx4*>(qp + 4 * m);
    }

    // Block i holds tokens start + 16i .. +15, all in one frame (start is a
    // multiple of 16 and tokens_per_block a power of two >= 16). Tokens past
    // the split read in-frame bytes; their scores are masked and their values
    // zeroed when the block is computed.
    auto load = [&](int i, F32Tile<kD>& t) {
        const int tok0 = start + kF32Block * i;
        const int32_t blk = row[tok0 >> p.tpb_shift];
        const uint8_t* frame = p.kv_base + static_cast<uint64_t>(blk) * p.block_stride +
                               static_cast<uint64_t>(g) * p.head_stride;
        const uint8_t* kp = frame + p.k_off + static_cast<uint64_t>((tok0 + c) & tmask) * p.token_stride + kD * j;
#pragma unroll
        for (int m = 0; m < kK; ++m) t.k[m] = load4f(kp + 16 * m);
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint8_t* vp =
                frame + p.v_off + static_cast<uint64_t>((tok0 + 4 * j + s) & tmask) * p.token_stride + (kD / 4) * c;
#pragma unroll
            for (int x = 0; x < kV; ++x) t.v[s][x] = load4f(vp + 16 * x);
        }
    };

    floatx4 o[kK];
#pragma unroll
    for (int n = 0; n < kK; ++n) o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    float l_run = 0.f;

    auto compute = [&](F32Tile<kD>& t, int tok0) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < kD / 4; ++m) {
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(t.k[m >> 2][m & 3], q[m >> 2][m & 3], acc, 0, 0, 0);
        }
        float s[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = (tok0 + 4 * j + r < end) ? acc[r] * p.scale_log2 : -INFINITY;
        float mt = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
        mt = max_over_j(mt);
        const float m_new = fmaxf(m_run, mt);
        const float alpha = fast_exp2(m_run - m_new);
        m_run = m_new;
        float pw[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) pw[r] = fast_exp2(s[r] - m_new);
        l_run = l_run * alpha + ((pw[0] + pw[1]) + (pw[2] + pw[3]));
        if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
            for (int n = 0; n < kK; ++n) o[n] *= alpha;
        }
        // Values of tokens past the split are not data (0 * NaN would poison O).
        if (tok0 + kF32Block > end) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (tok0 + 4 * j + r >= end) {
#pragma unroll
                    for (int x = 0; x < kV; ++x) t.v[r][x] = floatx4{0.f, 0.f, 0.f, 0.f};
                }
            }
        }
#pragma unroll
        for (int n = 0; n < kK; ++n) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(t.v[r][n >> 2][n & 3], pw[r], o[n], 0, 0, 0);
            }
        }
    };

    F32Tile<kD> nxt;
    if (wave < nblk) load(wave, nxt);
    for (int i = wave; i < nblk; i += kF32Waves) {
        F32Tile<kD> cur = nxt;
        if (i + kF32Waves < nblk) load(i + kF32Waves, nxt);
        compute(cur, start + kF32Block * i);
    }

    // Merge the four waves (a wave without blocks has m = -inf, l = 0, O = 0).
    l_run = sum_over_j(l_run);
    if (j == 0) {
        sm_m[wave][c] = m_run;
        sm_l[wave][c] = l_run;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int n = 0; n < kK; ++n) sm_o[wave][c][(kD / 4) * j + (kD / 16) * r + n] = o[n][r];
    __syncthreads();
    const uint64_t head0 = static_cast<uint64_t>(split) * p.num_q_heads + static_cast<uint64_t>(g) * G;
    for (int e = threadIdx.x; e < G * kD; e += kF32Threads) {
        const int hc = e / kD;
        const int dd = e - hc * kD;
        float mmax = sm_m[0][hc];
#pragma unroll
        for (int w = 1; w < kF32Waves; ++w) mmax = fmaxf(mmax, sm_m[w][hc]);
        float acc = 0.f;
        float lsum = 0.f;
#pragma unroll
        for (int w = 0; w < kF32Waves; ++w) {
            const float f = fast_exp2(sm_m[w][hc] - mmax);
            acc += sm_o[w][hc][dd] * f;
            lsum += sm_l[w][hc] * f;
        }
        sa.ws_acc[(head0 + hc) * kD + dd] = acc;
        if (dd == 0) {
            sa.ws_ml[(head0 + hc) * 2 + 0] = mmax;
            sa.ws_ml[(head0 + hc) * 2 + 1] = lsum;
        }
    }
}

}  // namespace

bool f32_grouped_supported(const DecodeGeometry& g, uint32_t kv_dtype, uint32_t split_tokens, uintptr_t query_addr,
                           uintptr_t kv_base_addr) {
    const bool pow2 = g.tpb != 0 && (g.tpb & (g.tpb - 1)) == 0;
    const bool aligned = (g.block_stride % 16 == 0) && (g.k_off % 16 == 0) && (g.v_off % 16 == 0) &&
                         (g.token_stride % 16 == 0) && (g.head_stride % 16 == 0) && (kv_base_addr % 16 == 0) &&
                         (query_addr % 16 == 0);
    return kv_dtype == QVP_DTYPE_F32 && (g.head_dim == 128 || g.head_dim == 64) && g.group >= 1 && g.group <= 16 &&
           pow2 && g.tpb >= 16 && split_tokens % kF32Block == 0 && aligned;
}

int launch_f32_grouped_decode(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t out_dtype, void* out,
                              void* workspace, hipEvent_t split_event, hipStream_t stream) {
    const uint64_t heads = static_cast<uint64_t>(v.num_splits) * g.num_q_heads;
    F32SplitArgs sa{};
    sa.split_seq = v.split_seq;
    sa.split_start = v.split_start;
    sa.split_tokens = v.split_tokens;
    sa.ws_ml = static_cast<float*>(workspace);
    sa.ws_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + round_up(heads * 2 * sizeof(float), 256));
    const uint64_t groups = static_cast<uint64_t>(v.num_splits) * g.num_kv_heads;
    if (groups > 0x7fffffffu) return fail(QVP_ERR_INVALID_ARGUMENT, "too many (split, kv head) pairs");
    if (g.head_dim == 64) {
        hipLaunchKernelGGL(decode_f32_grouped<64>, dim3(static_cast<unsigned>(groups)), dim3(kF32Threads), 0, stream, g,
                           sa);
    } else {
        hipLaunchKernelGGL(decode_f32_grouped<128>, dim3(static_cast<unsigned>(groups)), dim3(kF32Threads), 0, stream,
                           g, sa);
    }
    QVP_HIP(hipGetLastError());
    if (split_event != nullptr) QVP_HIP(hipEventRecord(split_event, stream));
    return launch_merge_splits(g, v, out_dtype, out, sa.ws_ml, sa.ws_acc, stream);
}

}  // namespace qvp

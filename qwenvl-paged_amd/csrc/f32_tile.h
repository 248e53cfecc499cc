// fp32 tiles of the persistent decode (v_mfma_f32_16x16x4_f32), for fp32
// caches with head_dim 128 -- the reference's paged_attention_decode<float>
// (include/qwenvl_paged/PagedAttention.h:53-127).
//
// A 16-token half tile of one kv head is 8 KiB of K and 8 KiB of V, the
// bytes of a bf16 32-token tile, held in the same KvTile registers (16
// 16-byte words per lane); the persistent kernel runs each 32-token schedule
// tile as two halves, one half in flight while the other is computed.
//
// Contraction indices are assigned so every lane reads contiguous bytes and P
// never moves (lane l = (c = l % 16, j = l / 16)):
//   QK: S^T = K Q^T in 32 steps m of 4 dims; at step m lane (c, j) gives dim
//       32j + m of token c (K words 0..7: 128 contiguous bytes of token c's
//       row) and the same dim of query head c. C register r of lane (c, j)
//       is the score of token 4j + r for head c.
//   PV: O^T = V^T P^T in 32 MFMAs (8 dim blocks n x 4 token steps r); lane
//       (c, j) gives V[token 4j + r][dim 8c + n] (V words 8 + 2r, 9 + 2r: 32
//       contiguous bytes of token 4j + r's row) and its own weight of that
//       token. C register r' of PV MFMA n in lane (c, j) is O[head c][dim 32j
//       + 8r' + n] -- the layout of the bf16 tiles' accumulators, so the
//       kernel's merges are shared.
// Weights stay fp32 (no hi/lo split).
#pragma once

#include "mfma_tile.h"

namespace qvp {

// K word m (m = 0..7): dims 32j + 4m .. +3 of token c; V words 8 + 2s + h: dims
// 8c + 4h .. +3 of token 4j + s.
__device__ inline floatx4 f32_word(const KvTile& t, int w) {
    const u32x4 v = w < 8 ? t.k[w >> 2][w & 3] : t.v[w - 8];
    return __builtin_bit_cast(floatx4, v);
}

__device__ inline u32x4 load16_plain(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }

// Issues the 16 loads of half `half` (tokens 32 t + 16 half .. +15) of tile r.
// Tokens past the context read in-frame bytes of the last valid block (the
// tile's frames are resolved that way); the compute masks them.
__device__ inline void load_half_f32(const uint8_t* kv_base, uint64_t block_stride, uint64_t head_stride,
                                     uint64_t k_off, uint64_t v_off, uint64_t token_stride, uint32_t tpb, int g,
                                     int blk, int tok0, int c, int j, KvTile& tile) {
    const uint32_t tmask = tpb - 1;
    const uint8_t* frame = kv_base + static_cast<uint64_t>(g) * head_stride + static_cast<uint64_t>(blk) * block_stride;
    const uint8_t* kp = frame + k_off + static_cast<uint64_t>((tok0 + c) & tmask) * token_stride + 128u * j;
#pragma unroll
    for (int m = 0; m < 8; ++m) tile.k[m >> 2][m & 3] = load16_plain(kp + 16 * m);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const uint8_t* vp = frame + v_off + static_cast<uint64_t>((tok0 + 4 * j + s) & tmask) * token_stride + 32u * c;
        tile.v[2 * s] = load16_plain(vp);
        tile.v[2 * s + 1] = load16_plain(vp + 16);
    }
}

// One 16-token half tile of online softmax + PV (scale > 0: the running
// maximum is taken on raw scores, as in the 16-bit tiles). Column c sees
// tokens t <= col_last; values of tokens at or past v_end are zeroed in place
// (not data: 0 * NaN would poison O). q holds query words 0..7 of lane (c, j):
// dims 32j + 4i .. +3 of head c.
__device__ inline void compute_half_f32(KvTile& cur, const u32x4 (&q)[8], int tok0, int col_last, int v_end,
                                        float scale_log2, int j, float& m_run, float& l_run, floatx4 (&o)[8]) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 32; ++m) {
        const floatx4 qw = __builtin_bit_cast(floatx4, q[m >> 2]);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(f32_word(cur, m >> 2)[m & 3], qw[m & 3], acc, 0, 0, 0);
    }
    // The mask is applied without a branch. Behind `if (tok0 + 15 >
    // col_last)` the compiler put the first read of the scores at the branch
    // target with no wait states on the taken (unmasked) path after the last
    // MFMA, so that read could see the previous contents of the result
    // registers: the running maximum then varied between launches (the state
    // stayed equivalent, the bits did not), and stale bits far from the scores
    // would have broken the weights.
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = tok0 + 4 * j + r > col_last ? -INFINITY : acc[r];
    float mt = fmaxf(fmaxf(acc[0], acc[1]), fmaxf(acc[2], acc[3]));
    mt = max_over_j(mt) * scale_log2;
    const float m_new = fmaxf(m_run, mt);
    const float alpha = fast_exp2(m_run - m_new);
    m_run = m_new;
    float pw[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) pw[r] = fast_exp2(fmaf(acc[r], scale_log2, -m_new));
    l_run = l_run * alpha + ((pw[0] + pw[1]) + (pw[2] + pw[3]));
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int n = 0; n < 8; ++n) o[n] *= alpha;
    }
    if (tok0 + 16 > v_end) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (tok0 + 4 * j + r >= v_end) {
                cur.v[2 * r] = u32x4{0u, 0u, 0u, 0u};
                cur.v[2 * r + 1] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            o[n] = __builtin_amdgcn_mfma_f32_16x16x4f32(f32_word(cur, 8 + 2 * r + (n >> 2))[n & 3], pw[r], o[n], 0, 0,
                                                        0);
        }
    }
}

}  // namespace qvp

// Vector-ALU tile math of the persistent bf16 decode: the same 32-token tile
// registers as the matrix-core path (KvTile, loaded by the same code), the
// GQA group folded into each lane's dot products instead of the MFMA columns.
//
// Lane l = (c = l % 16, j = l / 16). K: lane (c, j) of half u holds dims
// 32i + 8j .. 32i + 8j + 7 (i = 0..3) of token kt = 16u + (c >> 2) + 4 (c & 3).
// It multiplies them with every head's query (kVG heads, fp32 in LDS as
// [dim][head]) and the four j lanes of a token add their partial dots, so
// every lane ends with the token's score for every head. The tile's running
// max per head is reduced over the 16 lanes c (DPP butterflies inside a row;
// the j rows agree), the weights go to a wave-private LDS row per token, and
// PV runs on the V registers as loaded: lane (c, j) of load q holds dims
// 8c .. 8c + 7 of token 4q + j, so it accumulates those 8 dims of every head
// over its 8 tokens; the four j lanes' partial outputs are added when the
// piece ends. Weights stay fp32 (no bf16 split): the arithmetic is plain fp32
// FMA on bf16-exact inputs.
#pragma once

#include "mfma_tile.h"

namespace qvp {

// The query group is padded to the bound 1 or 2 of the instantiation
// (kVectorTileMaxGroup); a padded head repeats the last one and is never
// written. Wider groups would hold 8 accumulators per head per lane beside
// the two tiles in flight: past two heads the kernel spills registers.

// LDS of the vector tiles, per workgroup: the queries of up to four kv heads
// side by side and one weight row per token for each wave.
template <int kVG>
struct VectorTileLds {
    float q[4][128][kVG];
    float p[8][kTileTokens][kVG];
};
template <>
struct VectorTileLds<0> {};

constexpr uint32_t vector_tile_lds_bytes(int vg) {
    return vg == 0 ? 0u : static_cast<uint32_t>((4 * 128 + 8 * kTileTokens) * vg * sizeof(float));
}

template <int kCtrl>
__device__ inline float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

// Max / sum over the 16 lanes of a row (lane bits 0..3): quad swaps, then the
// half-row and row mirrors.
__device__ inline float max_over_c(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    return fmaxf(v, dpp_f<0x140>(v));
}

__device__ inline float sum_over_c(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    return v + dpp_f<0x140>(v);
}

// Writes the piece's query (the MFMA B operand registers: lane (c, j) holds
// head c's dims 32i + 8j .. +7) into q[dim][head] for heads c < kVG.
template <int kVG>
__device__ inline void stage_query(float (*q)[kVG], const u32x4 (&qop)[4], int c, int j) {
    if (c >= kVG) return;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const int d = 32 * i + 8 * j + 2 * w;
            q[d][c] = __uint_as_float(qop[i][w] << 16);
            q[d + 1][c] = __uint_as_float(qop[i][w] & 0xffff0000u);
        }
}

// One tile of online softmax + PV on the vector ALUs for heads 0..kVG-1.
// m_run: running max (base 2) per head, uniform over the wave; l_part: this
// lane's share of the running sum (its two tokens, the same in the four j
// lanes); o[h][e]: this lane's share of O[h][8c + e] (its eight tokens).
template <int kVG>
__device__ inline void compute_tile_vector(KvTile& cur, const float (*q)[kVG], float (*pw)[kVG], int tok0,
                                           int col_last, int v_end, float scale_log2, int c, int j,
                                           float (&m_run)[kVG], float (&l_part)[kVG], float (&o)[kVG][8]) {
    float s[2][kVG];
    // The previous tile's weight reads stay above this tile's writes.
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int h = 0; h < kVG; ++h) s[u][h] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const int d = 32 * i + 8 * j + 2 * w;
                const float k0 = __uint_as_float(cur.k[u][i][w] << 16);
                const float k1 = __uint_as_float(cur.k[u][i][w] & 0xffff0000u);
#pragma unroll
                for (int h = 0; h < kVG; ++h) s[u][h] = fmaf(k0, q[d][h], fmaf(k1, q[d + 1][h], s[u][h]));
            }
        }
#pragma unroll
        for (int h = 0; h < kVG; ++h) s[u][h] = sum_over_j(s[u][h]);
    }

    const int kt = (c >> 2) + 4 * (c & 3);
    float alpha[kVG];
#pragma unroll
    for (int h = 0; h < kVG; ++h) {
        const float a0 = tok0 + kt <= col_last ? s[0][h] * scale_log2 : -INFINITY;
        const float a1 = tok0 + 16 + kt <= col_last ? s[1][h] * scale_log2 : -INFINITY;
        const float m_new = fmaxf(m_run[h], max_over_c(fmaxf(a0, a1)));
        alpha[h] = fast_exp2(m_run[h] - m_new);
        m_run[h] = m_new;
        const float p0 = fast_exp2(a0 - m_new);
        const float p1 = fast_exp2(a1 - m_new);
        l_part[h] = l_part[h] * alpha[h] + p0 + p1;
        if (j == 0) {
            pw[kt][h] = p0;
            pw[16 + kt][h] = p1;
        }
    }
    // Keeps the compiler from moving the weight reads below above the writes
    // of other lanes (it emits no instruction).
    __builtin_amdgcn_wave_barrier();

#pragma unroll
    for (int h = 0; h < kVG; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[h][e] *= alpha[h];
    if (tok0 + kTileTokens > v_end) {
#pragma unroll
        for (int qq = 0; qq < 8; ++qq) {
            if (tok0 + 4 * qq + j >= v_end) cur.v[qq] = u32x4{0u, 0u, 0u, 0u};
        }
    }
    // The weights were written by this wave's j == 0 lanes just above; LDS
    // operations of one wave complete in order, so the reads see them.
#pragma unroll
    for (int qq = 0; qq < 8; ++qq) {
        const int t = 4 * qq + j;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const float v0 = __uint_as_float(cur.v[qq][w] << 16);
            const float v1 = __uint_as_float(cur.v[qq][w] & 0xffff0000u);
#pragma unroll
            for (int h = 0; h < kVG; ++h) {
                o[h][2 * w] = fmaf(pw[t][h], v0, o[h][2 * w]);
                o[h][2 * w + 1] = fmaf(pw[t][h], v1, o[h][2 * w + 1]);
            }
        }
    }
}

}  // namespace qvp

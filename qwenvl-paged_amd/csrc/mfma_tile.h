// MFMA tile math shared by the paged decode and the paged prefill (bf16 K/V,
// head_dim 128, v_mfma_f32_16x16x32_bf16; lane l = (c = l % 16, j = l / 16)).
//
// One tile is 32 tokens of one kv head against 16 query columns (the query
// heads of a group in the decode, 16 query positions of one head in the
// prefill). S^T = K Q^T is computed per 16-token half u: row r of half u
// carries token (r / 4) + 16u + 4 (r % 4), so C register r of lane (c, j) is
// the score of token j + 4 (4u + r) for column c. PV is O^T = V^T P^T with V
// loaded coalesced (lane (c, j) of load q holds dims 8c .. 8c + 7 of token
// 4q + j) and transposed in registers; P enters the bf16 MFMA as hi + lo
// (hi = P truncated to bf16, lo = P - hi rounded to bf16), which keeps the
// weights at about 2^-16 relative error. C register r of PV MFMA n in lane
// (c, j) is O[column c][dim 32j + 8r + n].
#pragma once

#include "decode_common.h"

namespace qvp {

constexpr int kTileTokens = 32;
static_assert(kTileTokens == static_cast<int>(kScheduleTileTokens), "schedule and tiles count the same tokens");

struct KvTile {
    u32x4 k[2][4];  // [half u][QK mfma i]
    u32x4 v[8];     // [load q]
};

__device__ inline u32x4 load16(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }
// A decode reads every K/V byte exactly once: its tile loads carry the
// non-temporal hint (global_load_dwordx4 ... nt), so the lines stream through
// the caches instead of being kept. On the Qwen2-VL-7B batch this took the
// persistent decode from 57.4 to 52.9 us (the same bits), on the 72B batch
// from 471.7 to 440.5 us.
__device__ inline u32x4 load16_stream(const uint8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Reductions over the four lanes (c, 0..3) of one query head: lanes l, l^16,
// l^32, l^48, through the gfx950 row/half swaps (VALU only, so they never wait
// on LDS or scalar-memory counters).
__device__ inline float max_over_j(float v) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ inline float sum_over_j(float v) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(h[0]) + __uint_as_float(h[1]);
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Workgroup barrier that orders LDS only: outstanding global loads (the next
// tile) stay in flight across it.
__device__ inline void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Pieces of the tile step for callers that stage K and V themselves (the
// prefill reads V already transposed from LDS and runs several query tiles
// per K/V tile).

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// 16x16x32 MFMA over the cache's 16-bit element type: bf16, or (kF16) IEEE
// binary16. Operands are eight elements per lane, passed as raw dwords.
template <bool kF16>
__device__ inline floatx4 mfma16(const u32x4& a, const u32x4& b, floatx4 c) {
    if constexpr (kF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                      0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                       c, 0, 0, 0);
    }
}

// S^T of one tile per 16-token half u (C layout as above).
template <bool kF16 = false>
__device__ inline void qk_tile(const u32x4 (&k)[2][4], const u32x4 (&qop)[4], floatx4 (&acc)[2]) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        floatx4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) a = mfma16<kF16>(k[u][i], qop[i], a);
        acc[u] = a;
    }
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// fp16 weights carry a factor 2^15 (folded into the exponent of exp2): P
// then spans (0, 32768] instead of (0, 1], so small weights stay normal
// binary16 numbers and hi + lo keeps ~22 significant bits. The running sum
// carries the same factor, so O / l -- and every merge, which combines (m, l,
// O) of equal scale -- is unchanged.
constexpr float kF16WeightLog2 = 15.0f;

// Largest score of one tile for column c of this lane (raw, before scaling).
__device__ inline float tile_max(const floatx4 (&s)[2]) {
    const float mt = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                           fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    return max_over_j(mt);
}

// Weights of one tile against the maximum m_use (scaled base-2 units): P as
// the hi and lo B operands of the PV MFMAs (see softmax_p); returns this
// lane's sum of its eight weights.
template <bool kF16 = false>
__device__ inline float tile_weights(const floatx4 (&s)[2], float scale_log2, float m_use, u32x4& bhi, u32x4& blo) {
    float psum = 0.f;
    uint32_t phi[4], plo[4];
    const float bias = kF16 ? kF16WeightLog2 - m_use : -m_use;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
#pragma unroll
        for (int r = 0; r < 4; r += 2) {
            const float p0 = fast_exp2(fmaf(s[u][r], scale_log2, bias));
            const float p1 = fast_exp2(fmaf(s[u][r + 1], scale_log2, bias));
            psum += p0 + p1;
            if constexpr (kF16) {
                const f16x2_t hi = {static_cast<_Float16>(p0), static_cast<_Float16>(p1)};
                const f16x2_t lo = {static_cast<_Float16>(p0 - static_cast<float>(hi[0])),
                                    static_cast<_Float16>(p1 - static_cast<float>(hi[1]))};
                phi[2 * u + r / 2] = __builtin_bit_cast(uint32_t, hi);
                plo[2 * u + r / 2] = __builtin_bit_cast(uint32_t, lo);
            } else {
                const uint32_t b0 = __float_as_uint(p0);
                const uint32_t b1 = __float_as_uint(p1);
                const bf16x2_t lo = {static_cast<__bf16>(p0 - __uint_as_float(b0 & 0xffff0000u)),
                                     static_cast<__bf16>(p1 - __uint_as_float(b1 & 0xffff0000u))};
                // High halves of p0 (low word) and p1 (high word) in one byte permute.
                phi[2 * u + r / 2] = __builtin_amdgcn_perm(b1, b0, 0x07060302u);
                plo[2 * u + r / 2] = __builtin_bit_cast(uint32_t, lo);
            }
        }
    }
    bhi = u32x4{phi[0], phi[1], phi[2], phi[3]};
    blo = u32x4{plo[0], plo[1], plo[2], plo[3]};
    return psum;
}

// Online-softmax step of one tile for column c of this lane. The running
// maximum m is kept in scaled base-2 units, so with scale_log2 > 0 the
// maximum is taken on the raw scores and each weight is one fma and one exp2.
// l is rescaled here; O must be scaled by the returned alpha by the caller
// (alpha is exactly 1 when no column's maximum moved). P is returned as the
// hi and lo B operands of the PV MFMAs: for bf16, hi = P truncated to bf16 and
// lo = P - hi rounded to nearest even; for fp16 (weights scaled by 2^15, see
// kF16WeightLog2) hi = P and lo = P - hi, each rounded to nearest even.
// kGuard: a column may have seen no token yet after this tile (running
// maximum still -inf); its weights and alpha are then 0 instead of
// exp2(-inf - -inf).
// kLazy: the running maximum moves only when the tile's maximum exceeds it by
// more than kLazyMaxLog2, so weights stay below 2^kLazyMaxLog2 and O is
// rescaled on few tiles (alpha is exactly 1 otherwise). O / l is unchanged:
// O and l always carry the same factor. Every column must have seen a token
// (the causal prefill's tile 0 holds token 0 for every position).
constexpr float kLazyMaxLog2 = 8.0f;

template <bool kF16 = false, bool kGuard = false, bool kLazy = false>
__device__ inline void softmax_p(const floatx4 (&s)[2], float scale_log2, float& m_run, float& l_run, u32x4& bhi,
                                 u32x4& blo, float& alpha) {
    const float mt = tile_max(s) * scale_log2;
    const float m_new = kLazy ? (mt > m_run + kLazyMaxLog2 ? mt : m_run) : fmaxf(m_run, mt);
    const float m_use = kGuard && m_new == -INFINITY ? 0.f : m_new;
    alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    const float psum = tile_weights<kF16>(s, scale_log2, m_use, bhi, blo);
    l_run = l_run * alpha + psum;
}

// O^T += V^T P^T for one tile: `a` holds V^T operands (lane (c, j) of MFMA n:
// the caller's dim for row c of block n, the tile's tokens in the P operand's
// k order); C register r of MFMA n in lane (c, j) is O[column c][that block's
// row 4j + r].
template <bool kF16 = false>
__device__ inline void pv_tile(const u32x4 (&a)[8], const u32x4& bhi, const u32x4& blo, floatx4 (&o)[8]) {
#pragma unroll
    for (int n = 0; n < 8; ++n) {
        o[n] = mfma16<kF16>(a[n], bhi, o[n]);
        o[n] = mfma16<kF16>(a[n], blo, o[n]);
    }
}

// One tile of online softmax + PV for the wave (scale > 0: the running
// maximum is taken on the raw scores, see softmax_p). Column c (this lane's
// c) sees tokens t <= col_last; only a tile that reaches past col_last takes
// the mask. Values of tokens at or past v_end are zeroed in place (their
// weights are 0, but the bytes read for them are not data and 0 * NaN would
// poison O); only the last tile of a sequence has such tokens. O is rescaled
// only when some column's maximum moved. V's A operands come from the loaded
// rows by byte permutes: lane (c, j) holds dims 8c .. 8c + 7 of tokens
// 4q + j, and PV MFMA n takes element n of each, two tokens per dword.
// kMasked: col_last differs between columns and may be below the tile (a
// sequence's private tile run beside other sequences' columns): the mask is
// applied without a branch and a column that has seen no token keeps weight 0.
template <bool kF16 = false, bool kMasked = false>
__device__ inline void compute_tile(KvTile& cur, const u32x4 (&qop)[4], int tok0, int col_last, int v_end,
                                    float scale_log2, int j, float& m_run, float& l_run, floatx4 (&o)[8]) {
    floatx4 s[2];
    qk_tile<kF16>(cur.k, qop, s);
    if constexpr (kMasked) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) s[u][r] = tok0 + j + 16 * u + 4 * r > col_last ? -INFINITY : s[u][r];
    } else if (tok0 + kTileTokens - 1 > col_last) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (tok0 + j + 16 * u + 4 * r > col_last) s[u][r] = -INFINITY;
            }
    }
    u32x4 bhi, blo;
    float alpha;
    softmax_p<kF16, kMasked>(s, scale_log2, m_run, l_run, bhi, blo, alpha);
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int n = 0; n < 8; ++n) o[n] *= alpha;
    }
    if (tok0 + kTileTokens > v_end) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            if (tok0 + 4 * q + j >= v_end) cur.v[q] = u32x4{0u, 0u, 0u, 0u};
        }
    }
#pragma unroll
    for (int n = 0; n < 8; ++n) {
        const int w = n >> 1;
        u32x4 a;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // Element n of tokens 2k and 2k + 1 of this lane's loads: their
            // low halves (n even) or high halves (n odd), token 2k low.
            a[k] = __builtin_amdgcn_perm(cur.v[2 * k + 1][w], cur.v[2 * k][w], (n & 1) ? 0x07060302u : 0x05040100u);
        }
        o[n] = mfma16<kF16>(a, bhi, o[n]);
        o[n] = mfma16<kF16>(a, blo, o[n]);
    }
}

}  // namespace qvp

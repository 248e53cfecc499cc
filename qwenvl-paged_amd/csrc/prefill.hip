// qvp_paged_prefill: causal attention of a step's new tokens over the paged
// cache. The reference defines prefill as paged_attention_decode<T> applied per
// prompt position p with context_len = p + 1 (include/qwenvl_paged/
// PagedAttention.h:43-44; tests/EndToEnd.test.cpp:252-256), so every output
// row here is the decode of its position.
//
// MFMA path (bf16 cache, head_dim 128, GQA group <= 16, power-of-two
// tokens_per_block >= 16). A work item is (sequence b, kv head g, 16 new
// positions p0 .. p0 + 15, up to 8 query heads of g's group). Its workgroup
// streams tokens [0, p0 + 16) of kv head g in 32-token tiles: each tile is
// loaded once, from HBM straight into LDS, one tile of compute ahead of its
// use, into a double buffer holding the K and V rows as in the frame (16-byte
// chunks XOR-permuted by row so the fragment reads spread over the banks; the
// PV operands come out of V transposed by ds_read_b64_tr_b16), and every wave
// runs the tile math of mfma_tile.h for its two query heads with the 16
// positions in the MFMA columns, column c
// seeing tokens t <= p0 + c (masks only on tiles that reach p0). The tile
// loop is software-pipelined: PV of tile t runs beside QK and the softmax of
// tile t + 1. A wave therefore covers the whole causal context of its
// queries: no split, no merge. Items are launched longest context first so
// the short ones fill the tail. Each K/V tile feeds 16 positions x up to 8
// heads from LDS.
//
// Decode path (any other shape): one virtual sequence per new position (same
// frames, context p + 1), packed into a private batch and run through
// qvp_paged_decode, whose query and output rows are exactly the prefill's.
#include "mfma_tile.h"

#include <algorithm>
#include <climits>
#include <type_traits>
#include <cstring>
#include <vector>

namespace qvp {
namespace {

constexpr int kPrefillWaves = 4;
constexpr int kPrefillThreads = kPrefillWaves * 64;
constexpr int kPrefillPositions = 16;     // MFMA columns
constexpr int kPrefillHeadsPerItem = 8;   // two query heads per wave
constexpr int kHeadBytes = 256;           // 128 bf16
// Block ids per virtual batch of the decode-kernel path.
constexpr size_t kMaxVirtualIds = size_t{1} << 20;

// One K/V tile in LDS: K and V rows as in the frame (token-major). PV MFMA n
// takes dims 16n .. 16n + 15 as its rows; lane (c, j) needs V[4i + j][16n + c]
// for i = 0 .. 7 (the k order of the P operand). ds_read_b64_tr_b16 hands lane
// c of each 16-lane group element c % 4 of the 8 bytes that lane 4e + c / 4
// of the group addressed, as element e: so lane (c, j) addresses dims
// 16n + 4 (c % 4) .. + 3 of token 4 (c / 4 + 4h) + j, and two such reads
// (h = 0, 1) give its eight operand elements.
struct PrefillTile {
    uint8_t k[kTileTokens][kHeadBytes];
    uint8_t v[kTileTokens][kHeadBytes];
};
// Byte of (row, logical byte) in a swizzled 256-byte row: 16-byte chunk x at x ^ (row % 16).
__device__ inline uint32_t swz(int row, int byte) {
    return 16u * static_cast<uint32_t>((byte >> 4) ^ (row & 15)) + static_cast<uint32_t>(byte & 15);
}

struct PrefillItem {
    int32_t b;     // sequence
    int32_t g;     // kv head
    int32_t p0;    // first position of the block
    int32_t np;    // positions in the block, 1 .. 16
    int32_t row0;  // query / output row of p0
    int32_t h0;    // first query head of the group handled by the item
};
static_assert(sizeof(PrefillItem) == 6 * sizeof(int32_t), "PrefillItem is six int32");

template <typename T>
__device__ inline const __attribute__((address_space(4))) T* as_const(const T* ptr) {
    return (const __attribute__((address_space(4))) T*)(ptr);
}

__device__ inline u32x4 lds16(const uint8_t* p) { return *reinterpret_cast<const u32x4*>(p); }
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef uint32_t uint2v __attribute__((ext_vector_type(2)));

template <typename OutT>
__global__ __launch_bounds__(kPrefillThreads, 2) void prefill_mfma(DecodeGeometry p, const PrefillItem* items,
                                                                    void* out_ptr) {
    __shared__ __attribute__((aligned(16))) PrefillTile sm[2];

    const auto* itp = as_const(items) + blockIdx.x;
    const int b = itp->b;
    const int g = itp->g;
    const int p0 = itp->p0;
    const int np = itp->np;
    const int row0 = itp->row0;
    const int h0 = itp->h0;

    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int c = lane & 15;
    const int j = lane >> 4;
    const int G = static_cast<int>(p.group);
    const int nh = min(G - h0, kPrefillHeadsPerItem);
    // This wave's query heads (within the group): h0 + wave and h0 + wave + 4.
    const bool has_a = wave < nh;
    const bool has_b = wave + kPrefillWaves < nh;
    const int ctx_end = p0 + np;
    const int ntiles = (ctx_end + kTileTokens - 1) / kTileTokens;

    // Column c is position p0 + c; columns past the block repeat its last
    // position (valid data, never written).
    const int cc = min(c, np - 1);
    const int col_last = p0 + cc;
    const uint16_t* qrow = static_cast<const uint16_t*>(p.query) +
                           (static_cast<uint64_t>(row0 + cc) * p.num_q_heads + static_cast<uint64_t>(g) * G) * 128;
    u32x4 qa[4], qb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        qa[i] = *reinterpret_cast<const u32x4*>(qrow + (h0 + min(wave, nh - 1)) * 128 + 32 * i + 8 * j);
        qb[i] = *reinterpret_cast<const u32x4*>(qrow + (h0 + min(wave + kPrefillWaves, nh - 1)) * 128 + 32 * i + 8 * j);
    }
    floatx4 oa[8], ob[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) {
        oa[n] = floatx4{0.f, 0.f, 0.f, 0.f};
        ob[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    float ma = -INFINITY, la = 0.f, mb = -INFINITY, lb = 0.f;

    // Tile loads go from HBM straight into LDS (global_load_lds_dwordx4): one
    // instruction fills four rows (1 KiB), lane l landing at byte 16 l of them
    // -- row r0 + l / 16, physical chunk l % 16, which holds logical chunk
    // (l % 16) ^ (row % 16). A tile's two 16-token halves lie in one block each
    // (tokens_per_block is a power of two >= 16); a half past the context's
    // last block reads that block, and rows past the context load the
    // context's last token (finite data under weights of 0), so every address
    // stays inside a mapped frame. With an odd group the last wave holds one
    // head and issues all sixteen loads of a tile (K and V, rows 0 .. 31),
    // leaving the two-head waves none to issue or wait for; otherwise wave w
    // loads rows 8w .. 8w + 7.
    const auto* trow = as_const(p.tables) + static_cast<uint64_t>(b) * p.max_nb;
    const int last_tok = ctx_end - 1;
    const int last_blk = last_tok >> p.tpb_shift;
    const uint8_t* kbase = p.kv_base + p.k_off;
    const uint8_t* vbase = p.kv_base + p.v_off;
    const bool one_loader = nh == kPrefillHeadsPerItem - 1;
    auto load_rows = [&](int buf, int tile, int r0) {
        const int row = r0 + (lane >> 4);
        const int tok = min(tile * kTileTokens + row, last_tok);
        const int half_tok0 = tile * kTileTokens + (r0 & 16);
        const uint64_t off = static_cast<uint64_t>(trow[min(half_tok0 >> p.tpb_shift, last_blk)]) * p.block_stride +
                             static_cast<uint64_t>(g) * p.head_stride +
                             static_cast<uint64_t>(tok & (p.tpb - 1)) * p.token_stride +
                             16u * static_cast<uint32_t>((lane & 15) ^ (row & 15));
        __builtin_amdgcn_global_load_lds(kbase + off, (__attribute__((address_space(3))) void*)(&sm[buf].k[r0][0]), 16,
                                         0, 0);
        __builtin_amdgcn_global_load_lds(vbase + off, (__attribute__((address_space(3))) void*)(&sm[buf].v[r0][0]), 16,
                                         0, 0);
    };
    auto load_tile_lds = [&](int buf, int tile) {
        if (one_loader) {
            if (wave == kPrefillWaves - 1) {
#pragma unroll
                for (int q = 0; q < 8; ++q) load_rows(buf, tile, 4 * q);
            }
        } else {
#pragma unroll
            for (int q = 0; q < 2; ++q) load_rows(buf, tile, 8 * wave + 4 * q);
        }
    };

    auto read_k = [&](int buf, u32x4 (&kf)[2][4]) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * u + (c >> 2) + 4 * (c & 3);
                kf[u][i] = lds16(&sm[buf].k[row][swz(row, 16 * j + 64 * i)]);
            }
    };
    auto read_v = [&](int buf, u32x4 (&vf)[8]) {
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            u32x4 a;
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const int row = 4 * ((c >> 2) + 4 * hh) + j;
                const v4i16 t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (v4i16 __attribute__((address_space(3)))*)(&sm[buf].v[row][swz(row, 2 * (16 * n + 4 * (c & 3)))]));
                a[2 * hh] = __builtin_bit_cast(uint2v, t)[0];
                a[2 * hh + 1] = __builtin_bit_cast(uint2v, t)[1];
            }
            vf[n] = a;
        }
    };
    // Causal mask of tile t for both heads: column c sees tokens <= col_last.
    auto mask2 = [&](floatx4 (&sa)[2], floatx4 (&sb)[2], int t) {
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool out = t * kTileTokens + j + 16 * u + 4 * r > col_last;
                sa[u][r] = out ? -INFINITY : sa[u][r];
                sb[u][r] = out ? -INFINITY : sb[u][r];
            }
    };

    // Software pipeline over tiles. Iteration t issues PV(t) (P and V of tile
    // t already in registers) in one basic block with QK and the softmax of
    // tile t + 1, which do not depend on it, so the MFMAs of one overlap the
    // VALU work of the other; tile t + 2 is loaded into the LDS buffer tile t
    // used, and every wave waits for its loads before the iteration's closing
    // barrier. Tiles from t_diag on reach the block's first
    // position and take the causal mask; the loop is split there so the
    // others carry no mask code. A wave with two query heads runs both in one
    // block; a wave with one (the last wave of an odd group) runs a
    // one-head copy of the loop, leaving its SIMD's issue slots to the
    // other workgroup's wave there.
    const int t_diag = (p0 + 1) / kTileTokens;
    const int last_tile = ntiles - 1;
    auto run = [&](auto two_heads) {
        constexpr bool kTwo = decltype(two_heads)::value;
        u32x4 kf[2][4], vf[8];
        floatx4 sa[2], sb[2];
        u32x4 ahi, alo, bhi, blo;
        float alpha_a, alpha_b = 1.0f;
        // A direct load has landed in LDS once vmcnt counts it done: each wave
        // waits for all of its loads (s_waitcnt 0) before the barrier that
        // hands the tile to the other waves.
        load_tile_lds(0, 0);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (last_tile >= 1) load_tile_lds(1, 1);
        read_k(0, kf);
        read_v(0, vf);
        qk_tile(kf, qa, sa);
        if constexpr (kTwo) qk_tile(kf, qb, sb);
        if (t_diag == 0) mask2(sa, sb, 0);
        softmax_p<false, false, true>(sa, p.scale_log2, ma, la, ahi, alo, alpha_a);
        if constexpr (kTwo) softmax_p<false, false, true>(sb, p.scale_log2, mb, lb, bhi, blo, alpha_b);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        // O is rescaled for tile t's maximum just before PV(t) accumulates
        // into it, skipped when no column's maximum moved (the factor is then
        // exactly 1); the branch sits at the top of the iteration, outside
        // the block above. The maximum moves lazily (softmax_p's kLazy: only
        // past kLazyMaxLog2 above the current one), so after the first tiles
        // almost no iteration rescales.
        auto rescale = [&]() {
            if (__builtin_amdgcn_ballot_w64(alpha_a != 1.0f || alpha_b != 1.0f) != 0) {
#pragma unroll
                for (int n = 0; n < 8; ++n) {
                    oa[n] *= alpha_a;
                    if constexpr (kTwo) ob[n] *= alpha_b;
                }
            }
        };
        auto step = [&](int t, auto masked) {
            const int nb = (t + 1) & 1;
            rescale();
            // Tile t + 2; near the end the last tile again, which lands in a
            // buffer no later iteration reads.
            // Tile t + 2 into the buffer tile t used (read at iteration t - 1).
            if (t + 2 <= last_tile) load_tile_lds(t & 1, t + 2);
            read_k(nb, kf);
            qk_tile(kf, qa, sa);
            if constexpr (kTwo) qk_tile(kf, qb, sb);
            pv_tile(vf, ahi, alo, oa);
            if constexpr (kTwo) pv_tile(vf, bhi, blo, ob);
            read_v(nb, vf);
            if constexpr (decltype(masked)::value) mask2(sa, sb, t + 1);
            softmax_p<false, false, true>(sa, p.scale_log2, ma, la, ahi, alo, alpha_a);
            if constexpr (kTwo) softmax_p<false, false, true>(sb, p.scale_log2, mb, lb, bhi, blo, alpha_b);
            // Schedule: the QK MFMAs first, then the PV MFMAs spread over the
            // softmax's VALU work.
            constexpr int kHeads = kTwo ? 2 : 1;
#pragma unroll
            for (int k = 0; k < 8 * kHeads; ++k) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
            for (int k = 0; k < 16 * kHeads; ++k) {
                __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            }
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        };
        int t = 0;
        for (; t + 1 < min(t_diag, ntiles); ++t) step(t, std::false_type{});
        for (; t + 1 < ntiles; ++t) step(t, std::true_type{});
        rescale();
        pv_tile(vf, ahi, alo, oa);
        if constexpr (kTwo) pv_tile(vf, bhi, blo, ob);
    };
    if (has_b) {
        run(std::true_type{});
    } else {
        run(std::false_type{});
    }

    OutT* out = static_cast<OutT*>(out_ptr);
    // C register r of PV MFMA n in lane (c, j) is O[column c][dim 16n + 4j +
    // r]: four contiguous outputs per n, stored as one vector, so a store
    // instruction writes 16 contiguous dims (4 lanes) of each of its 16 rows
    // (one 2-byte store per element took a fifth of the kernel).
    auto write = [&](int hq, const floatx4 (&o)[8], float l) {
        if (c >= np) return;
        OutT* dst = out + (static_cast<uint64_t>(row0 + c) * p.num_q_heads + static_cast<uint64_t>(g) * G + hq) * 128 +
                    4 * j;
#pragma unroll
        for (int n = 0; n < 8; ++n) {
            if constexpr (sizeof(OutT) == 4) {
                u32x4 a;
#pragma unroll
                for (int r = 0; r < 4; ++r) a[r] = __float_as_uint(o[n][r] / l);
                *reinterpret_cast<u32x4*>(dst + 16 * n) = a;
            } else {
                uint2v a;
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const OutT lo_v = from_float<OutT>(o[n][2 * k] / l);
                    const OutT hi_v = from_float<OutT>(o[n][2 * k + 1] / l);
                    a[k] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, lo_v)) |
                           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, hi_v)) << 16);
                }
                *reinterpret_cast<uint2v*>(dst + 16 * n) = a;
            }
        }
    };
    la = sum_over_j(la);
    lb = sum_over_j(lb);
    if (has_a) write(h0 + wave, oa, la);
    if (has_b) write(h0 + wave + kPrefillWaves, ob, lb);
}

bool prefill_mfma_supported(const DecodeGeometry& g, uint32_t kv_dtype, uintptr_t query_addr, uintptr_t kv_base_addr,
                            uintptr_t out_addr) {
    const bool pow2 = g.tpb != 0 && (g.tpb & (g.tpb - 1)) == 0;
    const bool aligned = (g.block_stride % 16 == 0) && (g.k_off % 16 == 0) && (g.v_off % 16 == 0) &&
                         (g.token_stride % 16 == 0) && (g.head_stride % 16 == 0) && (kv_base_addr % 16 == 0) &&
                         (query_addr % 16 == 0) && (out_addr % 16 == 0);
    return kv_dtype == QVP_DTYPE_BF16 && g.head_dim == 128 && g.group >= 1 && g.group <= 16 && pow2 && g.tpb >= 16 &&
           aligned;
}

uint32_t log2_u32(uint32_t x) {
    uint32_t r = 0;
    while ((1u << r) < x) ++r;
    return r;
}

}  // namespace

void destroy_prefill_plan(qvp_prefill_plan& p) {
    if (p.staging_pending) (void)hipEventSynchronize(p.staging_done);
    if (p.staging != nullptr) (void)hipHostFree(p.staging);
    if (p.staging_done != nullptr) (void)hipEventDestroy(p.staging_done);
    if (p.device != nullptr) (void)hipFree(p.device);
    if (p.virt != nullptr) (void)qvp_batch_destroy(p.virt);
    p = qvp_prefill_plan{};
}

}  // namespace qvp

extern "C" int qvp_paged_prefill(const qvp_prefill_args* a, void* stream) {
    using qvp::fail;
    if (a == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "args is NULL");
    qvp_packed_view v{};
    QVP_TRY(qvp_batch_view(a->batch, &v));
    qvp_batch* batch = const_cast<qvp_batch*>(a->batch);
    if (a->query == nullptr || a->out == nullptr || a->kv_base == nullptr) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "query, out or kv_base is NULL");
    }
    if (v.num_seqs > 0 && a->q_start == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "q_start is NULL");
    const size_t esz = qvp::dtype_size(a->kv_dtype);
    const size_t osz = qvp::dtype_size(a->out_dtype);
    if (esz == 0 || osz == 0) return fail(QVP_ERR_INVALID_ARGUMENT, "unknown dtype");
    if (a->num_query_heads == 0 || a->num_kv_heads == 0 || a->num_query_heads % a->num_kv_heads != 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "%u query heads do not group onto %u kv heads", a->num_query_heads,
                    a->num_kv_heads);
    }
    if (a->layer >= a->num_layers) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "layer %u outside %u layers", a->layer, a->num_layers);
    }
    if (a->head_dim == 0) return fail(QVP_ERR_INVALID_ARGUMENT, "head_dim is 0");
    if (a->tokens_per_block != v.tokens_per_block) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "batch packed for %u tokens per block, args say %u", v.tokens_per_block,
                    a->tokens_per_block);
    }
    if (a->head_stride < a->head_dim || a->token_stride == 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "head vectors overlap");
    }
    const uint64_t last_elem = static_cast<uint64_t>(a->num_layers - 1) * a->layer_stride + a->stream_stride +
                               static_cast<uint64_t>(a->tokens_per_block - 1) * a->token_stride +
                               static_cast<uint64_t>(a->num_kv_heads - 1) * a->head_stride + a->head_dim;
    if (last_elem * esz > a->block_stride) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "layout addresses %llu bytes but frames are %llu bytes",
                    static_cast<unsigned long long>(last_elem * esz),
                    static_cast<unsigned long long>(a->block_stride));
    }
    const std::vector<int32_t>& lens = batch->host_seq_lens;
    uint64_t total_new = 0;
    for (uint32_t s = 0; s < v.num_seqs; ++s) {
        if (a->q_start[s] >= static_cast<uint32_t>(lens[s])) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "sequence %u: first new position %u is not below its context %d", s,
                        a->q_start[s], lens[s]);
        }
        total_new += static_cast<uint32_t>(lens[s]) - a->q_start[s];
    }
    if (total_new > 0x7fffffffu) return fail(QVP_ERR_INVALID_ARGUMENT, "too many new tokens");
    if (v.num_seqs == 0) return QVP_OK;

    qvp::DecodeGeometry g{};
    g.kv_base = static_cast<const uint8_t*>(a->kv_base);
    g.block_stride = a->block_stride;
    g.k_off = static_cast<uint64_t>(a->layer) * a->layer_stride * esz;
    g.v_off = g.k_off + a->stream_stride * esz;
    g.token_stride = a->token_stride * esz;
    g.head_stride = a->head_stride * esz;
    g.tables = v.block_tables;
    g.seq_lens = v.seq_lens;
    g.query = a->query;
    g.max_nb = v.max_blocks_per_seq;
    g.tpb = a->tokens_per_block;
    g.tpb_shift = qvp::log2_u32(a->tokens_per_block);
    g.num_q_heads = a->num_query_heads;
    g.num_kv_heads = a->num_kv_heads;
    g.group = a->num_query_heads / a->num_kv_heads;
    g.head_dim = a->head_dim;
    g.scale_log2 = a->scale * qvp::kLog2e;
    hipStream_t s = qvp::as_stream(stream);
    qvp_prefill_plan& plan = batch->prefill;
    // A pack left pending by qvp_pack_ahead is uploaded before its prefill.
    QVP_TRY(qvp::flush_own_upload(batch, s));

    // The MFMA kernel takes its running maximum on raw scores: scale > 0.
    if (!(a->scale > 0.0f) || !qvp::prefill_mfma_supported(g, a->kv_dtype, reinterpret_cast<uintptr_t>(a->query),
                                                            reinterpret_cast<uintptr_t>(a->kv_base),
                                                            reinterpret_cast<uintptr_t>(a->out))) {
        // One virtual sequence per new position, over the same frames, run in
        // chunks of at most kMaxVirtualIds block ids (a long prompt needs
        // about n^2 / (2 tokens_per_block) of them). Chunks are packed and
        // decoded in order on the stream; the query and output rows of a
        // chunk start at its first position's row.
        if (plan.virt == nullptr) QVP_TRY(qvp_batch_create(&plan.virt));
        qvp_decode_args d{};
        d.kv_base = a->kv_base;
        d.block_stride = a->block_stride;
        d.batch = plan.virt;
        d.kv_dtype = a->kv_dtype;
        d.out_dtype = a->out_dtype;
        d.layer = a->layer;
        d.num_layers = a->num_layers;
        d.num_query_heads = a->num_query_heads;
        d.num_kv_heads = a->num_kv_heads;
        d.head_dim = a->head_dim;
        d.tokens_per_block = a->tokens_per_block;
        d.head_stride = a->head_stride;
        d.token_stride = a->token_stride;
        d.stream_stride = a->stream_stride;
        d.layer_stride = a->layer_stride;
        d.scale = a->scale;
        const uint64_t row_elems = static_cast<uint64_t>(a->num_query_heads) * a->head_dim;
        std::vector<uint32_t> ids, cu{0}, ctx;
        uint64_t first_row = 0;
        auto flush = [&]() -> int {
            if (ctx.empty()) return QVP_OK;
            QVP_TRY(qvp_pack(plan.virt, static_cast<uint32_t>(ctx.size()), ids.data(), cu.data(), ctx.data(),
                             a->tokens_per_block, v.num_pool_blocks, v.split_tokens, stream));
            d.query = static_cast<const uint8_t*>(a->query) + first_row * row_elems * esz;
            d.out = static_cast<uint8_t*>(a->out) + first_row * row_elems * osz;
            QVP_TRY(qvp_paged_decode(&d, stream));
            first_row += ctx.size();
            ids.clear();
            cu.assign(1, 0);
            ctx.clear();
            return QVP_OK;
        };
        for (uint32_t sq = 0; sq < v.num_seqs; ++sq) {
            const uint32_t* row = batch->host_ids.data() + batch->host_cu_blocks[sq];
            for (uint32_t pos = a->q_start[sq]; pos < static_cast<uint32_t>(lens[sq]); ++pos) {
                const uint32_t nb = (pos + a->tokens_per_block) / a->tokens_per_block;
                if (ids.size() + nb > qvp::kMaxVirtualIds) QVP_TRY(flush());
                ids.insert(ids.end(), row, row + nb);
                cu.push_back(static_cast<uint32_t>(ids.size()));
                ctx.push_back(pos + 1);
            }
        }
        return flush();
    }

    // Work items, longest context first.
    const uint32_t G = g.group;
    const uint32_t head_sets = (G + qvp::kPrefillHeadsPerItem - 1) / qvp::kPrefillHeadsPerItem;
    std::vector<qvp::PrefillItem> items;
    uint32_t row = 0;
    for (uint32_t sq = 0; sq < v.num_seqs; ++sq) {
        const uint32_t start = a->q_start[sq];
        const uint32_t end = static_cast<uint32_t>(lens[sq]);
        for (uint32_t p0 = start; p0 < end; p0 += qvp::kPrefillPositions) {
            const uint32_t np = std::min<uint32_t>(qvp::kPrefillPositions, end - p0);
            for (uint32_t kv = 0; kv < a->num_kv_heads; ++kv) {
                for (uint32_t hs = 0; hs < head_sets; ++hs) {
                    items.push_back(qvp::PrefillItem{static_cast<int32_t>(sq), static_cast<int32_t>(kv),
                                                     static_cast<int32_t>(p0), static_cast<int32_t>(np),
                                                     static_cast<int32_t>(row + (p0 - start)),
                                                     static_cast<int32_t>(hs * qvp::kPrefillHeadsPerItem)});
                }
            }
        }
        row += end - start;
    }
    std::stable_sort(items.begin(), items.end(), [](const qvp::PrefillItem& x, const qvp::PrefillItem& y) {
        return x.p0 + x.np > y.p0 + y.np;
    });
    if (items.size() > 0x7fffffffu) return fail(QVP_ERR_INVALID_ARGUMENT, "too many prefill items");
    const size_t ints = items.size() * (sizeof(qvp::PrefillItem) / sizeof(int32_t));
    // Host-side reuse of pinned staging only: no system-scope release.
    if (plan.staging_done == nullptr) {
        QVP_HIP(hipEventCreateWithFlags(&plan.staging_done, hipEventDisableTiming | hipEventDisableSystemFence));
    }
    if (plan.staging_pending) {
        QVP_HIP(hipEventSynchronize(plan.staging_done));
        plan.staging_pending = false;
    }
    if (plan.staging_cap < ints) {
        if (plan.staging != nullptr) QVP_HIP(hipHostFree(plan.staging));
        plan.staging = nullptr;
        plan.staging_cap = 0;
        QVP_HIP(hipHostMalloc(reinterpret_cast<void**>(&plan.staging), ints * sizeof(int32_t), hipHostMallocCoherent));
        plan.staging_cap = ints;
    }
    if (plan.device_cap < ints) {
        // The device list may still be read by an earlier prefill on this batch.
        if (plan.device != nullptr) {
            QVP_HIP(hipStreamSynchronize(s));
            QVP_HIP(hipFree(plan.device));
        }
        plan.device = nullptr;
        plan.device_cap = 0;
        QVP_HIP(hipMalloc(reinterpret_cast<void**>(&plan.device), ints * sizeof(int32_t)));
        plan.device_cap = ints;
    }
    std::memcpy(plan.staging, items.data(), ints * sizeof(int32_t));
    QVP_TRY(qvp::pull_from_pinned(plan.device, plan.staging, ints * sizeof(int32_t), s));
    QVP_HIP(hipEventRecord(plan.staging_done, s));
    plan.staging_pending = true;

    const auto* dev_items = reinterpret_cast<const qvp::PrefillItem*>(plan.device);
    const dim3 grid(static_cast<unsigned>(items.size()));
    switch (a->out_dtype) {
        case QVP_DTYPE_F32:
            hipLaunchKernelGGL(qvp::prefill_mfma<float>, grid, dim3(qvp::kPrefillThreads), 0, s, g, dev_items, a->out);
            break;
        case QVP_DTYPE_BF16:
            hipLaunchKernelGGL(qvp::prefill_mfma<uint16_t>, grid, dim3(qvp::kPrefillThreads), 0, s, g, dev_items,
                               a->out);
            break;
        default:
            hipLaunchKernelGGL(qvp::prefill_mfma<_Float16>, grid, dim3(qvp::kPrefillThreads), 0, s, g, dev_items,
                               a->out);
            break;
    }
    QVP_HIP(hipGetLastError());
    // The kernel reads the packed block tables: a later pack into this slot
    // from another stream waits for it.
    return qvp::note_reader(batch->readers[batch->current], s, batch->upload_stream[batch->current]);
}

// Persistent MFMA paged decode for bf16 caches with head_dim 128.
//
// Semantics: include/qwenvl_paged/PagedAttention.h:53-127 (softmax(scale q K^T) V
// per query head, GQA head h reads kv head h / (Hq / Hkv), fp32 accumulation).
//
// Work decomposition. Every (sequence b, kv head g) pair is a segment of
// ceil(len_b / 32) tiles of 32 tokens. The host lays the sequences' tiles end
// to end and cuts them into equal-sized contiguous ranges, one per workgroup
// and kv head (one resident workgroup of eight waves per CU, launched once:
// no tail of half-empty rounds, no per-item start-up cost, and no CU-mate
// workgroup whose loads queue behind another's); the workgroups of one range
// have consecutive ids, so a frame's kv heads are read side by side. A range
// covers one or more pieces (its intersection with segments). Inside a piece
// the waves of the workgroup take tiles round-robin, keep an online-softmax state (running max
// m, running sum l, unnormalised accumulator O) and merge it through LDS when
// the piece ends. A piece that is a whole segment writes the final output; the
// other pieces write (m, l, O) to a workspace slot with agent-scope stores,
// which are written through to the point of coherence shared by all XCDs.
// When a workgroup has run through its range, each wave waits until its
// stores have completed there (vmcnt(0)) and, after a workgroup barrier, one
// thread per partial piece increments that segment's counter with an
// agent-scope atomic; the workgroup that completes a segment's count reads the
// slots with agent-scope loads (which read at that point of coherence),
// merges them in one pass, out = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M)
// with M = max_s m_s, and resets the counter for the next launch. Publishing
// once at the end keeps the store wait off the prefetch pipeline. (An
// agent-scope release/acquire fence pair would also write back and invalidate
// the XCD's L2; measured, that doubles the kernel's time.)
// Each wave prefetches its next tile (possibly in the next piece) before it
// computes the current one, so loads stay in flight across piece boundaries.
//
// MFMA mapping (v_mfma_f32_16x16x32_bf16; lane l = (c = l % 16, j = l / 16);
// A[row][k] comes from lane (row, k / 8), B[k][col] from lane (col, k / 8), and
// C[4j + r][c] lands in register r of lane (c, j)):
//   QK^T is computed transposed, S^T = K Q^T, per 16-token half u of a tile.
//   Row r of half u carries token (r / 4) + 16u + 4 (r % 4), so C register r of
//   lane (c, j) is the score of token j + 4 (4u + r) for query head c. The
//   query-head group of the kv head fills the 16 columns (up to 16 heads), so
//   each K/V byte is read from HBM once for the whole group. The four k-groups
//   of QK MFMA i cover head dims 32i .. 32i + 31.
//   PV is computed as O^T = V^T P^T. Lane (c, j) holds P for tokens j + 4q,
//   q = 0..7, which is the B operand as it stands (k slot q <-> token j + 4q).
//   V is read with 16-byte coalesced loads, lane (c, j) of load q taking dims
//   8c .. 8c + 7 of token 4q + j; with row x of PV MFMA n standing for dim
//   8x + n, lane (c, j) already holds its A operand (element n of its 8 loads)
//   and only an in-register 16-bit transpose is needed. P enters the bf16 MFMA
//   as hi + lo (hi = P truncated to bf16, lo = P - hi rounded to bf16), which
//   keeps the weights at about 2^-16 relative error. C register r of PV MFMA n
//   in lane (c, j) is O[head c][dim 32j + 8r + n].
#include "f32_tile.h"
#include "mfma_tile.h"
#include "valu_tile.h"

#include <algorithm>
#include <mutex>
#include <vector>

namespace qvp {
namespace {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kD = 128;
constexpr int kRowPad = kD + 4;
// One workgroup of eight waves per CU. Two four-wave workgroups per CU (the
// same waves) were measured 5% slower on the 72B shape: the dispatcher starts
// a CU's second workgroup after every CU has its first, and its waves then
// lose issue arbitration to the older ones.
constexpr int kWgsPerCu = 1;
// Tiles per wave (whole batch over the resident waves) from which kv heads are
// decoded four side by side.
constexpr uint64_t kMinTilesPerWaveForHeadGroups = 32;
// A workgroup's range is contiguous, so only its first and last pieces can be
// partial segments -- unless shared prefixes split its sequences' segments,
// each of which then ends in one piece of the range. Partial pieces one
// workgroup may hold (the planner keeps schedules within it).
constexpr int kMaxMergesPerWg = 64;
// Slots combined per round of loads in the end-of-range merge, and work items
// (four dims of a row) per thread per round.
constexpr int kMergeChunk = 8;
constexpr int kMergeBatch = 2;

// Cost of a piece boundary inside a range, in one wave's tile times: the
// waves' LDS merge (a workgroup barrier) and the piece's stores, which the
// next tile's wait then covers. Per-wave timestamps of the Qwen2-VL-7B batch
// (15 launches): with 0.5 a range's loop still ended ~0.9 us later per extra
// piece (a wave-tile takes ~4.0 us in the steady state), so a boundary costs
// ~0.7 tile times; with 0.7 the residue is ~0.5 us per piece.
constexpr double kPieceBoundaryTiles = 0.7;

// LDS of one workgroup: the CU's 160 KiB (one workgroup per CU), of which the
// kernel's static arrays take kStaticLdsBytes; the rest can hold deferred
// piece results.
constexpr uint32_t kMaxLdsBytes = 160u * 1024u;
constexpr uint32_t kStaticLdsBytes = (2 * kWaves * 16 + kWaves * 16 * kRowPad + kMaxMergesPerWg + 1) * 4 + 64;

// Words per wave of the schedule's first-tile table.
constexpr int kFirstWords = 8;

struct MfmaArgs {
    const qvp_piece* pieces;
    const int32_t* wg_begin;
    const int32_t* first;  // [wg][wave][kFirstWords]: piece, tile, kv head, blk0, blk1, range begin, end
    int32_t* counters;
    float* ws_ml;   // [slot][hps][group][2] : running max (base 2), running sum
    float* ws_acc;  // [slot][hps][group][128]
    void* out;      // [num_seqs][Hq][128]
    int hps;        // kv heads per segment (4, 2 or 1)
    int defer;      // hold piece results in LDS and write them after the range
    // Workgroups past num_decode_wgs copy another pack's pending upload:
    // up_n16 16-byte words up_src -> up_dst, then up_tail 4-byte words.
    int num_decode_wgs;
    const uint4* up_src;
    uint4* up_dst;
    uint64_t up_n16;
    uint32_t up_tail;
};


// The schedule and the block tables do not change while the kernel runs;
// reading them through the constant address space lets the compiler use
// scalar loads (which do not wait behind the wave's outstanding K/V loads)
// although the kernel also performs atomics.
template <typename T>
__device__ inline const __attribute__((address_space(4))) T* as_const(const T* ptr) {
    return (const __attribute__((address_space(4))) T*)(ptr);
}
__device__ inline qvp_piece piece_at(const qvp_piece* pieces, int i) {
    const auto* q = as_const(pieces) + i;
    qvp_piece d;
    d.b = q->b;
    d.g = q->g;
    d.t0 = q->t0;
    d.t1 = q->t1;
    d.ctx = q->ctx;
    d.slot = q->slot;
    d.seg_slot0 = q->seg_slot0;
    d.seg_nslots = q->seg_nslots;
    return d;
}

// A tile of one wave's sequence with its block ids already fetched, so its
// loads can be issued without waiting on the block table.
struct TileRef {
    int b, g, t, ctx;
    int32_t blk0, blk1;  // frames of tokens 32t .. 32t+15 and 32t+16 .. 32t+31
};

// Advances (pi, t) to this wave's next tile: t + tl in the same piece, else
// the first piece after it where the wave has a tile (start t0 + lane). The tl
// tile lanes of a kv head take a piece's tiles round-robin. Starts from piece
// pi when t < 0. Returns false when the range is exhausted.
__device__ inline bool next_tile(const MfmaArgs& a, int pe, int lane, int tl, int& pi, int& t) {
    if (t >= 0) {
        if (t + tl < piece_at(a.pieces, pi).t1) {
            t += tl;
            return true;
        }
        ++pi;
    }
    for (; pi < pe; ++pi) {
        const qvp_piece d = piece_at(a.pieces, pi);
        if (d.t0 + lane < d.t1) {
            t = d.t0 + lane;
            return true;
        }
    }
    t = -1;
    return false;
}

// Fetches the block ids of tile t of piece pi for kv head d.g * hps + hl. A
// 16-token half never straddles a block (tpb is a power of two >= 16); tokens
// past the context fall back to the last valid block.
__device__ inline TileRef resolve_tile(const DecodeGeometry& p, const MfmaArgs& a, int pi, int t, int hl) {
    const qvp_piece d = piece_at(a.pieces, pi);
    TileRef r;
    r.b = d.b;
    r.g = d.g * a.hps + hl;
    r.t = t;
    r.ctx = d.ctx;
    const auto* row = as_const(p.tables) + static_cast<uint64_t>(d.b) * p.max_nb;
    const int tok0 = t * kTileTokens;
    r.blk0 = row[min(tok0, r.ctx - 1) >> p.tpb_shift];
    r.blk1 = row[min(tok0 + 16, r.ctx - 1) >> p.tpb_shift];
    return r;
}

// Issues the 16 loads of a tile. Tokens at or past ctx read in-frame bytes of
// the last valid block; compute masks their scores and zeroes their values when
// it consumes the tile (doing it here would make the wave wait for the loads it
// is prefetching). kStream: non-temporal loads (the persistent decode, which
// reads every byte once: 57.4 -> 52.9 us on the 7B batch); the shared-prefix
// launch keeps plain loads (42.9 us with the hint against 36.8 us without on
// the copy-on-write batch).
template <bool kStream = true>
__device__ inline void load_tile(const DecodeGeometry& p, const TileRef& r, int c, int j, KvTile& tile) {
    const uint32_t tmask = p.tpb - 1;
    const int tok0 = r.t * kTileTokens;
    const uint8_t* head_base = p.kv_base + static_cast<uint64_t>(r.g) * p.head_stride;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const uint8_t* frame = head_base + static_cast<uint64_t>(u == 0 ? r.blk0 : r.blk1) * p.block_stride;
        const int ktok = tok0 + 16 * u + (c >> 2) + 4 * (c & 3);
        const uint8_t* kp = frame + p.k_off + static_cast<uint64_t>(ktok & tmask) * p.token_stride + 16u * j;
#pragma unroll
        for (int i = 0; i < 4; ++i) tile.k[u][i] = kStream ? load16_stream(kp + 64 * i) : load16(kp + 64 * i);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            const int q = 4 * u + qq;
            const int vtok = tok0 + 4 * q + j;
            const uint8_t* vp = frame + p.v_off + static_cast<uint64_t>(vtok & tmask) * p.token_stride + 16u * c;
            tile.v[q] = kStream ? load16_stream(vp) : load16(vp);
        }
    }
}

// load_tile through buffer resources, for kernels bound by their vector ALU
// (the shared-prefix launch): a half tile's frame address is uniform and goes
// into the resource (SGPRs), the lane's part of each address is fixed for the
// kernel and goes into voffset, and the half tile's token offset into
// soffset -- no per-load 64-bit address arithmetic. With tiles starting on
// 16-token boundaries and tokens_per_block a power of two >= 16, token
// 32t + 16u + x (x < 16) sits at slot ((32t + 16u) mod tpb) + x of its frame.
// lane_k = ((c >> 2) + 4 (c & 3)) token_stride + 16 j and lane_v =
// j token_stride + 16 c are the fixed lane offsets of load_tile's K and V rows.
constexpr int kBufferWord3Raw = 0x00020000;  // word 3 of a raw buffer resource on gfx9 parts

__device__ inline void load_tile_buffer(const DecodeGeometry& p, const TileRef& r, uint32_t lane_k, uint32_t lane_v,
                                        KvTile& tile) {
    const uint32_t tmask = p.tpb - 1;
    const int tok0 = r.t * kTileTokens;
    const uint8_t* head_base = p.kv_base + static_cast<uint64_t>(r.g) * p.head_stride;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        uint8_t* frame = const_cast<uint8_t*>(head_base + static_cast<uint64_t>(u == 0 ? r.blk0 : r.blk1) * p.block_stride);
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(frame, 0, 0x7fffffff, kBufferWord3Raw);
        const uint32_t tok = static_cast<uint32_t>((tok0 + 16 * u) & tmask) * static_cast<uint32_t>(p.token_stride);
        const int koff = static_cast<int>(static_cast<uint32_t>(p.k_off) + tok);
        const int voff = static_cast<int>(static_cast<uint32_t>(p.v_off) + tok);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            tile.k[u][i] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, static_cast<int>(lane_k + 64u * i), koff, 0));
        }
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
            tile.v[4 * u + qq] = __builtin_bit_cast(
                u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           rs, static_cast<int>(lane_v), voff + static_cast<int>(4u * qq * p.token_stride), 0));
        }
    }
}

// kVG = 0: matrix-core tiles; 1, 2: vector tiles for query groups up to kVG.
// kElem: the cache's element type (kElemBf16, kElemF16, kElemF32); fp16 and
// fp32 caches run matrix-core tiles only.
template <typename OutT, int kVG, uint32_t kElem>
__global__ __launch_bounds__(kThreads, kWgsPerCu) void decode_mfma_persistent(DecodeGeometry p, MfmaArgs a) {
    static_assert(kElem == kElemBf16 || kVG == 0, "vector tiles read bf16 caches");
    constexpr bool kF16 = kElem == kElemF16;
    constexpr bool kF32 = kElem == kElemF32;
    // Query words per lane: eight bf16 / fp16 elements each of four MFMA
    // k-groups, or four fp32 elements each of eight (f32_tile.h).
    constexpr int kQWords = kF32 ? 8 : 4;
    __shared__ VectorTileLds<kVG> vt;
    __shared__ float sm_m[kWaves][16];
    __shared__ float sm_l[kWaves][16];
    __shared__ float sm_o[kWaves][16][kRowPad];
    __shared__ int sm_merge[kMaxMergesPerWg];
    __shared__ int sm_nmerge;
    // Piece results held until the range is done (a.defer): [piece][hps *
    // G][kD] accumulators, then [piece][hps * G][2] (m, l).
    extern __shared__ float sm_def[];

    // A copy workgroup: launched after the decode workgroups, it only gets a
    // CU once one of them has finished (one decode workgroup fills a CU), so
    // the next step's upload runs in this launch's tail. One 16-byte read of
    // pinned host memory per thread.
    if (static_cast<int>(blockIdx.x) >= a.num_decode_wgs) {
        const uint64_t i = static_cast<uint64_t>(blockIdx.x - a.num_decode_wgs) * kThreads + threadIdx.x;
        if (i < a.up_n16) a.up_dst[i] = a.up_src[i];
        if (static_cast<int>(blockIdx.x) == a.num_decode_wgs && threadIdx.x < a.up_tail) {
            reinterpret_cast<uint32_t*>(a.up_dst + a.up_n16)[threadIdx.x] =
                reinterpret_cast<const uint32_t*>(a.up_src + a.up_n16)[threadIdx.x];
        }
        return;
    }

    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int c = lane & 15;
    const int j = lane >> 4;
    const int G = static_cast<int>(p.group);
    // Wave w decodes kv head hl = w % hps of each segment, tile lane w / hps.
    const int hps = a.hps;
    const int tl = kWaves / hps;
    const int hl = wave % hps;
    const int tlane = wave / hps;
    const int hpsG = hps * G;

    // The wave's first tile (already resolved to frames by the host) and the
    // range come in one scalar load, so its first K/V loads issue without a
    // chain of dependent reads of the schedule and the block table (which
    // every wave of the grid would make at once at start-up).
    const auto* fd = as_const(a.first) + (static_cast<int>(blockIdx.x) * kWaves + wave) * kFirstWords;
    const int pb = fd[5];
    const int pe = fd[6];
    float* def_acc = sm_def;
    float* def_ml = sm_def + (pe - pb) * hpsG * kD;
    OutT* out = static_cast<OutT*>(a.out);

    // Writes element (ri, dd) of a piece's merged state: the output row when
    // the piece is a whole segment, else its workspace slot, with agent-scope
    // stores (written through to the point of coherence shared by all XCDs;
    // the wait before the count-in makes sure they have arrived).
    auto store_result = [&](const qvp_piece& d, int ri, int dd, float acc, float mmax, float lsum) {
        if (d.slot < 0) {
            out[(static_cast<uint64_t>(d.b) * p.num_q_heads + d.g * hpsG + ri) * kD + dd] = from_float<OutT>(acc / lsum);
        } else {
            const uint64_t row = static_cast<uint64_t>(d.slot) * hpsG + ri;
            __hip_atomic_store(&a.ws_acc[row * kD + dd], acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (dd == 0) {
                __hip_atomic_store(&a.ws_ml[row * 2 + 0], mmax, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&a.ws_ml[row * 2 + 1], lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    };
    // A piece's merged element goes to LDS when results are deferred: a
    // global store here would sit in the wave's memory counter ahead of the
    // next tile's loads, and the next tile's wait would then wait for the
    // store's write-through as well.
    auto emit = [&](int pi, const qvp_piece& d, int ri, int dd, float acc, float mmax, float lsum) {
        if (a.defer) {
            const int row = (pi - pb) * hpsG + ri;
            def_acc[row * kD + dd] = acc;
            if (dd == 0) {
                def_ml[2 * row] = mmax;
                def_ml[2 * row + 1] = lsum;
            }
        } else {
            store_result(d, ri, dd, acc, mmax, lsum);
        }
    };

    // Software pipeline per wave: while the current tile is computed, the next
    // tile's loads are in flight (nxt) and the block ids of the tile after that
    // are being fetched (r2), so no table lookup sits between a tile's arrival
    // and the issue of the following loads. (pi2, t2) is the cursor of r2.
    // fp32 caches: a 32-token tile is two 16-token halves, loaded one half
    // ahead; `pend` is the tile whose second half is still to be loaded.
    KvTile nxt;
    TileRef pend{};
    int pi2 = fd[0];
    int t2 = fd[1];
    bool have_partial = false;
    bool has2 = pi2 >= 0;
    if (has2) {
        TileRef r0{};
        r0.g = fd[2];
        r0.t = t2;
        r0.blk0 = fd[3];
        r0.blk1 = fd[4];
        if constexpr (kF32) {
            load_half_f32(p.kv_base, p.block_stride, p.head_stride, p.k_off, p.v_off, p.token_stride, p.tpb, r0.g,
                          r0.blk0, r0.t * kTileTokens, c, j, nxt);
            pend = r0;
        } else {
            load_tile(p, r0, c, j, nxt);
        }
    }
    has2 = has2 && next_tile(a, pe, tlane, tl, pi2, t2);
    TileRef r2{};
    if (has2) r2 = resolve_tile(p, a, pi2, t2, hl);

    // Query B operand: lane (c, j), MFMA i -> Q[head g*G + c][dims 32i + 8j
    // .. +8]. Columns past the group repeat the group's last head: their
    // scores, weights and outputs stay in their own columns and are never
    // written, and not masking leaves the loads' results unused until the
    // first tile is computed (a select on them would wait at once). The next
    // piece's query is loaded when a piece starts, so it has arrived when
    // that piece's first tile is computed.
    // (fp32: lane (c, j) holds dims 32j .. 32j + 31 of head c, f32_tile.h.)
    auto load_query = [&](int pi, u32x4 (&qo)[kQWords]) {
        const qvp_piece d = piece_at(a.pieces, pi);
        const uint64_t row = (static_cast<uint64_t>(d.b) * p.num_q_heads + (d.g * hps + hl) * G + min(c, G - 1)) * kD;
        if constexpr (kF32) {
            const float* q = static_cast<const float*>(p.query) + row + 32 * j;
#pragma unroll
            for (int i = 0; i < 8; ++i) qo[i] = *reinterpret_cast<const u32x4*>(q + 4 * i);
        } else {
            const uint16_t* q = static_cast<const uint16_t*>(p.query) + row;
#pragma unroll
            for (int i = 0; i < 4; ++i) qo[i] = *reinterpret_cast<const u32x4*>(q + 32 * i + 8 * j);
        }
    };
    // fp32 loads each piece's query when the piece starts: holding the next
    // one as well (32 more registers) made the kernel spill.
    constexpr bool kQueryAhead = !kF32;
    u32x4 qnext[kQueryAhead ? kQWords : 1];
    if constexpr (kQueryAhead) {
        if (pb < pe) load_query(pb, qnext);
    }
    for (int pi = pb; pi < pe; ++pi) {
        const qvp_piece d = piece_at(a.pieces, pi);
        const int ctx = d.ctx;
        u32x4 qop[kQWords];
        if constexpr (kQueryAhead) {
#pragma unroll
            for (int i = 0; i < kQWords; ++i) qop[i] = qnext[i];
            if (pi + 1 < pe) load_query(pi + 1, qnext);
        } else {
            load_query(pi, qop);
        }

        if constexpr (kVG == 0) {
            floatx4 o[8];
#pragma unroll
            for (int n = 0; n < 8; ++n) o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
            float m_run = -INFINITY;
            float l_run = 0.f;

            if constexpr (kF32) {
                for (int t = d.t0 + tlane; t < d.t1; t += tl) {
                    KvTile cur = nxt;  // first half of tile t
                    load_half_f32(p.kv_base, p.block_stride, p.head_stride, p.k_off, p.v_off, p.token_stride, p.tpb,
                                  pend.g, pend.blk1, pend.t * kTileTokens + 16, c, j, nxt);
                    compute_half_f32(cur, qop, t * kTileTokens, ctx - 1, ctx, p.scale_log2, j, m_run, l_run, o);
                    cur = nxt;  // second half
                    if (has2) {
                        load_half_f32(p.kv_base, p.block_stride, p.head_stride, p.k_off, p.v_off, p.token_stride,
                                      p.tpb, r2.g, r2.blk0, r2.t * kTileTokens, c, j, nxt);
                        pend = r2;
                    }
                    has2 = has2 && next_tile(a, pe, tlane, tl, pi2, t2);
                    if (has2) r2 = resolve_tile(p, a, pi2, t2, hl);
                    compute_half_f32(cur, qop, t * kTileTokens + 16, ctx - 1, ctx, p.scale_log2, j, m_run, l_run, o);
                }
            } else {
                for (int t = d.t0 + tlane; t < d.t1; t += tl) {
                    KvTile cur = nxt;
                    if (has2) load_tile(p, r2, c, j, nxt);
                    has2 = has2 && next_tile(a, pe, tlane, tl, pi2, t2);
                    if (has2) r2 = resolve_tile(p, a, pi2, t2, hl);
                    compute_tile<kF16>(cur, qop, t * kTileTokens, ctx - 1, ctx, p.scale_log2, j, m_run, l_run, o);
                }
            }

            // This wave's state for (piece, head g) goes to LDS in row layout.
            l_run = sum_over_j(l_run);
            if (j == 0) {
                sm_m[wave][c] = m_run;
                sm_l[wave][c] = l_run;
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int n = 0; n < 8; ++n) sm_o[wave][c][32 * j + 8 * r + n] = o[n][r];
        } else {
            // The piece's query to LDS as [dim][head]; every wave of this kv
            // head writes the same values and reads only what it wrote (the
            // previous piece's reads ended at its closing barrier).
            stage_query<kVG>(vt.q[hl], qop, c, j);
            __builtin_amdgcn_wave_barrier();
            float o[kVG][8];
            float m_run[kVG];
            float l_part[kVG];
#pragma unroll
            for (int h = 0; h < kVG; ++h) {
                m_run[h] = -INFINITY;
                l_part[h] = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) o[h][e] = 0.f;
            }

            for (int t = d.t0 + tlane; t < d.t1; t += tl) {
                KvTile cur = nxt;
                if (has2) load_tile(p, r2, c, j, nxt);
                has2 = has2 && next_tile(a, pe, tlane, tl, pi2, t2);
                if (has2) r2 = resolve_tile(p, a, pi2, t2, hl);
                compute_tile_vector<kVG>(cur, vt.q[hl], vt.p[wave], t * kTileTokens, ctx - 1, ctx, p.scale_log2, c,
                                         j, m_run, l_part, o);
            }

            // The same row layout as the matrix-core state: the running sum
            // adds the 16 lanes c (the j rows agree), the outputs the four
            // j lanes' token classes.
#pragma unroll
            for (int h = 0; h < kVG; ++h) {
                const float lsum = sum_over_c(l_part[h]);
                if (lane == 0) {
                    sm_m[wave][h] = m_run[h];
                    sm_l[wave][h] = lsum;
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float ov = sum_over_j(o[h][e]);
                    if (j == 0) sm_o[wave][h][8 * c + e] = ov;
                }
            }
        }

        have_partial = have_partial || d.slot >= 0;
        if (hps == 1) {
            // The eight waves are tile lanes of one head: merge them through LDS.
            lds_barrier();
            for (int e = threadIdx.x; e < G * kD; e += kThreads) {
                const int hc = e >> 7;
                const int dd = e & (kD - 1);
                float mmax = sm_m[0][hc];
#pragma unroll
                for (int w = 1; w < kWaves; ++w) mmax = fmaxf(mmax, sm_m[w][hc]);
                float acc = 0.f;
                float lsum = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) {
                    const float f = fast_exp2(sm_m[w][hc] - mmax);
                    acc += sm_o[w][hc][dd] * f;
                    lsum += sm_l[w][hc] * f;
                }
                emit(pi, d, hc, dd, acc, mmax, lsum);
            }
            lds_barrier();
        } else {
            // hps heads of kWaves / hps tile lanes each: merge each head's lanes
            // through LDS.
            lds_barrier();
            for (int e = threadIdx.x; e < hpsG * kD; e += kThreads) {
                const int ri = e >> 7;  // row within the segment: head ri / G, query column ri % G
                const int h2 = ri / G;
                const int hc = ri - h2 * G;
                const int dd = e & (kD - 1);
                float mmax = sm_m[h2][hc];
                for (int w = h2 + hps; w < kWaves; w += hps) mmax = fmaxf(mmax, sm_m[w][hc]);
                float acc = 0.f;
                float lsum = 0.f;
                for (int w = h2; w < kWaves; w += hps) {
                    const float f = fast_exp2(sm_m[w][hc] - mmax);
                    acc += sm_o[w][hc][dd] * f;
                    lsum += sm_l[w][hc] * f;
                }
                emit(pi, d, ri, dd, acc, mmax, lsum);
            }
            lds_barrier();
        }
    }

    // Deferred results: every piece's rows, now that the range's loads are
    // done (the last piece's merge ended with a barrier, so all rows are in
    // LDS).
    if (a.defer) {
        for (int k = 0; k < pe - pb; ++k) {
            const qvp_piece d = piece_at(a.pieces, pb + k);
            for (int e = threadIdx.x; e < hpsG * kD; e += kThreads) {
                const int row = k * hpsG + (e >> 7);
                store_result(d, e >> 7, e & (kD - 1), def_acc[row * kD + (e & (kD - 1))], def_ml[2 * row],
                             def_ml[2 * row + 1]);
            }
        }
    }

    if (!have_partial) return;

    // Count this workgroup's partial slots in; the workgroup whose increment
    // completes a segment merges it. A workgroup barrier alone does not wait
    // for outstanding stores, so each wave first waits for all of its memory
    // operations (the slot stores are agent-scope stores: they are complete
    // once written through to the point of coherence), and the barrier then
    // orders all the waves' stores before any counter moves. The asm's
    // memory clobber keeps the compiler from moving memory accesses across
    // the wait. A contiguous range holds at most two partial pieces (its
    // first and last) unless shared prefixes split the segments of its
    // sequences (each then ends in one private piece of the range, counted in
    // after the prefix launch counted its chunks): thread k counts piece
    // pb + k in, all in parallel, and the completed segments go to a list.
    // The descriptors of the pieces to count in are read before the wait, so
    // their loads overlap it.
    int my_slot = -1;
    int my_seg = 0;
    int my_n = 0;
    if (static_cast<int>(threadIdx.x) < pe - pb) {
        const qvp_piece d = piece_at(a.pieces, pb + static_cast<int>(threadIdx.x));
        my_slot = d.slot;
        my_seg = d.seg_slot0;
        my_n = d.seg_nslots;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (threadIdx.x == 0) sm_nmerge = 0;
    __syncthreads();
    for (int k = threadIdx.x; k < pe - pb; k += kThreads) {
        if (k != static_cast<int>(threadIdx.x)) {
            const qvp_piece d = piece_at(a.pieces, pb + k);
            my_slot = d.slot;
            my_seg = d.seg_slot0;
            my_n = d.seg_nslots;
        }
        if (my_slot < 0) continue;
        const int done = __hip_atomic_fetch_add(&a.counters[my_seg], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == my_n - 1) {
            const int at = __hip_atomic_fetch_add(&sm_nmerge, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            sm_merge[at] = pb + k;
        }
    }
    __syncthreads();
    // Merge the segments this workgroup completed. All their elements are
    // spread over the workgroup's threads, kMergeBatch per thread per round,
    // and each round issues every slot load of its elements before combining
    // (agent-scope loads read the slots of other workgroups, on other XCDs,
    // from the point of coherence): the merge costs about one round trip.
    const int nm = __builtin_amdgcn_readfirstlane(sm_nmerge);
    if (nm == 0) return;
    // Work items are four consecutive dims of one row: per slot one 8-byte
    // agent-scope load of the row's (m, l) and two of its four accumulators.
    const int per_seg = hpsG * (kD / 4);
    const int total = nm * per_seg;
    int max_ns = 0;
    for (int i = 0; i < nm; ++i) max_ns = max(max_ns, piece_at(a.pieces, __builtin_amdgcn_readfirstlane(sm_merge[i])).seg_nslots);
    for (int f0 = threadIdx.x; f0 < total; f0 += kThreads * kMergeBatch) {
        int ri[kMergeBatch], dq[kMergeBatch], s0[kMergeBatch], ns[kMergeBatch];
        uint64_t orow[kMergeBatch];
        float mmax[kMergeBatch], lsum[kMergeBatch], acc[kMergeBatch][4];
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            const int f = f0 + i * kThreads;
            const int si = f < total ? f / per_seg : 0;
            const int e = f < total ? f - si * per_seg : 0;
            const qvp_piece m = piece_at(a.pieces, sm_merge[si]);
            ri[i] = e >> 5;
            dq[i] = e & 31;
            s0[i] = m.seg_slot0;
            ns[i] = f < total ? m.seg_nslots : 0;
            orow[i] = (static_cast<uint64_t>(m.b) * p.num_q_heads + m.g * hpsG) * kD;
            mmax[i] = -INFINITY;
            lsum[i] = 0.f;
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[i][k] = 0.f;
        }
        for (int c0 = 0; c0 < max_ns; c0 += kMergeChunk) {
            uint64_t ml[kMergeBatch][kMergeChunk], o01[kMergeBatch][kMergeChunk], o23[kMergeBatch][kMergeChunk];
#pragma unroll
            for (int i = 0; i < kMergeBatch; ++i) {
#pragma unroll
                for (int x = 0; x < kMergeChunk; ++x) {
                    ml[i][x] = 0;
                    o01[i][x] = 0;
                    o23[i][x] = 0;
                    if (c0 + x < ns[i]) {
                        const uint64_t row = static_cast<uint64_t>(s0[i] + c0 + x) * hpsG + ri[i];
                        ml[i][x] = __hip_atomic_load(reinterpret_cast<const uint64_t*>(a.ws_ml + row * 2),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        const uint64_t* op = reinterpret_cast<const uint64_t*>(a.ws_acc + row * kD + 4 * dq[i]);
                        o01[i][x] = __hip_atomic_load(op, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        o23[i][x] = __hip_atomic_load(op + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < kMergeBatch; ++i) {
                float cm = mmax[i];
#pragma unroll
                for (int x = 0; x < kMergeChunk; ++x) {
                    if (c0 + x < ns[i]) cm = fmaxf(cm, __uint_as_float(static_cast<uint32_t>(ml[i][x])));
                }
                // Items past the end have no slot: keep them finite.
                const float rescale = cm == -INFINITY ? 0.f : fast_exp2(mmax[i] - cm);
                lsum[i] *= rescale;
#pragma unroll
                for (int k = 0; k < 4; ++k) acc[i][k] *= rescale;
#pragma unroll
                for (int x = 0; x < kMergeChunk; ++x) {
                    const float m = __uint_as_float(static_cast<uint32_t>(ml[i][x]));
                    const float f = c0 + x < ns[i] ? fast_exp2(m - cm) : 0.f;
                    lsum[i] += __uint_as_float(static_cast<uint32_t>(ml[i][x] >> 32)) * f;
                    acc[i][0] += __uint_as_float(static_cast<uint32_t>(o01[i][x])) * f;
                    acc[i][1] += __uint_as_float(static_cast<uint32_t>(o01[i][x] >> 32)) * f;
                    acc[i][2] += __uint_as_float(static_cast<uint32_t>(o23[i][x])) * f;
                    acc[i][3] += __uint_as_float(static_cast<uint32_t>(o23[i][x] >> 32)) * f;
                }
                mmax[i] = cm;
            }
        }
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            if (f0 + i * kThreads < total) {
                OutT* dst = out + orow[i] + ri[i] * kD + 4 * dq[i];
#pragma unroll
                for (int k = 0; k < 4; ++k) dst[k] = from_float<OutT>(acc[i][k] / lsum[i]);
            }
        }
    }
    for (int k = threadIdx.x; k < nm; k += kThreads) {
        __hip_atomic_store(&a.counters[piece_at(a.pieces, sm_merge[k]).seg_slot0], 0, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
}

struct PrefixArgs {
    const qvp_prefix_item* items;
    int32_t* counters;
    float* ws_ml;   // the main launch's workspace layout: [slot][group][2]
    float* ws_acc;  // [slot][group][128]
    void* out;
    int num_items;
};

// Segments the prefix launch completes hold only its own slots: the prefix
// chunks and a short suffix (kPrefixMaxChunks + 1). plan_schedule drops the
// shared prefixes of a batch whose plan would give such a segment more.
constexpr int kPrefixMaxSlots = 9;

// Final merge of the (sequence, kv head) segments a prefix-launch workgroup
// completed: segs[i] = (sequence, kv head, first slot, slots). Slots written
// by other workgroups of the launch are read with agent-scope loads. Each
// segment's counter returns to zero for the next launch.
template <typename OutT>
__device__ void merge_prefix_segments(const DecodeGeometry& p, const PrefixArgs& a, int n, const int (*segs)[4]) {
    // Work items are four consecutive dims of one row; each round issues the
    // slot loads of kMergeBatch items per thread together (one 8-byte load of
    // the row's (m, l) and two of its accumulators per slot), so the merge
    // costs about one round trip per round.
    const int G = static_cast<int>(p.group);
    const int per_seg = G * (kD / 4);
    const int total = n * per_seg;
    OutT* out = static_cast<OutT*>(a.out);
    for (int f0 = threadIdx.x; f0 < total; f0 += kThreads * kMergeBatch) {
        int ri[kMergeBatch], dq[kMergeBatch], s0[kMergeBatch], ns[kMergeBatch];
        uint64_t orow[kMergeBatch];
        uint64_t ml[kMergeBatch][kPrefixMaxSlots], o01[kMergeBatch][kPrefixMaxSlots], o23[kMergeBatch][kPrefixMaxSlots];
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            const int f = f0 + i * kThreads;
            const int si = f < total ? f / per_seg : 0;
            const int e = f < total ? f - si * per_seg : 0;
            ri[i] = e >> 5;
            dq[i] = e & 31;
            s0[i] = segs[si][2];
            ns[i] = f < total ? min(segs[si][3], kPrefixMaxSlots) : 0;
            orow[i] = (static_cast<uint64_t>(segs[si][0]) * p.num_q_heads + segs[si][1] * G + ri[i]) * kD;
#pragma unroll
            for (int x = 0; x < kPrefixMaxSlots; ++x) {
                ml[i][x] = 0;
                o01[i][x] = 0;
                o23[i][x] = 0;
                if (x < ns[i]) {
                    const uint64_t row = static_cast<uint64_t>(s0[i] + x) * G + ri[i];
                    ml[i][x] = __hip_atomic_load(reinterpret_cast<const uint64_t*>(a.ws_ml + row * 2), __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
                    const uint64_t* op = reinterpret_cast<const uint64_t*>(a.ws_acc + row * kD + 4 * dq[i]);
                    o01[i][x] = __hip_atomic_load(op, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    o23[i][x] = __hip_atomic_load(op + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kMergeBatch; ++i) {
            if (f0 + i * kThreads >= total) continue;
            float mmax = -INFINITY;
#pragma unroll
            for (int x = 0; x < kPrefixMaxSlots; ++x) {
                if (x < ns[i]) mmax = fmaxf(mmax, __uint_as_float(static_cast<uint32_t>(ml[i][x])));
            }
            float lsum = 0.f;
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int x = 0; x < kPrefixMaxSlots; ++x) {
                const float m = __uint_as_float(static_cast<uint32_t>(ml[i][x]));
                const float f = x < ns[i] && m != -INFINITY ? fast_exp2(m - mmax) : 0.f;
                lsum += __uint_as_float(static_cast<uint32_t>(ml[i][x] >> 32)) * f;
                acc[0] += __uint_as_float(static_cast<uint32_t>(o01[i][x])) * f;
                acc[1] += __uint_as_float(static_cast<uint32_t>(o01[i][x] >> 32)) * f;
                acc[2] += __uint_as_float(static_cast<uint32_t>(o23[i][x])) * f;
                acc[3] += __uint_as_float(static_cast<uint32_t>(o23[i][x] >> 32)) * f;
            }
            OutT* dst = out + orow[i] + 4 * dq[i];
#pragma unroll
            for (int k = 0; k < 4; ++k) dst[k] = from_float<OutT>(acc[k] / lsum);
        }
    }
    for (int i = threadIdx.x; i < n; i += kThreads) {
        __hip_atomic_store(&a.counters[segs[i][2]], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Shared-prefix launch: one workgroup per item -- kv head g of a prefix
// group, one MFMA column block of its members (up to 16 / G sequences of G
// query heads, column c = member c / G, head c % G; columns past the last
// member repeat it and are never stored), shared tiles [t0, t1) of one chunk
// of the prefix. An item of the prefix's last chunk also runs its members'
// short private suffixes (member m's tiles [t1, sfx_t1[m]) from its own
// frames, the other members' columns masked). The items of one (group, kv
// head, chunk) differ only in their columns and read the same tiles; the
// planner numbers them so the dispatcher puts them on one XCD, where all but
// the first read of a tile come from L2. Each wave streams every eighth tile
// with the next one in flight and the frames of the one after resolved, like
// the persistent decode, reading them through buffer
// resources (load_tile_buffer: the kernel is bound by its vector ALU); the
// eight waves merge through LDS. A member whose segment the item completes (one chunk, short
// suffix) gets its output written here; otherwise the item's (m, l, O) goes to
// the member's slot and counts in (agent-scope stores, then, after they have
// completed, one increment per member), and the workgroup completing a
// segment merges it -- or the persistent decode does, later on the stream,
// for a member with a long suffix.
template <typename OutT>
__global__ __launch_bounds__(kThreads, kWgsPerCu) void decode_prefix_columns(DecodeGeometry p, PrefixArgs a) {
    __shared__ float sm_m[kWaves][16];
    __shared__ float sm_l[kWaves][16];
    __shared__ float sm_o[kWaves][16][kRowPad];
    __shared__ int sm_seg[kPrefixMaxMembers][4];
    __shared__ int sm_nseg;
    const auto* it = as_const(a.items) + blockIdx.x;
    const int gq = it->g;
    const int t0 = it->t0;
    const int t1 = it->t1;
    const int nmem = it->nmem;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int c = lane & 15;
    const int j = lane >> 4;
    const int G = static_cast<int>(p.group);
    const int ncol = nmem * G;
    const int cc = min(c, ncol - 1);
    const int mem = cc / G;
    u32x4 qop[4];
    {
        const uint16_t* qp = static_cast<const uint16_t*>(p.query) +
                             (static_cast<uint64_t>(it->b[mem]) * p.num_q_heads + gq * G + cc % G) * kD;
#pragma unroll
        for (int i = 0; i < 4; ++i) qop[i] = *reinterpret_cast<const u32x4*>(qp + 32 * i + 8 * j);
    }

    // The item's tiles, numbered: shared tiles t0 .. t1 - 1, then the suffix
    // tiles member by member; wave w takes numbers w, w + kWaves, ... (a fixed
    // assignment: the waves' merge then adds the same partial results in the
    // same order on every launch, so the output repeats bit for bit).
    const int nshared = t1 - t0;
    int total = nshared;
    for (int m = 0; m < nmem; ++m) total += it->sfx_t1[m] - t1;
    // Tile k: its frames, and for a suffix tile the member (-1: a shared
    // tile, every column sees it).
    const auto* row0 = as_const(p.tables) + static_cast<uint64_t>(it->b[0]) * p.max_nb;
    auto tile_of = [&](int k, int& member) {
        TileRef r{};
        r.g = gq;
        if (k < nshared) {
            member = -1;
            r.b = it->b[0];
            r.t = t0 + k;
            r.ctx = t1 * kTileTokens;
            r.blk0 = row0[(r.t * kTileTokens) >> p.tpb_shift];
            r.blk1 = row0[(r.t * kTileTokens + 16) >> p.tpb_shift];
            return r;
        }
        int e = k - nshared;
        member = 0;
        while (member + 1 < nmem && e >= it->sfx_t1[member] - t1) {
            e -= it->sfx_t1[member] - t1;
            ++member;
        }
        r.t = t1 + e;
        r.b = it->b[member];
        r.ctx = it->ctx[member];
        const auto* row = as_const(p.tables) + static_cast<uint64_t>(r.b) * p.max_nb;
        r.blk0 = row[min(r.t * kTileTokens, r.ctx - 1) >> p.tpb_shift];
        r.blk1 = row[min(r.t * kTileTokens + 16, r.ctx - 1) >> p.tpb_shift];
        return r;
    };

    floatx4 o[8];
#pragma unroll
    for (int n = 0; n < 8; ++n) o[n] = floatx4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    float l_run = 0.f;
    const uint32_t lane_k = static_cast<uint32_t>((c >> 2) + 4 * (c & 3)) * static_cast<uint32_t>(p.token_stride) + 16u * j;
    const uint32_t lane_v = static_cast<uint32_t>(j) * static_cast<uint32_t>(p.token_stride) + 16u * c;
    KvTile nxt;
    TileRef r_nxt{}, r_after{};
    int mem_nxt = -1, mem_after = -1;
    int k_nxt = wave;
    int k_after = wave + kWaves;
    if (k_nxt < total) {
        r_nxt = tile_of(k_nxt, mem_nxt);
        load_tile_buffer(p, r_nxt, lane_k, lane_v, nxt);
    }
    if (k_after < total) r_after = tile_of(k_after, mem_after);
    while (k_nxt < total) {
        KvTile cur = nxt;
        const TileRef r_cur = r_nxt;
        const int mem_cur = mem_nxt;
        k_nxt = k_after;
        if (k_nxt < total) {
            load_tile_buffer(p, r_after, lane_k, lane_v, nxt);
            r_nxt = r_after;
            mem_nxt = mem_after;
            k_after += kWaves;
            if (k_after < total) r_after = tile_of(k_after, mem_after);
        }
        // One body for both kinds of tile (a shared tile masks nothing).
        const int col_last = mem_cur < 0 || mem == mem_cur ? r_cur.ctx - 1 : -1;
        compute_tile<false, true>(cur, qop, r_cur.t * kTileTokens, col_last, r_cur.ctx, p.scale_log2, j, m_run, l_run,
                                  o);
    }

    // Merge the eight waves (a wave with no tile for a column holds -inf, 0
    // and zeros there).
    l_run = sum_over_j(l_run);
    if (j == 0) {
        sm_m[wave][c] = m_run;
        sm_l[wave][c] = l_run;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int n = 0; n < 8; ++n) sm_o[wave][c][32 * j + 8 * r + n] = o[n][r];
    lds_barrier();
    bool counted = false;
    for (int m = 0; m < nmem; ++m) counted = counted || it->slot[m] >= 0;
    OutT* out = static_cast<OutT*>(a.out);
    for (int e = threadIdx.x; e < 16 * kD; e += kThreads) {
        const int col = e >> 7;
        const int dd = e & (kD - 1);
        if (col >= ncol) continue;
        float mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, sm_m[w][col]);
        float acc = 0.f;
        float lsum = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = sm_m[w][col];
            const float f = mw == -INFINITY ? 0.f : fast_exp2(mw - mx);
            acc += sm_o[w][col][dd] * f;
            lsum += sm_l[w][col] * f;
        }
        const int mm = col / G;
        const int h = col - mm * G;
        const int slot = it->slot[mm];
        if (slot < 0) {
            out[(static_cast<uint64_t>(it->b[mm]) * p.num_q_heads + gq * G + h) * kD + dd] = from_float<OutT>(acc / lsum);
        } else {
            const uint64_t ri = static_cast<uint64_t>(slot) * G + h;
            __hip_atomic_store(&a.ws_acc[ri * kD + dd], acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (dd == 0) {
                __hip_atomic_store(&a.ws_ml[ri * 2 + 0], mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(&a.ws_ml[ri * 2 + 1], lsum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (!counted) return;
    // Every wave's slot stores have completed before any member is counted.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (threadIdx.x == 0) sm_nseg = 0;
    __syncthreads();
    if (static_cast<int>(threadIdx.x) < nmem && it->slot[threadIdx.x] >= 0) {
        const int mi = static_cast<int>(threadIdx.x);
        const int seg0 = it->seg_slot0[mi];
        const int nsl = it->nslots[mi];
        const int done = __hip_atomic_fetch_add(&a.counters[seg0], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == nsl - 1) {
            const int at = __hip_atomic_fetch_add(&sm_nseg, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            sm_seg[at][0] = it->b[mi];
            sm_seg[at][1] = gq;
            sm_seg[at][2] = seg0;
            sm_seg[at][3] = nsl;
        }
    }
    __syncthreads();
    const int nseg = __builtin_amdgcn_readfirstlane(sm_nseg);
    if (nseg > 0) merge_prefix_segments<OutT>(p, a, nseg, sm_seg);
}

template <typename OutT>
const void* prefix_kernel_for() {
    return reinterpret_cast<const void*>(&decode_prefix_columns<OutT>);
}

const void* prefix_kernel(uint32_t out_dtype) {
    switch (out_dtype) {
        case QVP_DTYPE_F32: return prefix_kernel_for<float>();
        case QVP_DTYPE_BF16: return prefix_kernel_for<uint16_t>();
        default: return prefix_kernel_for<_Float16>();
    }
}

// The kernel instantiation for an output type, a tile engine and the cache's
// element type (fp16 caches run matrix-core tiles only).
template <typename OutT>
const void* kernel_for_group(uint32_t tile_group, uint32_t elem) {
    if (elem == kElemF16) return reinterpret_cast<const void*>(&decode_mfma_persistent<OutT, 0, kElemF16>);
    if (elem == kElemF32) return reinterpret_cast<const void*>(&decode_mfma_persistent<OutT, 0, kElemF32>);
    switch (tile_group) {
        case 0: return reinterpret_cast<const void*>(&decode_mfma_persistent<OutT, 0, kElemBf16>);
        case 1: return reinterpret_cast<const void*>(&decode_mfma_persistent<OutT, 1, kElemBf16>);
        default: return reinterpret_cast<const void*>(&decode_mfma_persistent<OutT, 2, kElemBf16>);
    }
}

const void* decode_kernel(uint32_t out_dtype, uint32_t tile_group, uint32_t elem) {
    switch (out_dtype) {
        case QVP_DTYPE_F32: return kernel_for_group<float>(tile_group, elem);
        case QVP_DTYPE_BF16: return kernel_for_group<uint16_t>(tile_group, elem);
        default: return kernel_for_group<_Float16>(tile_group, elem);
    }
}

constexpr uint32_t kTileGroups[] = {0, 1, 2};

// Static LDS of an instantiation (the vector tiles add their query and
// weight arrays).
constexpr uint32_t static_lds_bytes(uint32_t tile_group) {
    return kStaticLdsBytes + vector_tile_lds_bytes(static_cast<int>(tile_group));
}

// Resident workgroups per device (one per CU), cached per device ordinal.
std::mutex g_dev_mutex;
std::vector<uint32_t> g_dev_wgs;

int device_max_wgs(uint32_t* wgs) {
    int dev = 0;
    QVP_HIP(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lock(g_dev_mutex);
    if (g_dev_wgs.size() <= static_cast<size_t>(dev)) g_dev_wgs.resize(dev + 1, 0);
    if (g_dev_wgs[dev] == 0) {
        // The kernels may take all of the CU's LDS (deferred piece results
        // beside the static arrays); allowed once per device, before any
        // launch (and so before any graph capture).
        for (uint32_t dt : {QVP_DTYPE_F32, QVP_DTYPE_BF16, QVP_DTYPE_F16}) {
            for (uint32_t tg : kTileGroups) {
                const int dyn = static_cast<int>(kMaxLdsBytes - static_lds_bytes(tg));
                QVP_HIP(hipFuncSetAttribute(decode_kernel(dt, tg, kElemBf16),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, dyn));
            }
            for (uint32_t el : {kElemF16, kElemF32}) {
                QVP_HIP(hipFuncSetAttribute(decode_kernel(dt, 0, el), hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(kMaxLdsBytes - static_lds_bytes(0))));
            }
        }
        int cus = 0;
        QVP_HIP(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        g_dev_wgs[dev] = static_cast<uint32_t>(std::max(1, cus) * kWgsPerCu);
    }
    *wgs = g_dev_wgs[dev];
    return QVP_OK;
}

size_t align_ints(size_t n) { return (n + 63) / 64 * 64; }

// kv heads decoded side by side by one workgroup. Four (when they divide the
// kv head count) gives each head two tile lanes of the same tiles: whole
// token rows are read together and each piece end merges only two lanes. But
// a segment then spans four heads, so the batch is cut into 4x fewer, longer
// segments and each split segment gathers more, larger slots in its final
// merge; that pays only when every wave streams many tiles (long contexts).
uint32_t head_group_size(uint32_t num_kv_heads, uint64_t tiles_per_head, uint32_t max_wgs) {
    const uint64_t per_wave = tiles_per_head * num_kv_heads / (static_cast<uint64_t>(max_wgs) * kWaves);
    if (per_wave < kMinTilesPerWaveForHeadGroups) return 1;
    return num_kv_heads % 4 == 0 ? 4u : (num_kv_heads % 2 == 0 ? 2u : 1u);
}

// Relative streaming cost of kv head group q (hps heads from q * hps). On
// MI355X the bytes at offsets 256 .. 511 of every 1 KiB of device address
// space stream slower than the rest when the 256-byte slices of a 1 KiB row
// are read by different workgroups, and bytes 768 .. 1023 slightly slower
// (Qwen2-VL-7B layout, one kv head per workgroup, per-wave timestamps of 15
// launches: a head-1 wave-tile took 4.9 us in the steady state against 4.0
// us for heads 0 and 2 and 4.1 us for head 3, and its first tile landed ~4 us
// later; with the frame stride padded by 256 bytes the slowness moved with the
// address, not with the head, and laying the head groups' sequences out in
// different orders, so that the four heads of a token are not read at the
// same time, changed nothing). A head's weight is 1 + kSlowSliceCost x the
// fraction of its bytes in slice 1 + kSlice3Cost x the fraction in slice 3,
// over the four token rows that repeat the pattern; with these values the
// four heads' ranges end within 0.7 us of each other on average. The classes
// are fixed only when the pool base, the frame stride and the K/V offsets are
// multiples of 1 KiB and the token and head strides multiples of 256 bytes,
// otherwise every group weighs the same. Groups that cover whole kilobytes
// (four heads of 256 bytes) weigh the same as each other.
constexpr double kSlowSliceCost = 0.36;
constexpr double kSlice3Cost = 0.05;
std::vector<double> head_group_weights(const DecodeGeometry& g, uint32_t hps, uint32_t nq) {
    std::vector<double> w(nq, 1.0);
    const uint64_t base = reinterpret_cast<uintptr_t>(g.kv_base);
    if (base % 1024 != 0 || g.block_stride % 1024 != 0 || g.k_off % 1024 != 0 || g.v_off % 1024 != 0 ||
        g.token_stride % 256 != 0 || g.head_stride % 256 != 0 || g.head_stride * hps >= 1024) {
        return w;
    }
    for (uint32_t q = 0; q < nq; ++q) {
        double slow = 0.0;
        double slow3 = 0.0;
        for (uint32_t h = q * hps; h < (q + 1) * hps; ++h) {
            for (uint64_t t = 0; t < 4; ++t) {
                const uint64_t off = (h * g.head_stride + t * g.token_stride) % 1024;
                if (off >= 256 && off < 512) slow += 1.0;
                if (off >= 768) slow3 += 1.0;
            }
        }
        w[q] = 1.0 + (kSlowSliceCost * slow + kSlice3Cost * slow3) / (4.0 * hps);
    }
    return w;
}

// The allowed range ends of a split-K partition of `part` tiles: every
// multiple of part positions from the start of a sequence (segment) and every
// sequence end, increasing; the last one is T.
std::vector<uint64_t> partition_ends(const std::vector<uint64_t>& pos_cum, uint32_t part) {
    std::vector<uint64_t> ends;
    for (size_t b = 0; b + 1 < pos_cum.size(); ++b) {
        for (uint64_t e = pos_cum[b] + part; e < pos_cum[b + 1]; e += part) ends.push_back(e);
        if (pos_cum[b + 1] > pos_cum[b]) ends.push_back(pos_cum[b + 1]);
    }
    return ends;
}

// Cuts T = pos_cum.back() tile positions into R contiguous ranges of equal
// cost, a position costing 1 and every segment start inside a range (a
// piece boundary: the waves' LDS merge and the piece's stores) costing cb
// more. With part > 0 every cut is the partition end (partition_ends)
// nearest the cost-balanced one that still leaves one partition to each
// later range; R must then not exceed the number of partitions.
std::vector<uint64_t> cut_ranges(const std::vector<uint64_t>& pos_cum, uint32_t R, double cb, uint32_t part) {
    const uint64_t T = pos_cum.back();
    const size_t S = pos_cum.size() - 1;
    std::vector<uint64_t> bd(R + 1, 0);
    bd[R] = T;
    const std::vector<uint64_t> ends = part > 0 ? partition_ends(pos_cum, part) : std::vector<uint64_t>{};
    size_t next_end = 0;  // first partition end the next cut may take
    uint64_t pos = 0;
    size_t seg = 0;
    for (uint32_t r = 0; r + 1 < R; ++r) {
        while (seg < S && pos_cum[seg + 1] <= pos) ++seg;
        // Cost left from pos: its positions plus the segment starts after
        // pos (each one a boundary inside some range), shared evenly by
        // the ranges left, so rounding never piles up in the last one.
        const double left = static_cast<double>(T - pos) + cb * static_cast<double>(S - 1 - seg);
        const double target = left / (R - r);
        double acc = 0.0;
        const uint64_t lo = pos + 1;
        const uint64_t hi = T - (R - 1 - r);
        uint64_t cut = hi;
        uint64_t p = pos;
        size_t sg = seg;
        while (p < T) {
            const uint64_t rem = pos_cum[sg + 1] - p;
            if (acc + static_cast<double>(rem) >= target) {
                // The target can fall before p when the boundary cost just
                // added overshot it (segments shorter than that cost): cut at
                // the segment's start then.
                const double off = target - acc + 0.5;
                cut = p + (off > 0.0 ? static_cast<uint64_t>(off) : 0u);
                break;
            }
            acc += static_cast<double>(rem);
            p = pos_cum[sg + 1];
            ++sg;
            if (p < T) acc += cb;
        }
        cut = std::min(std::max(cut, lo), hi);
        if (part > 0) {
            // Partition ends next_end .. last (inclusive) are open to this
            // cut: each later range keeps one of the ends after it.
            const size_t last = ends.size() - 1 - (R - 1 - r);
            size_t k = static_cast<size_t>(std::lower_bound(ends.begin(), ends.end(), cut) - ends.begin());
            k = std::min(std::max(k, next_end), last);
            if (k > next_end && ends[k] > cut && cut - ends[k - 1] < ends[k] - cut) --k;
            cut = ends[k];
            next_end = k + 1;
        }
        bd[r + 1] = cut;
        pos = cut;
    }
    return bd;
}

// Shared prefixes. A prefix group is up to 4 x (16 / G) sequences (four
// column blocks of 16 / G sequences of G query heads each) whose block lists
// agree over their first `tiles` 32-token tiles. Only whole tiles of shared
// frames count, and every member keeps at least its last tile for the main
// launch, so the prefix tiles are full and every member segment ends in an
// ordinary piece (which completes the segment's merge).
constexpr uint32_t kPrefixMinTiles = 4;
constexpr uint64_t kPrefixMinChunkTiles = 8;
constexpr uint64_t kPrefixMaxChunks = 8;
static_assert(kPrefixMaxSlots == kPrefixMaxChunks + 1, "prefix-launch merge holds every slot of a segment");
// Private suffixes of at most this many tiles are decoded by the prefix launch.
constexpr uint32_t kSuffixMaxTiles = 4;

struct PrefixGroup {
    int nmem{0};
    uint32_t b[kPrefixMaxMembers]{};
    uint32_t tiles{0};
    int chunks{0};
};

std::vector<PrefixGroup> find_prefix_groups(const ScheduleInput& in, const DecodeGeometry& g, uint32_t hps) {
    std::vector<PrefixGroup> out;
    // The shared-prefix launch reads bf16 caches with matrix-core tiles.
    if (hps != 1 || in.partition_tiles != 0 || g.tile_group != 0 || g.kv_elem != kElemBf16 || g.group == 0 ||
        g.group > 16 || in.tpb == 0) {
        return out;
    }
    const int cap = std::min<int>(kPrefixMaxMembers, 4 * static_cast<int>(16 / g.group));
    if (cap < 2) return out;
    // Sequences with at least one shared-candidate frame, ordered by their
    // first frame (then by index): forks of one prompt end up adjacent.
    std::vector<uint32_t> order;
    for (uint32_t b = 0; b < in.num_seqs; ++b) {
        if (in.cu_blocks[b + 1] > in.cu_blocks[b]) order.push_back(b);
    }
    std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) {
        return in.ids[in.cu_blocks[x]] < in.ids[in.cu_blocks[y]];
    });
    auto tiles_of = [&](uint32_t b) { return (static_cast<uint32_t>(in.lens[b]) + kTileTokens - 1) / kTileTokens; };
    size_t i = 0;
    while (i < order.size()) {
        size_t e = i + 1;
        while (e < order.size() && in.ids[in.cu_blocks[order[e]]] == in.ids[in.cu_blocks[order[i]]]) ++e;
        for (size_t g0 = i; g0 + 1 < e; g0 += cap) {
            const size_t g1 = std::min(e, g0 + cap);
            if (g1 - g0 < 2) break;
            // Frames every member shares with the first one, from the start.
            const uint32_t* ids0 = in.ids + in.cu_blocks[order[g0]];
            uint32_t common = in.cu_blocks[order[g0] + 1] - in.cu_blocks[order[g0]];
            uint32_t min_tiles = tiles_of(order[g0]);
            for (size_t k = g0 + 1; k < g1; ++k) {
                const uint32_t b = order[k];
                const uint32_t* ids = in.ids + in.cu_blocks[b];
                const uint32_t nb = std::min(common, in.cu_blocks[b + 1] - in.cu_blocks[b]);
                uint32_t n = 0;
                while (n < nb && ids[n] == ids0[n]) ++n;
                common = n;
                min_tiles = std::min(min_tiles, tiles_of(b));
            }
            const uint64_t shared_tokens = static_cast<uint64_t>(common) * in.tpb;
            uint32_t tiles = static_cast<uint32_t>(shared_tokens / kTileTokens);
            if (min_tiles == 0) continue;
            tiles = std::min(tiles, min_tiles - 1);
            if (tiles < kPrefixMinTiles) continue;
            PrefixGroup pg;
            pg.nmem = static_cast<int>(g1 - g0);
            for (int m = 0; m < pg.nmem; ++m) pg.b[m] = order[g0 + m];
            pg.tiles = tiles;
            out.push_back(pg);
        }
        i = e;
    }
    return out;
}

}  // namespace

void destroy_schedule(qvp_schedule& s) {
    for (int i = 0; i < 2; ++i) {
        if (s.staging_pending[i]) (void)hipEventSynchronize(s.staging_done[i]);
        if (s.staging[i] != nullptr) (void)hipHostFree(s.staging[i]);
        if (s.staging_done[i] != nullptr) (void)hipEventDestroy(s.staging_done[i]);
    }
    if (s.device != nullptr) (void)hipFree(s.device);
    destroy_reader(s.reader);
    s = qvp_schedule{};
}

// The tile math takes its running maximum on raw scores (scale > 0); other
// scales go to the generic kernel.
bool mfma_supported(const DecodeGeometry& g, uint32_t kv_dtype, uintptr_t query_addr, uintptr_t kv_base_addr) {
    const bool pow2 = g.tpb != 0 && (g.tpb & (g.tpb - 1)) == 0;
    const bool aligned = (g.block_stride % 16 == 0) && (g.k_off % 16 == 0) && (g.v_off % 16 == 0) &&
                         (g.token_stride % 16 == 0) && (g.head_stride % 16 == 0) && (kv_base_addr % 16 == 0) &&
                         (query_addr % 16 == 0);
    return (kv_dtype == QVP_DTYPE_BF16 || kv_dtype == QVP_DTYPE_F16 || kv_dtype == QVP_DTYPE_F32) && g.head_dim == kD &&
           g.group >= 1 && g.group <= 16 && pow2 && g.tpb >= 16 && aligned && g.scale_log2 > 0.0f;
}

bool mfma_schedule_current(const qvp_batch* batch, const DecodeGeometry& g) {
    const qvp_schedule& s = batch->sched;
    if (!s.valid || s.pack_generation != batch->generation || s.num_kv_heads != g.num_kv_heads ||
        s.group != g.group || s.tile_group != g.tile_group || s.kv_elem != g.kv_elem ||
        s.partition_tiles != batch->partition_tiles) {
        return false;
    }
    uint32_t max_wgs = 0;
    if (device_max_wgs(&max_wgs) != QVP_OK || s.max_wgs != max_wgs) return false;
    const uint32_t nq = s.num_kv_heads / s.hps;
    return s.weights == head_group_weights(g, s.hps, nq);
}

namespace {

// The schedule, with shared-prefix groups when allow_prefix.
int plan_schedule(qvp_schedule& s, const ScheduleInput& in, const DecodeGeometry& g, bool allow_prefix) {
    const uint32_t num_kv_heads = g.num_kv_heads;
    uint32_t max_wgs = 0;
    QVP_TRY(device_max_wgs(&max_wgs));
    const uint32_t nseq = in.num_seqs;
    std::vector<uint64_t> pos_cum(nseq + 1, 0);
    for (uint32_t b = 0; b < nseq; ++b) {
        pos_cum[b + 1] = pos_cum[b] + (static_cast<uint64_t>(in.lens[b]) + kTileTokens - 1) / kTileTokens;
    }
    const uint32_t hps = head_group_size(num_kv_heads, pos_cum[nseq], max_wgs);
    const uint32_t nq = num_kv_heads / hps;
    const std::vector<double> weights = head_group_weights(g, hps, nq);
    s.valid = false;

    // Shared prefixes: sequences whose block tables start with the same
    // frames (forks of one prompt) have those tiles decoded once for the
    // whole group by a launch before the main one; the main launch covers
    // each sequence's tiles from start[b] on.
    std::vector<PrefixGroup> groups = allow_prefix ? find_prefix_groups(in, g, hps) : std::vector<PrefixGroup>{};
    std::vector<uint32_t> start(nseq, 0);
    // A member whose private suffix is short has it decoded by the prefix
    // launch too (in the items of the prefix's last chunk) and leaves the
    // main launch.
    std::vector<uint8_t> short_suffix(nseq, 0);
    for (const PrefixGroup& pg : groups) {
        for (int m = 0; m < pg.nmem; ++m) {
            const uint32_t b = pg.b[m];
            const uint32_t tiles = (in.lens[b] + kTileTokens - 1) / kTileTokens;
            short_suffix[b] = tiles - pg.tiles <= kSuffixMaxTiles;
            start[b] = short_suffix[b] ? tiles : pg.tiles;
        }
    }
    if (!groups.empty()) {
        for (uint32_t b = 0; b < nseq; ++b) {
            pos_cum[b + 1] = pos_cum[b] + (static_cast<uint64_t>(in.lens[b]) + kTileTokens - 1) / kTileTokens - start[b];
        }
    }
    const uint64_t T = pos_cum[nseq];

    // Segments (b, q): sequence b's kv heads q * hps .. q * hps + hps - 1. With
    // hps kv heads per segment the eight waves of a workgroup split as hps
    // heads x (8 / hps) tile lanes. Every segment of sequence b has the same
    // tiles, so the tile positions of all sequences laid end to end (T per
    // head group) are cut into R_q ranges of equal cost per head group q
    // (tiles plus piece boundaries), R_q in proportion to the group's
    // streaming weight (all equal unless some kv heads sit in the slower
    // address slice). Every workgroup is resident
    // from the start (one per CU). Workgroup ids follow the ranges' start
    // positions, head group breaking ties, so consecutive ids -- which the
    // dispatcher places on consecutive XCDs -- read the kv heads of
    // neighbouring tokens (measured on config2: 1.3 us faster than one XCD
    // per token's heads).
    const uint64_t tl = kWaves / hps;
    // At least one tile per tile lane, at least one range.
    // With a split-K partition the cuts can only fall on partition
    // boundaries: no more ranges than partitions.
    uint64_t cut_room = T;
    if (in.partition_tiles > 0) {
        cut_room = 0;
        for (uint32_t b = 0; b < nseq; ++b) {
            cut_room += (pos_cum[b + 1] - pos_cum[b] + in.partition_tiles - 1) / in.partition_tiles;
        }
    }
    // With shared prefixes the main launch holds the members' private tails,
    // often a tile or two each: one tile per range then keeps them spread
    // over the CUs instead of queued behind one another in a few ranges.
    const uint64_t min_range_tiles = groups.empty() ? tl : 1;
    const uint64_t max_ranges =
        std::max<uint64_t>(1, std::min<uint64_t>((T + min_range_tiles - 1) / min_range_tiles, cut_room));
    const uint32_t R = static_cast<uint32_t>(std::min<uint64_t>(std::max<uint32_t>(1, max_wgs / nq), max_ranges));
    const uint32_t W = R * nq;
    std::vector<uint32_t> Rq(nq, R);
    if (R >= 2) {
        double wsum = 0.0;
        for (double x : weights) wsum += x;
        uint32_t given = 0;
        for (uint32_t q = 0; q < nq; ++q) {
            Rq[q] = std::max<uint32_t>(1, static_cast<uint32_t>(W * weights[q] / wsum + 0.5));
            given += Rq[q];
        }
        // Rounding leftovers go to (or come from) the heaviest group.
        const uint32_t heavy = static_cast<uint32_t>(std::max_element(weights.begin(), weights.end()) - weights.begin());
        Rq[heavy] = static_cast<uint32_t>(std::max<int64_t>(1, static_cast<int64_t>(Rq[heavy]) + W - given));
        for (uint32_t q = 0; q < nq; ++q) Rq[q] = static_cast<uint32_t>(std::min<uint64_t>(Rq[q], max_ranges));
    }

    struct RangeRef {
        uint64_t begin, end;
        uint32_t q;
    };
    std::vector<RangeRef> ranges;
    // A piece boundary costs a wave about kPieceBoundaryTiles tile times;
    // in positions of this segment shape (each position is hps tiles over
    // kWaves waves) that is kPieceBoundaryTiles * kWaves / hps.
    const double cb = kPieceBoundaryTiles * kWaves / hps;
    for (uint32_t q = 0; q < nq && T > 0; ++q) {
        const std::vector<uint64_t> bd = cut_ranges(pos_cum, Rq[q], cb, in.partition_tiles);
        for (uint32_t r = 0; r < Rq[q]; ++r) ranges.push_back({bd[r], bd[r + 1], q});
    }
    std::stable_sort(ranges.begin(), ranges.end(), [](const RangeRef& x, const RangeRef& y) {
        return x.begin != y.begin ? x.begin < y.begin : x.q < y.q;
    });
    const uint32_t Wn = static_cast<uint32_t>(ranges.size());
    std::vector<int32_t>& wg_begin = s.plan_wg_begin;
    std::vector<qvp_piece>& pieces = s.plan_pieces;
    wg_begin.assign(Wn + 1, 0);
    pieces.clear();
    pieces.reserve(static_cast<size_t>(Wn) + static_cast<size_t>(nseq) * nq);
    for (uint32_t w = 0; w < Wn; ++w) {
        const RangeRef& rr = ranges[w];
        wg_begin[w] = static_cast<int32_t>(pieces.size());
        uint64_t pos = rr.begin;
        size_t b = static_cast<size_t>(std::upper_bound(pos_cum.begin(), pos_cum.end(), pos) - pos_cum.begin()) - 1;
        while (pos < rr.end) {
            while (pos_cum[b + 1] <= pos) ++b;
            const uint64_t end = std::min(rr.end, pos_cum[b + 1]);
            qvp_piece pc{};
            pc.b = static_cast<int32_t>(b);
            pc.g = static_cast<int32_t>(rr.q);
            pc.t0 = static_cast<int32_t>(pos - pos_cum[b] + start[b]);
            pc.t1 = static_cast<int32_t>(end - pos_cum[b] + start[b]);
            pc.ctx = static_cast<int32_t>(in.lens[b]);
            pc.slot = -1;
            pc.seg_slot0 = -1;
            pc.seg_nslots = 0;
            pieces.push_back(pc);
            pos = end;
        }
    }
    wg_begin[Wn] = static_cast<int32_t>(pieces.size());

    // Whole-segment pieces need no slot; a split segment's pieces get
    // consecutive slots in tile order, segments numbered in (sequence, head
    // group) order. A head group's ranges were laid out in position order,
    // so a segment's pieces already appear in tile order: one counting pass
    // numbers them (no sort).
    const size_t nseg = static_cast<size_t>(nseq) * nq;
    std::vector<int32_t> seg_count(nseg, 0), seg_base(nseg, -1), seg_next(nseg, 0);
    for (const qvp_piece& pc : pieces) ++seg_count[static_cast<size_t>(pc.b) * nq + pc.g];
    // Prefix-launch items are (group, kv head, MFMA column block, chunk): a
    // prefix is cut into the number of chunks of about equal size that keeps
    // the items at about one per CU -- one chunk when the column blocks alone
    // fill the CUs, and the items then complete their members' segments. Each
    // chunk is one more slot of every member's segment and comes first in it;
    // a short suffix runs in the last chunk's items.
    const uint32_t mpb = 16 / g.group;  // sequences per column block
    uint64_t base_items = 0;
    for (const PrefixGroup& pg : groups) {
        base_items += static_cast<uint64_t>(nq) * ((static_cast<uint32_t>(pg.nmem) + mpb - 1) / mpb);
    }
    const uint64_t want_chunks = base_items > 0 ? std::max<uint64_t>(1, max_wgs / base_items) : 1;
    for (PrefixGroup& pg : groups) {
        pg.chunks = static_cast<int>(std::max<uint64_t>(
            1, std::min<uint64_t>({want_chunks, kPrefixMaxChunks, pg.tiles / kPrefixMinChunkTiles})));
        for (int m = 0; m < pg.nmem; ++m) {
            for (uint32_t q = 0; q < nq; ++q) {
                const size_t k = static_cast<size_t>(pg.b[m]) * nq + q;
                seg_count[k] += pg.chunks;
                seg_next[k] = pg.chunks;
            }
        }
    }
    // A segment whose every piece is in the prefix launch (a short-suffix
    // member's) is merged there, from at most kPrefixMaxSlots slots held in
    // registers; a plan that would give one more is planned without groups.
    for (const PrefixGroup& pg : groups) {
        for (int m = 0; m < pg.nmem; ++m) {
            if (!short_suffix[pg.b[m]]) continue;
            for (uint32_t q = 0; q < nq; ++q) {
                if (seg_count[static_cast<size_t>(pg.b[m]) * nq + q] > kPrefixMaxSlots) {
                    return plan_schedule(s, in, g, false);
                }
            }
        }
    }
    int32_t next_slot = 0;
    for (size_t k = 0; k < nseg; ++k) {
        if (seg_count[k] > 1) {
            seg_base[k] = next_slot;
            next_slot += seg_count[k];
        }
    }
    for (qvp_piece& pc : pieces) {
        const size_t k = static_cast<size_t>(pc.b) * nq + pc.g;
        if (seg_base[k] < 0) continue;
        pc.slot = seg_base[k] + seg_next[k]++;
        pc.seg_slot0 = seg_base[k];
        pc.seg_nslots = seg_count[k];
    }
    // Items of one (group, kv head, chunk) read the same tiles: they get ids
    // equal modulo the XCD count, which the dispatcher places on one XCD, so
    // the tiles are shared through its L2.
    constexpr size_t kXcds = 8;
    std::vector<qvp_prefix_item> by_xcd[kXcds];
    size_t unit = 0;
    for (const PrefixGroup& pg : groups) {
        const int ncb = (pg.nmem + static_cast<int>(mpb) - 1) / static_cast<int>(mpb);
        for (uint32_t q = 0; q < nq; ++q) {
            for (int ch = 0; ch < pg.chunks; ++ch, ++unit) {
                for (int cb = 0; cb < ncb; ++cb) {
                    qvp_prefix_item it{};
                    it.g = static_cast<int32_t>(q);
                    it.t0 = static_cast<int32_t>(static_cast<int64_t>(pg.tiles) * ch / pg.chunks);
                    it.t1 = static_cast<int32_t>(static_cast<int64_t>(pg.tiles) * (ch + 1) / pg.chunks);
                    it.nmem = std::min<int>(static_cast<int>(mpb), pg.nmem - cb * static_cast<int>(mpb));
                    for (int m = 0; m < kPrefixMaxMembers; ++m) {
                        const uint32_t b = pg.b[cb * static_cast<int>(mpb) + std::min(m, it.nmem - 1)];
                        const size_t k = static_cast<size_t>(b) * nq + q;
                        it.b[m] = static_cast<int32_t>(b);
                        it.ctx[m] = static_cast<int32_t>(in.lens[b]);
                        it.sfx_t1[m] = ch == pg.chunks - 1 && short_suffix[b] ? static_cast<int32_t>(start[b]) : it.t1;
                        it.slot[m] = seg_base[k] >= 0 ? seg_base[k] + ch : -1;
                        it.seg_slot0[m] = seg_base[k];
                        it.nslots[m] = seg_count[k];
                    }
                    by_xcd[unit % kXcds].push_back(it);
                }
            }
        }
    }
    std::vector<qvp_prefix_item>& items = s.plan_prefix;
    items.clear();
    for (size_t at = 0;; ++at) {
        bool any = false;
        for (size_t x = 0; x < kXcds; ++x) {
            if (at < by_xcd[x].size()) {
                items.push_back(by_xcd[x][at]);
                any = true;
            }
        }
        if (!any) break;
    }
    std::vector<qvp_piece>& suffix = s.plan_suffix;
    suffix.clear();
    // The kernel counts in at most kMaxMergesPerWg partial pieces per range:
    // without shared prefixes only a range's first and last piece are
    // partial; a schedule whose prefix groups would exceed the bound (many
    // tiny forked sequences in one range) is planned without them.
    uint32_t max_partial = 0;
    for (uint32_t w = 0; w < Wn; ++w) {
        uint32_t n = 0;
        for (int32_t pi = wg_begin[w]; pi < wg_begin[w + 1]; ++pi) {
            if (pieces[pi].slot < 0) continue;
            ++n;
            if (groups.empty() && pi != wg_begin[w] && pi != wg_begin[w + 1] - 1) {
                return fail(QVP_ERR_INVALID_ARGUMENT, "schedule puts a partial segment inside workgroup %u's range", w);
            }
        }
        max_partial = std::max(max_partial, n);
    }
    if (max_partial > static_cast<uint32_t>(kMaxMergesPerWg)) {
        if (!groups.empty()) return plan_schedule(s, in, g, false);
        return fail(QVP_ERR_INVALID_ARGUMENT, "schedule gives a workgroup %u partial pieces", max_partial);
    }

    // Piece results are held in LDS until a range is done when the largest
    // range's pieces fit beside the kernel's static arrays.
    uint32_t np_max = 0;
    for (uint32_t w = 0; w < Wn; ++w) {
        np_max = std::max<uint32_t>(np_max, static_cast<uint32_t>(wg_begin[w + 1] - wg_begin[w]));
    }
    const uint64_t def_bytes = static_cast<uint64_t>(np_max) * hps * g.group * (kD + 2) * sizeof(float);
    s.defer = def_bytes + static_lds_bytes(g.tile_group) <= kMaxLdsBytes;
    s.lds_bytes = s.defer ? static_cast<uint32_t>(def_bytes) : 0u;

    s.off_wg_begin = 0;
    s.off_pieces = align_ints(Wn + 1);
    s.off_counters = s.off_pieces + align_ints(pieces.size() * (sizeof(qvp_piece) / sizeof(int32_t)));
    s.off_first = s.off_counters + align_ints(std::max<int32_t>(next_slot, 1));
    const size_t first_words = static_cast<size_t>(Wn) * kWaves * kFirstWords;
    s.off_prefix = s.off_first + align_ints(first_words);
    s.off_suffix = s.off_prefix + align_ints(items.size() * (sizeof(qvp_prefix_item) / sizeof(int32_t)));
    s.total = s.off_suffix + align_ints(suffix.size() * (sizeof(qvp_piece) / sizeof(int32_t)));

    s.pack_generation = in.generation;
    s.num_kv_heads = num_kv_heads;
    s.group = g.group;
    s.tile_group = g.tile_group;
    s.kv_elem = g.kv_elem;
    s.partition_tiles = in.partition_tiles;
    s.max_wgs = max_wgs;
    s.weights = weights;
    s.num_wgs = Wn;
    s.num_pieces = static_cast<uint32_t>(pieces.size());
    s.num_slots = static_cast<uint32_t>(next_slot);
    s.hps = hps;
    s.max_partial_pieces_per_wg = max_partial;
    s.num_prefix_items = static_cast<uint32_t>(items.size());
    s.num_suffix = static_cast<uint32_t>(suffix.size());
    s.prefix_groups = static_cast<uint32_t>(groups.size());
    return QVP_OK;
}

}  // namespace

// A decode loop packs every step, and from one step to the next a sequence
// usually gains one token: its tile count and its frames' sharing stay the
// same, and so does the plan except for the context lengths stored in it.
// The key (tiles per sequence, the shared-prefix groups found, geometry) is
// compared first; on a match only those lengths are rewritten.
int mfma_plan_schedule(qvp_schedule& s, const ScheduleInput& in, const DecodeGeometry& g) {
    uint32_t max_wgs = 0;
    QVP_TRY(device_max_wgs(&max_wgs));
    std::vector<uint32_t> tiles(in.num_seqs);
    uint64_t total = 0;
    for (uint32_t b = 0; b < in.num_seqs; ++b) {
        tiles[b] = (static_cast<uint32_t>(in.lens[b]) + kTileTokens - 1) / kTileTokens;
        total += tiles[b];
    }
    const uint32_t hps = head_group_size(g.num_kv_heads, total, max_wgs);
    std::vector<uint32_t> groups;
    for (const PrefixGroup& pg : find_prefix_groups(in, g, hps)) {
        groups.push_back(static_cast<uint32_t>(pg.nmem));
        groups.push_back(pg.tiles);
        groups.insert(groups.end(), pg.b, pg.b + pg.nmem);
    }
    const bool same_geometry = s.key_valid && s.num_kv_heads == g.num_kv_heads && s.group == g.group &&
                               s.tile_group == g.tile_group && s.kv_elem == g.kv_elem &&
                               s.partition_tiles == in.partition_tiles && s.max_wgs == max_wgs && s.hps == hps &&
                               s.weights == head_group_weights(g, hps, g.num_kv_heads / hps);
    if (same_geometry && tiles == s.key_tiles && groups == s.key_groups) {
        for (qvp_piece& pc : s.plan_pieces) pc.ctx = in.lens[pc.b];
        for (qvp_piece& pc : s.plan_suffix) pc.ctx = in.lens[pc.b];
        for (qvp_prefix_item& it : s.plan_prefix) {
            for (int m = 0; m < kPrefixMaxMembers; ++m) it.ctx[m] = in.lens[it.b[m]];
        }
        s.pack_generation = in.generation;
        return QVP_OK;
    }
    s.key_valid = false;
    QVP_TRY(plan_schedule(s, in, g, true));
    s.key_tiles = std::move(tiles);
    s.key_groups = std::move(groups);
    s.key_valid = true;
    return QVP_OK;
}

void mfma_write_schedule(const qvp_schedule& s, const ScheduleInput& in, int32_t* h) {
    const std::vector<int32_t>& wg_begin = s.plan_wg_begin;
    const std::vector<qvp_piece>& pieces = s.plan_pieces;
    const uint32_t Wn = s.num_wgs;
    const int32_t hps = static_cast<int32_t>(s.hps);
    std::fill(h, h + s.total, 0);  // counters start at zero
    std::copy(wg_begin.begin(), wg_begin.end(), h + s.off_wg_begin);
    const int32_t* praw = reinterpret_cast<const int32_t*>(pieces.data());
    std::copy(praw, praw + pieces.size() * (sizeof(qvp_piece) / sizeof(int32_t)), h + s.off_pieces);
    const int32_t* xraw = reinterpret_cast<const int32_t*>(s.plan_prefix.data());
    std::copy(xraw, xraw + s.plan_prefix.size() * (sizeof(qvp_prefix_item) / sizeof(int32_t)), h + s.off_prefix);
    const int32_t* sraw = reinterpret_cast<const int32_t*>(s.plan_suffix.data());
    std::copy(sraw, sraw + s.plan_suffix.size() * (sizeof(qvp_piece) / sizeof(int32_t)), h + s.off_suffix);
    // Each wave's first tile, resolved to frames here (the kernel's
    // next_tile and resolve_tile for its first step), written straight into
    // the staging buffer (its other words stay zero).
    uint32_t shift = 0;
    while ((1u << shift) < in.tpb) ++shift;
    for (uint32_t w = 0; w < Wn; ++w) {
        for (int wave = 0; wave < kWaves; ++wave) {
            int32_t* f = h + s.off_first + (static_cast<size_t>(w) * kWaves + wave) * kFirstWords;
            const int32_t hl = wave % hps;
            const int32_t tlane = wave / hps;
            f[0] = -1;
            f[5] = wg_begin[w];
            f[6] = wg_begin[w + 1];
            for (int32_t pi = wg_begin[w]; pi < wg_begin[w + 1]; ++pi) {
                const qvp_piece& pc = pieces[pi];
                if (pc.t0 + tlane >= pc.t1) continue;
                const int32_t t = pc.t0 + tlane;
                const uint32_t* row = in.ids + in.cu_blocks[pc.b];
                const int32_t tok0 = t * kTileTokens;
                f[0] = pi;
                f[1] = t;
                f[2] = pc.g * hps + hl;
                f[3] = static_cast<int32_t>(row[std::min(tok0, pc.ctx - 1) >> shift]);
                f[4] = static_cast<int32_t>(row[std::min(tok0 + 16, pc.ctx - 1) >> shift]);
                break;
            }
        }
    }
}

int mfma_prepare_schedule(qvp_batch* batch, const DecodeGeometry& g, hipStream_t stream, bool may_allocate) {
    if (mfma_schedule_current(batch, g)) return QVP_OK;
    qvp_schedule& s = batch->sched;
    ScheduleInput in{};
    in.num_seqs = static_cast<uint32_t>(batch->host_seq_lens.size());
    in.lens = batch->host_seq_lens.data();
    in.ids = batch->host_ids.data();
    in.cu_blocks = batch->host_cu_blocks.data();
    in.tpb = batch->view.tokens_per_block;
    in.generation = batch->generation;
    in.partition_tiles = batch->partition_tiles;
    if (!may_allocate) {
        // Plan into a copy, so that a refusal leaves the schedule as it was.
        qvp_schedule probe{};
        QVP_TRY(mfma_plan_schedule(probe, in, g));
        const int next = s.staging_slot;
        if (s.staging_done[next] == nullptr || s.staging_cap[next] < probe.total || s.device_cap < probe.total) {
            return fail(QVP_ERR_CAPACITY,
                        "the decode's work schedule needs %zu words of buffers this batch does not have yet: pack it "
                        "with qvp_pack_for_decode for this decode, or decode it once with qvp_paged_decode",
                        probe.total);
        }
    }
    QVP_TRY(mfma_plan_schedule(s, in, g));

    const int slot = s.staging_slot;
    s.staging_slot ^= 1;
    if (s.staging_done[slot] == nullptr) {
        QVP_HIP(hipEventCreateWithFlags(&s.staging_done[slot], hipEventDisableTiming));
    }
    // The staging buffer about to be refilled may still be read by the
    // upload of the rebuild before last.
    if (s.staging_pending[slot]) {
        QVP_HIP(hipEventSynchronize(s.staging_done[slot]));
        s.staging_pending[slot] = false;
    }
    if (s.staging_cap[slot] < s.total) {
        if (s.staging[slot] != nullptr) QVP_HIP(hipHostFree(s.staging[slot]));
        s.staging[slot] = nullptr;
        s.staging_cap[slot] = 0;
        QVP_HIP(hipHostMalloc(reinterpret_cast<void**>(&s.staging[slot]), s.total * sizeof(int32_t),
                              hipHostMallocCoherent));
        s.staging_cap[slot] = s.total;
    }
    if (s.device_cap < s.total) {
        // The old buffer may still be read by an earlier decode.
        if (s.device != nullptr) {
            QVP_HIP(hipDeviceSynchronize());
            QVP_HIP(hipFree(s.device));
        }
        s.device = nullptr;
        s.device_cap = 0;
        QVP_HIP(hipMalloc(reinterpret_cast<void**>(&s.device), s.total * sizeof(int32_t)));
        s.device_cap = s.total;
    }
    mfma_write_schedule(s, in, s.staging[slot]);
    // A decode enqueued on another stream may still read the previous
    // schedule in this buffer.
    QVP_TRY(wait_for_reader(s.reader, stream));
    QVP_TRY(pull_from_pinned(s.device, s.staging[slot], s.total * sizeof(int32_t), stream));
    QVP_HIP(hipEventRecord(s.staging_done[slot], stream));
    s.staging_pending[slot] = true;
    s.words = s.device;
    s.in_pack_buffer = false;
    s.valid = true;
    return QVP_OK;
}

uint64_t mfma_prefix_slot_bound(const qvp_batch* batch) {
    // A sequence can be a shared-prefix member only if another sequence
    // starts with the same frame; each member gets at most kPrefixMaxChunks
    // prefix slots per kv head.
    const std::vector<uint32_t>& cu = batch->host_cu_blocks;
    const std::vector<uint32_t>& ids = batch->host_ids;
    if (cu.size() < 3) return 0;
    std::vector<uint32_t> first;
    for (size_t b = 0; b + 1 < cu.size(); ++b) {
        if (cu[b + 1] > cu[b]) first.push_back(ids[cu[b]]);
    }
    std::sort(first.begin(), first.end());
    uint64_t members = 0;
    for (size_t i = 0; i < first.size(); ++i) {
        const bool dup = (i > 0 && first[i - 1] == first[i]) || (i + 1 < first.size() && first[i + 1] == first[i]);
        members += dup ? 1u : 0u;
    }
    return members * kPrefixMaxChunks;
}

uint64_t mfma_workspace_bytes(const qvp_batch* batch, uint32_t group, uint32_t head_dim) {
    const uint64_t rows = static_cast<uint64_t>(batch->sched.num_slots) * batch->sched.hps * group;
    return round_up(rows * 2 * sizeof(float), 256) + round_up(rows * head_dim * sizeof(float), 256);
}

int launch_mfma_decode(const DecodeGeometry& g, const qvp_batch* batch, uint32_t out_dtype, void* out,
                       void* workspace, hipEvent_t split_event, hipStream_t stream, const PendingUpload* upload) {
    const qvp_schedule& s = batch->sched;
    MfmaArgs a{};
    a.wg_begin = s.words + s.off_wg_begin;
    a.pieces = reinterpret_cast<const qvp_piece*>(s.words + s.off_pieces);
    a.counters = s.words + s.off_counters;
    a.first = s.words + s.off_first;
    const uint64_t rows = static_cast<uint64_t>(s.num_slots) * s.hps * g.group;
    a.ws_ml = static_cast<float*>(workspace);
    a.ws_acc = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + round_up(rows * 2 * sizeof(float), 256));
    a.out = out;
    a.hps = static_cast<int>(s.hps);
    a.defer = s.defer ? 1 : 0;
    a.num_decode_wgs = static_cast<int>(s.num_wgs);
    uint32_t copy_wgs = 0;
    if (upload != nullptr) {
        a.up_src = static_cast<const uint4*>(upload->src);
        a.up_dst = static_cast<uint4*>(upload->dst);
        a.up_n16 = upload->n16;
        a.up_tail = upload->tail;
        copy_wgs = static_cast<uint32_t>(std::max<uint64_t>(1, (upload->n16 + kThreads - 1) / kThreads));
    }
    if (s.tile_group != g.tile_group) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "the batch's schedule was planned for another tile engine");
    }
    DecodeGeometry gk = g;
    if (s.num_prefix_items > 0) {
        if (g.kv_elem != kElemBf16) return fail(QVP_ERR_INVALID_ARGUMENT, "shared-prefix schedule for a non-bf16 cache");
        PrefixArgs pa{};
        pa.items = reinterpret_cast<const qvp_prefix_item*>(s.words + s.off_prefix);
        pa.counters = a.counters;
        pa.ws_ml = a.ws_ml;
        pa.ws_acc = a.ws_acc;
        pa.out = out;
        pa.num_items = static_cast<int>(s.num_prefix_items);
        void* pargs[] = {&gk, &pa};
        QVP_HIP(hipLaunchKernel(prefix_kernel(out_dtype), dim3(s.num_prefix_items), dim3(kThreads), pargs, 0, stream));
    }
    // Every sequence may be covered by the prefix launch (then only a carried
    // upload, if any, needs this one).
    if (s.num_wgs + copy_wgs > 0) {
        void* kargs[] = {&gk, &a};
        QVP_HIP(hipLaunchKernel(decode_kernel(out_dtype, s.tile_group, g.kv_elem), dim3(s.num_wgs + copy_wgs),
                                dim3(kThreads), kargs, s.lds_bytes, stream));
    }
    // The merge runs inside the kernel; the event still marks the split/merge
    // boundary for callers that time the two phases.
    if (split_event != nullptr) QVP_HIP(hipEventRecord(split_event, stream));
    return QVP_OK;
}

}  // namespace qvp

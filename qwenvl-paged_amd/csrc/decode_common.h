// Definitions shared by the paged-decode kernels and their launcher.
#pragma once

#include "batch.h"
#include "common.h"

namespace qvp {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;

// Layout and batch arguments common to both decode paths (bytes unless noted).
struct DecodeGeometry {
    const uint8_t* kv_base;
    uint64_t block_stride;
    uint64_t k_off;         // frame start -> this layer's K half
    uint64_t v_off;         // frame start -> this layer's V half
    uint64_t token_stride;
    uint64_t head_stride;
    const int32_t* tables;  // [num_seqs][max_nb]
    const int32_t* seq_lens;
    const void* query;      // [num_seqs][Hq][D], cache element type
    uint32_t max_nb;
    uint32_t tpb;
    uint32_t tpb_shift;     // log2(tpb) when tpb is a power of two
    uint32_t num_q_heads;
    uint32_t num_kv_heads;
    uint32_t group;
    uint32_t head_dim;
    float scale_log2;       // scale * log2(e)
    // Persistent kernel: 0 for matrix-core tiles, else vector tiles for query
    // groups up to this bound (1, 2, 4 or 8).
    uint32_t tile_group;
    // Persistent kernel: the cache's (and query's) element type, kElemBf16,
    // kElemF16 or kElemF32.
    uint32_t kv_elem;
};

// Element codes of DecodeGeometry::kv_elem.
constexpr uint32_t kElemBf16 = 0;
constexpr uint32_t kElemF16 = 1;
constexpr uint32_t kElemF32 = 2;

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

template <typename T> __device__ inline float to_float(T v);
template <> __device__ inline float to_float<float>(float v) { return v; }
template <> __device__ inline float to_float<uint16_t>(uint16_t v) { return bf16_bits_to_float(v); }
template <> __device__ inline float to_float<_Float16>(_Float16 v) { return static_cast<float>(v); }

template <typename OutT> __device__ inline OutT from_float(float v);
template <> __device__ inline float from_float<float>(float v) { return v; }
template <> __device__ inline uint16_t from_float<uint16_t>(float v) { return float_to_bf16_bits(v); }
template <> __device__ inline _Float16 from_float<_Float16>(float v) { return static_cast<_Float16>(v); }

// Generic path: one workgroup per (split, query head), VALU only; splits are
// the packer's fixed-size token partitions. Returns a qvp_status.
int launch_generic_decode(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t kv_dtype,
                          uint32_t out_dtype, void* out, void* workspace, hipEvent_t split_event,
                          hipStream_t stream);
uint64_t generic_workspace_bytes(const qvp_packed_view& v, uint32_t hq, uint32_t d);
// GQA-folded split decode (groups of 1 .. 16, any element type, head_dim a
// multiple of four up to 1024 with rows aligned to four elements, its LDS
// within 64 KiB): one workgroup per (split, kv head), the generic workspace
// layout and merge. Returns a qvp_status.
bool grouped_supported(const DecodeGeometry& g, uint32_t kv_dtype, uint32_t split_tokens);
int launch_grouped_decode(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t kv_dtype, uint32_t out_dtype,
                          void* out, void* workspace, hipEvent_t split_event, hipStream_t stream);
// Combines the per-split (m, l, O) of the generic workspace layout into the
// output (one workgroup per (sequence, query head)).
int launch_merge_splits(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t out_dtype, void* out,
                        const float* ws_ml, const float* ws_acc, hipStream_t stream);

// fp32 caches, head_dim 128 or 64, GQA group <= 16, power-of-two tpb >= 16, splits a
// multiple of 16 tokens: the fp32 MFMA kernel, one workgroup per (split, kv
// head), in the generic workspace layout. Returns a qvp_status.
bool f32_grouped_supported(const DecodeGeometry& g, uint32_t kv_dtype, uint32_t split_tokens, uintptr_t query_addr,
                           uintptr_t kv_base_addr);
int launch_f32_grouped_decode(const DecodeGeometry& g, const qvp_packed_view& v, uint32_t out_dtype, void* out,
                              void* workspace, hipEvent_t split_event, hipStream_t stream);

// Vector tiles of the persistent kernel take query groups up to this size;
// the automatic choice uses them for groups up to kVectorTilesUpToGroup (0:
// never, matrix-core tiles for every group).
constexpr uint32_t kVectorTileMaxGroup = 2;
constexpr uint32_t kVectorTilesUpToGroup = 0;

// Validates decode arguments against a packed view (every refusal of
// qvp_paged_decode) and fills the kernels' geometry. *supported_mfma tells
// whether the persistent MFMA kernel runs this decode.
int decode_geometry(const qvp_decode_args* a, const qvp_packed_view& v, DecodeGeometry* g, bool* supported_mfma);

// MFMA path (bf16, fp16 or fp32, head_dim 128, group <= 16, power-of-two tpb
// >= 16, scale > 0): persistent workgroups over a balanced schedule built from
// the batch.
bool mfma_supported(const DecodeGeometry& g, uint32_t kv_dtype, uintptr_t query_addr,
                    uintptr_t kv_base_addr);

// Tokens per tile of the persistent decode (its schedule counts tiles).
constexpr uint32_t kScheduleTileTokens = 32;

// The host-side batch a schedule is planned from (context lengths and the
// needed block ids in CSR form).
struct ScheduleInput {
    uint32_t num_seqs;
    const int32_t* lens;
    const uint32_t* ids;
    const uint32_t* cu_blocks;
    uint32_t tpb;
    uint64_t generation;  // pack generation the schedule will belong to
    // Split-K partition in 32-token tiles: ranges are cut only at multiples of
    // it inside a sequence (or at sequence ends); 0 cuts anywhere.
    uint32_t partition_tiles;
};
// True when the batch's schedule was built for this pack and this geometry.
bool mfma_schedule_current(const qvp_batch* batch, const DecodeGeometry& g);
// Plans the schedule (host): fills s's plan, sizes and key; s.total words.
int mfma_plan_schedule(qvp_schedule& s, const ScheduleInput& in, const DecodeGeometry& g);
// Writes the planned schedule's s.total words to h (pinned staging).
void mfma_write_schedule(const qvp_schedule& s, const ScheduleInput& in, int32_t* h);
// Builds and uploads the schedule on `stream` unless it is current. Without
// may_allocate a rebuild that needs new staging or device buffers (or event
// objects) is refused with QVP_ERR_CAPACITY before anything changes.
int mfma_prepare_schedule(qvp_batch* batch, const DecodeGeometry& g, hipStream_t stream, bool may_allocate = true);
uint64_t mfma_workspace_bytes(const qvp_batch* batch, uint32_t group, uint32_t head_dim);
// Slots per query head that shared prefixes can add to a decode of the batch
// (an upper bound: members x the largest number of prefix chunks).
uint64_t mfma_prefix_slot_bound(const qvp_batch* batch);
// Enqueues the persistent kernel; with `upload`, extra workgroups of the same
// launch copy that pending pack upload in the launch's tail.
int launch_mfma_decode(const DecodeGeometry& g, const qvp_batch* batch, uint32_t out_dtype, void* out,
                       void* workspace, hipEvent_t split_event, hipStream_t stream,
                       const PendingUpload* upload = nullptr);

}  // namespace qvp

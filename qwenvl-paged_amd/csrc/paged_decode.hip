// qvp_paged_decode: host-side validation and dispatch of the paged decode
// (include/qwenvl_paged/PagedAttention.h:53-127).
//
// Every check the reference makes before computing (PagedAttention.h:59-68:
// element size, context length, layer, head grouping) happens here, plus the
// ones a device kernel needs (the layout stays inside a frame, buffers are
// large enough); the packer already refused unmapped or swapped blocks
// (:73-89). Only then is anything enqueued, so a refused call leaves `out`
// untouched. bf16, fp16 and fp32 caches with head_dim 128 run the persistent
// MFMA kernel (decode_mfma.hip); other shapes run a split kernel: the fp32
// MFMA one (decode_f32.hip), the 16-bit MFMA one for head_dim 64
// (decode_split16.hip), the GQA-folded one for groups up to 16 with
// four-element rows, or the per-query-head generic one (both in
// decode_generic.hip).
#include "decode_common.h"
#include "decode_split16.h"

#include <algorithm>
#include <mutex>
#include <vector>

namespace {

using qvp::fail;

struct Workspace {
    void* ptr{nullptr};
    uint64_t bytes{0};
};

std::mutex g_ws_mutex;
std::vector<Workspace> g_ws;

// Per-device workspace owned by the library, grown on demand.
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

// Workspace of qvp_paged_decode_noalloc: a fixed array in each device's
// memory, reserved when the code object loads and held until the process
// ends, so the call itself allocates nothing. In host code `scratch` names a
// host-side stand-in; its device address comes from hipGetSymbolAddress,
// taken once per device (with that device current) and kept below.
constexpr uint64_t kScratchBytes = 16ull << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxScratchDevices] = {};

int scratch_address(void** out) {
    int dev = 0;
    QVP_HIP(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxScratchDevices) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "device %d beyond the %d devices the scratch table covers", dev,
                    kMaxScratchDevices);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* ptr = nullptr;
        QVP_HIP(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)));
        if (ptr == nullptr) return fail(QVP_ERR_DEVICE, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return QVP_OK;
}

uint32_t log2_u32(uint32_t x) {
    uint32_t r = 0;
    while ((1u << r) < x) ++r;
    return r;
}

// Upper bound of the MFMA path's workspace: at most one slot per workgroup
// boundary plus one per segment, each holding a group of query heads.
uint64_t mfma_bound_bytes(const qvp_packed_view& v, uint32_t hq, uint32_t d) {
    int dev = 0;
    int cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    }
    const uint64_t rows = (static_cast<uint64_t>(std::max(cus, 1)) * 2 + v.num_seqs) * hq;
    return qvp::round_up(rows * 2 * sizeof(float), 256) + qvp::round_up(rows * d * sizeof(float), 256);
}

}  // namespace

namespace qvp {

int decode_geometry(const qvp_decode_args* a, const qvp_packed_view& v, DecodeGeometry* out, bool* supported_mfma) {
    if (a->query == nullptr || a->out == nullptr || a->kv_base == nullptr) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "query, out or kv_base is NULL");
    }
    const size_t esz = dtype_size(a->kv_dtype);
    const size_t osz = dtype_size(a->out_dtype);
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
        return fail(QVP_ERR_INVALID_ARGUMENT, "head vectors overlap (head_stride %llu < head_dim %u)",
                    static_cast<unsigned long long>(a->head_stride), a->head_dim);
    }
    // Every element the kernels can address must lie inside one frame.
    const uint64_t last_elem = static_cast<uint64_t>(a->num_layers - 1) * a->layer_stride + a->stream_stride +
                               static_cast<uint64_t>(a->tokens_per_block - 1) * a->token_stride +
                               static_cast<uint64_t>(a->num_kv_heads - 1) * a->head_stride + a->head_dim;
    if (last_elem * esz > a->block_stride) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "layout addresses %llu bytes but frames are %llu bytes",
                    static_cast<unsigned long long>(last_elem * esz),
                    static_cast<unsigned long long>(a->block_stride));
    }
    DecodeGeometry& g = *out;
    g = DecodeGeometry{};
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
    g.tpb_shift = log2_u32(a->tokens_per_block);
    g.num_q_heads = a->num_query_heads;
    g.num_kv_heads = a->num_kv_heads;
    g.group = a->num_query_heads / a->num_kv_heads;
    g.head_dim = a->head_dim;
    g.scale_log2 = a->scale * kLog2e;
    g.kv_elem = a->kv_dtype == QVP_DTYPE_F16 ? kElemF16 : (a->kv_dtype == QVP_DTYPE_F32 ? kElemF32 : kElemBf16);
    *supported_mfma = mfma_supported(g, a->kv_dtype, reinterpret_cast<uintptr_t>(a->query),
                                     reinterpret_cast<uintptr_t>(a->kv_base));
    if (a->tile_engine > QVP_TILE_VECTOR) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "unknown tile engine %u", a->tile_engine);
    }
    if (*supported_mfma) {
        if (g.kv_elem != kElemBf16 && a->tile_engine == QVP_TILE_VECTOR) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "vector tiles read bf16 caches; this cache runs matrix-core tiles");
        }
        const bool vector = g.kv_elem == kElemBf16 &&
                            (a->tile_engine == QVP_TILE_VECTOR ||
                             (a->tile_engine == QVP_TILE_AUTO && g.group <= kVectorTilesUpToGroup));
        if (vector && g.group > kVectorTileMaxGroup) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "vector tiles take query groups of at most %u (group %u)",
                        kVectorTileMaxGroup, g.group);
        }
        g.tile_group = vector ? (g.group <= 1 ? 1u : 2u) : 0u;
    }
    return QVP_OK;
}

}  // namespace qvp

extern "C" {

int qvp_decode_workspace_bytes(const qvp_batch* batch, uint32_t num_query_heads, uint32_t head_dim, uint64_t* bytes) {
    if (bytes == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "bytes is NULL");
    qvp_packed_view v{};
    QVP_TRY(qvp_batch_view(batch, &v));
    // Shared-prefix slots come on top of the persistent kernel's own bound.
    const uint64_t prefix_rows = qvp::mfma_prefix_slot_bound(batch) * num_query_heads;
    *bytes = std::max(qvp::generic_workspace_bytes(v, num_query_heads, head_dim),
                      mfma_bound_bytes(v, num_query_heads, head_dim) +
                          qvp::round_up(prefix_rows * 2 * sizeof(float), 256) +
                          qvp::round_up(prefix_rows * head_dim * sizeof(float), 256));
    return QVP_OK;
}

}  // extern "C"

namespace {

// Shared body of qvp_paged_decode and qvp_paged_decode_noalloc. With
// no_alloc, the device scratch array is the workspace and nothing is
// allocated: a schedule that would need new buffers, or a workspace beyond
// the scratch array, is refused with QVP_ERR_CAPACITY.
int decode_impl(const qvp_decode_args* a, void* stream, bool no_alloc) {
    if (a == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "args is NULL");
    qvp_packed_view v{};
    QVP_TRY(qvp_batch_view(a->batch, &v));
    qvp::DecodeGeometry g{};
    bool mfma = false;
    QVP_TRY(qvp::decode_geometry(a, v, &g, &mfma));
    if (v.num_seqs == 0) return QVP_OK;

    hipStream_t s = qvp::as_stream(stream);
    hipEvent_t ev = reinterpret_cast<hipEvent_t>(a->split_event);
    qvp_batch* batch = const_cast<qvp_batch*>(a->batch);
    uint64_t need = 0;
    void* ws = a->workspace;
    if (no_alloc) {
        if (ws != nullptr) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "the allocation-free decode uses its own scratch; workspace must be NULL");
        }
        QVP_TRY(scratch_address(&ws));
    }
    // A pack left pending by qvp_pack_ahead is uploaded before its decode;
    // under graph capture the copy would replay from staging a later pack
    // rewrites, so a capture neither uploads nor carries one. Refused before
    // anything (a schedule upload included) is enqueued.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    QVP_HIP(hipStreamIsCapturing(s, &capture));
    const bool capturing = capture != hipStreamCaptureStatusNone;
    if (capturing && batch->upload_pending[batch->current]) {
        return fail(QVP_ERR_INVALID_ARGUMENT,
                    "the batch's qvp_pack_ahead upload is still pending: enqueue it (qvp_batch_upload) before capture");
    }
    if (mfma) {
        QVP_TRY(qvp::mfma_prepare_schedule(batch, g, s, !no_alloc));
        need = qvp::mfma_workspace_bytes(batch, g.group, g.head_dim);
    } else {
        need = qvp::generic_workspace_bytes(v, a->num_query_heads, a->head_dim);
    }
    if (no_alloc) {
        if (need > kScratchBytes) {
            return fail(QVP_ERR_CAPACITY, "decode needs %llu bytes of workspace, the scratch array holds %llu",
                        static_cast<unsigned long long>(need), static_cast<unsigned long long>(kScratchBytes));
        }
    } else if (ws == nullptr) {
        QVP_TRY(library_workspace(need, &ws));
    } else if (a->workspace_bytes < need) {
        return fail(QVP_ERR_CAPACITY, "workspace of %llu bytes, need %llu",
                    static_cast<unsigned long long>(a->workspace_bytes), static_cast<unsigned long long>(need));
    } else if ((reinterpret_cast<uintptr_t>(ws) & 255u) != 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "workspace must be 256-byte aligned");
    }
    QVP_TRY(qvp::flush_own_upload(batch, s, !no_alloc));
    qvp_decode_plan plan{};
    plan.query_group = g.group;
    int status = QVP_OK;
    if (mfma) {
        // Another batch's pending upload on this stream (the next step,
        // packed ahead) rides in this launch's tail.
        qvp::PendingUpload up{};
        const bool carry = !capturing && qvp::take_pending_upload(s, batch, &up);
        status = qvp::launch_mfma_decode(g, batch, a->out_dtype, a->out, ws, ev, s, carry ? &up : nullptr);
        if (carry && status == QVP_OK) status = qvp::finish_taken_upload(up, s);
        const qvp_schedule& sc = batch->sched;
        plan.kernel = QVP_DECODE_MFMA;
        plan.workgroups = sc.num_wgs;
        plan.pieces = sc.num_pieces;
        plan.slots = sc.num_slots;
        plan.kv_heads_per_segment = sc.hps;
        plan.deferred_results = sc.defer ? 1u : 0u;
        plan.tile_engine = g.tile_group != 0 ? QVP_TILE_VECTOR : QVP_TILE_MATRIX;
        plan.split_tokens = sc.partition_tiles * qvp::kScheduleTileTokens;
        plan.shared_prefix_groups = sc.prefix_groups;
        plan.shared_prefix_items = sc.num_prefix_items;
    } else {
        const bool f32 = qvp::f32_grouped_supported(g, a->kv_dtype, v.split_tokens,
                                                    reinterpret_cast<uintptr_t>(a->query),
                                                    reinterpret_cast<uintptr_t>(a->kv_base));
        const bool s16 = !f32 && qvp::split16_supported(g, a->kv_dtype, v.split_tokens,
                                                        reinterpret_cast<uintptr_t>(a->query));
        const bool grouped = !f32 && !s16 && qvp::grouped_supported(g, a->kv_dtype, v.split_tokens);
        status = f32       ? qvp::launch_f32_grouped_decode(g, v, a->out_dtype, a->out, ws, ev, s)
                 : s16     ? qvp::launch_split16_decode(g, v, a->kv_dtype, a->out_dtype, a->out, ws, ev, s)
                 : grouped ? qvp::launch_grouped_decode(g, v, a->kv_dtype, a->out_dtype, a->out, ws, ev, s)
                           : qvp::launch_generic_decode(g, v, a->kv_dtype, a->out_dtype, a->out, ws, ev, s);
        plan.kernel = f32       ? QVP_DECODE_F32_GROUPED
                      : s16     ? QVP_DECODE_SPLIT_MFMA
                      : grouped ? QVP_DECODE_GROUPED
                                : QVP_DECODE_GENERIC;
        plan.workgroups = v.num_splits * (f32 || s16 || grouped ? a->num_kv_heads : a->num_query_heads);
        plan.pieces = v.num_splits;
        plan.slots = v.num_splits;
        plan.kv_heads_per_segment = 1;
        plan.split_tokens = v.split_tokens;
    }
    if (status != QVP_OK) return status;
    batch->last_plan = plan;
    // Later packs and schedule rebuilds on other streams wait for this read.
    QVP_TRY(qvp::note_reader(batch->readers[batch->current], s, batch->upload_stream[batch->current], !no_alloc));
    if (mfma && !batch->sched.in_pack_buffer) QVP_TRY(qvp::note_reader(batch->sched.reader, s, s, !no_alloc));
    return QVP_OK;
}

}  // namespace

extern "C" {

int qvp_paged_decode(const qvp_decode_args* a, void* stream) { return decode_impl(a, stream, false); }

int qvp_paged_decode_noalloc(const qvp_decode_args* a, void* stream) { return decode_impl(a, stream, true); }

int qvp_decode_plan_info(const qvp_batch* batch, qvp_decode_plan* plan) {
    if (batch == nullptr || plan == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "NULL argument");
    *plan = batch->last_plan;
    return QVP_OK;
}

}  // extern "C"

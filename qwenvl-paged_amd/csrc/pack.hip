// Ragged-batch packing: per scheduler step, flatten the decode batch's block
// tables into the device arrays the decode kernels index.
//
// Reference: docs/architecture.md:117-120 ("flatten entries() into the
// [num_seqs, max_blocks_per_seq] tensor that a paged kernel indexes"),
// include/qwenvl_paged/PagedAttention.h:15-22 (per-sequence context lengths)
// and :73-89 (resolve every needed block before writing any output).
//
// Host work is one pass over the CSR input into a pinned staging buffer; the
// device receives all arrays -- and, when the caller names the decode the
// pack is for, that decode's work schedule -- in a single upload kernel on
// the caller's stream. Packs alternate between two slots (staging and device
// buffers), so the host fills one while the device still reads the other,
// and a pack enqueued on a second stream can upload step n + 1 while step
// n's decode runs.
#include "batch.h"
#include "common.h"
#include "decode_common.h"

#include <algorithm>
#include <mutex>
#include <new>
#include <vector>

namespace {

constexpr uint32_t kSplitQuantum = 128;   // 4 waves x 32-token tiles
constexpr uint32_t kDefaultSplit = 512;
constexpr uint32_t kMaxSplit = 8192;
constexpr size_t kAlignInts = 64;         // 256-byte alignment of sub-arrays

size_t align_ints(size_t n) { return (n + kAlignInts - 1) / kAlignInts * kAlignInts; }

struct Layout {
    size_t tables, seq_lens, cu_seqlens, cu_splits, split_seq, split_start, total;
};

Layout make_layout(uint32_t num_seqs, uint32_t max_nb, uint32_t num_splits) {
    Layout l{};
    size_t off = 0;
    l.tables = off;
    off += align_ints(static_cast<size_t>(num_seqs) * max_nb);
    l.seq_lens = off;
    off += align_ints(num_seqs);
    l.cu_seqlens = off;
    off += align_ints(static_cast<size_t>(num_seqs) + 1);
    l.cu_splits = off;
    off += align_ints(static_cast<size_t>(num_seqs) + 1);
    l.split_seq = off;
    off += align_ints(num_splits);
    l.split_start = off;
    off += align_ints(num_splits);
    l.total = off;
    return l;
}

// Batches whose last pack (qvp_pack_ahead) still waits in staging, in the
// order they were packed.
std::mutex g_pending_mutex;
std::vector<qvp_batch*> g_pending;

void unregister_pending(qvp_batch* batch) {
    std::lock_guard<std::mutex> lock(g_pending_mutex);
    g_pending.erase(std::remove(g_pending.begin(), g_pending.end(), batch), g_pending.end());
}

// The upload of `slot` as a PendingUpload (device mapping of its staging).
int describe_upload(qvp_batch* batch, int slot, qvp::PendingUpload* u) {
    void* src = nullptr;
    QVP_HIP(hipHostGetDevicePointer(&src, batch->staging[slot], 0));
    const size_t bytes = batch->upload_bytes[slot];
    u->batch = batch;
    u->slot = slot;
    u->src = src;
    u->dst = batch->device[slot];
    u->n16 = bytes / 16;
    u->tail = static_cast<uint32_t>((bytes % 16) / 4);
    return QVP_OK;
}

}  // namespace

namespace qvp {

int finish_taken_upload(const PendingUpload& u, hipStream_t stream) {
    qvp_batch* b = u.batch;
    QVP_HIP(hipEventRecord(b->staging_done[u.slot], stream));
    b->staging_pending[u.slot] = true;
    b->upload_stream[u.slot] = stream;
    b->upload_pending[u.slot] = false;
    return QVP_OK;
}

int flush_own_upload(qvp_batch* batch, hipStream_t stream, bool may_allocate) {
    const int slot = batch->current;
    if (!batch->upload_pending[slot]) return QVP_OK;
    // The pack waited on its own stream for the slot's previous reader; an
    // upload enqueued on another stream has to wait for that reader too.
    QVP_TRY(wait_for_reader(batch->readers[slot], stream, may_allocate));
    unregister_pending(batch);
    QVP_TRY(pull_from_pinned(batch->device[slot], batch->staging[slot], batch->upload_bytes[slot], stream));
    PendingUpload u{};
    u.batch = batch;
    u.slot = slot;
    return finish_taken_upload(u, stream);
}

bool take_pending_upload(hipStream_t stream, const qvp_batch* exclude, PendingUpload* out) {
    std::lock_guard<std::mutex> lock(g_pending_mutex);
    for (size_t i = 0; i < g_pending.size(); ++i) {
        qvp_batch* b = g_pending[i];
        if (b == exclude || b->upload_stream[b->current] != stream || !b->upload_pending[b->current]) continue;
        if (describe_upload(b, b->current, out) != QVP_OK) return false;
        g_pending.erase(g_pending.begin() + static_cast<std::ptrdiff_t>(i));
        return true;
    }
    return false;
}

}  // namespace qvp

using qvp::fail;

extern "C" {

int qvp_batch_create(qvp_batch** batch) {
    if (batch == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "batch is NULL");
    *batch = nullptr;
    qvp_batch* b = new (std::nothrow) qvp_batch();
    if (b == nullptr) return fail(QVP_ERR_OUT_OF_MEMORY, "batch descriptor");
    // The staging events only tell the host that the device has finished
    // reading pinned memory; no device write needs to become visible to the
    // host through them, so they skip the system-scope release (a cache
    // writeback between two decodes when a decode carries an upload).
    for (int i = 0; i < 2; ++i) {
        hipError_t err =
            hipEventCreateWithFlags(&b->staging_done[i], hipEventDisableTiming | hipEventDisableSystemFence);
        if (err != hipSuccess) {
            if (i == 1) (void)hipEventDestroy(b->staging_done[0]);
            delete b;
            return qvp::hip_fail(err, "hipEventCreateWithFlags");
        }
    }
    *batch = b;
    return QVP_OK;
}

int qvp_batch_destroy(qvp_batch* batch) {
    if (batch == nullptr) return QVP_OK;
    unregister_pending(batch);
    int status = QVP_OK;
    // Decodes may still read the buffers.
    if (batch->readers[0].pending || batch->readers[1].pending || batch->sched.reader.pending) {
        (void)hipDeviceSynchronize();
    }
    for (int i = 0; i < 2; ++i) {
        if (batch->staging_pending[i]) (void)hipEventSynchronize(batch->staging_done[i]);
        if (batch->staging[i] != nullptr && hipHostFree(batch->staging[i]) != hipSuccess) {
            status = fail(QVP_ERR_DEVICE, "hipHostFree(staging)");
        }
        (void)hipEventDestroy(batch->staging_done[i]);
        if (batch->device[i] != nullptr && hipFree(batch->device[i]) != hipSuccess) {
            status = fail(QVP_ERR_DEVICE, "hipFree(batch)");
        }
        qvp::destroy_reader(batch->readers[i]);
    }
    qvp::destroy_schedule(batch->sched);
    qvp::destroy_prefill_plan(batch->prefill);
    delete batch;
    return status;
}

int qvp_batch_view(const qvp_batch* batch, qvp_packed_view* view) {
    if (batch == nullptr || view == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "NULL argument");
    if (!batch->valid) return fail(QVP_ERR_INVALID_ARGUMENT, "batch has not been packed");
    *view = batch->view;
    return QVP_OK;
}

int qvp_pack(qvp_batch* batch, uint32_t num_seqs, const uint32_t* block_ids,
             const uint32_t* cu_blocks, const uint32_t* context_lens, uint32_t tokens_per_block,
             uint32_t num_pool_blocks, uint32_t split_tokens, void* stream) {
    return qvp_pack_for_decode(batch, num_seqs, block_ids, cu_blocks, context_lens, tokens_per_block,
                               num_pool_blocks, split_tokens, nullptr, stream);
}

}  // extern "C"

namespace {

// qvp_pack_for_decode; with defer_upload the upload is left pending (see
// qvp_pack_ahead).
int pack_impl(qvp_batch* batch, uint32_t num_seqs, const uint32_t* block_ids, const uint32_t* cu_blocks,
              const uint32_t* context_lens, uint32_t tokens_per_block, uint32_t num_pool_blocks,
              uint32_t split_tokens, const qvp_decode_args* decode, void* stream, bool defer_upload) {
    if (batch == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "batch is NULL");
    if (tokens_per_block == 0) return fail(QVP_ERR_INVALID_ARGUMENT, "tokens_per_block is 0");
    if (num_seqs > 0 && (cu_blocks == nullptr || context_lens == nullptr)) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "cu_blocks or context_lens is NULL");
    }
    // A split size the caller gives is also where the persistent kernel may
    // cut a sequence between workgroups; 0 leaves its cuts free.
    const bool explicit_split = split_tokens != 0;
    if (split_tokens == 0) split_tokens = kDefaultSplit;
    if (split_tokens > kMaxSplit) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "split_tokens %u exceeds %u", split_tokens, kMaxSplit);
    }
    split_tokens = static_cast<uint32_t>(qvp::round_up(split_tokens, kSplitQuantum));

    // Pass 1: validate everything before touching the batch.
    uint32_t max_nb = 0;
    uint32_t max_len = 0;
    uint64_t num_splits = 0;
    uint64_t total_tokens = 0;
    if (num_seqs > 0 && cu_blocks[0] != 0) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "cu_blocks[0] must be 0");
    }
    for (uint32_t b = 0; b < num_seqs; ++b) {
        const uint32_t len = context_lens[b];
        if (len == 0) return fail(QVP_ERR_INVALID_ARGUMENT, "sequence %u has context_len 0", b);
        if (cu_blocks[b + 1] < cu_blocks[b]) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "cu_blocks decreases at sequence %u", b);
        }
        const uint32_t mapped = cu_blocks[b + 1] - cu_blocks[b];
        const uint32_t needed = (len + tokens_per_block - 1) / tokens_per_block;
        if (needed > mapped) {
            return fail(QVP_ERR_INVALID_ARGUMENT,
                        "sequence %u needs %u blocks for %u tokens but maps %u", b, needed, len,
                        mapped);
        }
        if (needed > 0 && block_ids == nullptr) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "block_ids is NULL");
        }
        const uint32_t* ids = block_ids + cu_blocks[b];
        for (uint32_t j = 0; j < needed; ++j) {
            if (ids[j] == QVP_UNMAPPED_BLOCK || ids[j] >= num_pool_blocks) {
                return fail(QVP_ERR_UNMAPPED, "sequence %u logical block %u has no frame (%u)", b,
                            j, ids[j]);
            }
        }
        max_nb = std::max(max_nb, needed);
        max_len = std::max(max_len, len);
        num_splits += (len + split_tokens - 1) / split_tokens;
        total_tokens += len;
    }
    if (num_pool_blocks > 0x7fffffffu) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "pool of %u blocks exceeds int32 ids", num_pool_blocks);
    }
    if (num_splits > 0x7fffffffu || total_tokens > 0x7fffffffu) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "batch too large for int32 indexing");
    }

    const Layout lay = make_layout(num_seqs, max_nb, static_cast<uint32_t>(num_splits));
    const int slot = batch->parity;

    // The decode this pack is for, when named and run by the MFMA kernel: its
    // schedule is planned now and travels in the same upload, after the
    // packed arrays. Its arguments are validated as qvp_paged_decode would.
    const uint64_t generation = batch->generation + 1;
    qvp::ScheduleInput sin{};
    bool with_schedule = false;
    if (decode != nullptr && num_seqs > 0) {
        qvp_packed_view pv{};
        pv.tokens_per_block = tokens_per_block;
        pv.num_seqs = num_seqs;
        pv.max_blocks_per_seq = max_nb;
        qvp::DecodeGeometry g{};
        QVP_TRY(qvp::decode_geometry(decode, pv, &g, &with_schedule));
        if (with_schedule) {
            batch->lens_scratch.assign(context_lens, context_lens + num_seqs);
            batch->ids_scratch.clear();
            batch->cu_scratch.assign(1, 0);
            for (uint32_t b = 0; b < num_seqs; ++b) {
                const uint32_t needed = (context_lens[b] + tokens_per_block - 1) / tokens_per_block;
                batch->ids_scratch.insert(batch->ids_scratch.end(), block_ids + cu_blocks[b],
                                          block_ids + cu_blocks[b] + needed);
                batch->cu_scratch.push_back(static_cast<uint32_t>(batch->ids_scratch.size()));
            }
            sin.num_seqs = num_seqs;
            sin.lens = batch->lens_scratch.data();
            sin.ids = batch->ids_scratch.data();
            sin.cu_blocks = batch->cu_scratch.data();
            sin.tpb = tokens_per_block;
            sin.generation = generation;
            sin.partition_tiles = explicit_split ? split_tokens / qvp::kScheduleTileTokens : 0u;
            batch->sched.valid = false;
            QVP_TRY(qvp::mfma_plan_schedule(batch->sched, sin, g));
        }
    }
    const size_t total = lay.total + (with_schedule ? batch->sched.total : 0);

    // A pack still waiting for its upload (qvp_pack_ahead) is superseded.
    if (batch->upload_pending[0] || batch->upload_pending[1]) {
        unregister_pending(batch);
        batch->upload_pending[0] = batch->upload_pending[1] = false;
    }
    // The staging buffer about to be reused may still be read by the upload
    // of the call before last.
    if (batch->staging_pending[slot]) {
        QVP_HIP(hipEventSynchronize(batch->staging_done[slot]));
        batch->staging_pending[slot] = false;
    }
    if (batch->staging_cap[slot] < total) {
        if (batch->staging[slot] != nullptr) QVP_HIP(hipHostFree(batch->staging[slot]));
        batch->staging[slot] = nullptr;
        batch->staging_cap[slot] = 0;
        const size_t cap = std::max<size_t>(total + total / 4, 4096);
        QVP_HIP(hipHostMalloc(reinterpret_cast<void**>(&batch->staging[slot]), cap * sizeof(int32_t),
                              hipHostMallocCoherent));
        batch->staging_cap[slot] = cap;
    }
    hipStream_t s = qvp::as_stream(stream);
    if (batch->device_cap[slot] < total) {
        // A decode may still read this slot's old buffer.
        if (batch->readers[slot].pending) QVP_HIP(hipDeviceSynchronize());
        if (batch->device[slot] != nullptr) QVP_HIP(hipFree(batch->device[slot]));
        batch->device[slot] = nullptr;
        batch->device_cap[slot] = 0;
        const size_t cap = std::max<size_t>(total + total / 4, 4096);
        QVP_HIP(hipMalloc(reinterpret_cast<void**>(&batch->device[slot]), cap * sizeof(int32_t)));
        batch->device_cap[slot] = cap;
    }

    // Pass 2: fill the staging buffer.
    int32_t* h = batch->staging[slot];
    int32_t* tables = h + lay.tables;
    int32_t* seq_lens = h + lay.seq_lens;
    int32_t* cu_seqlens = h + lay.cu_seqlens;
    int32_t* cu_splits = h + lay.cu_splits;
    int32_t* split_seq = h + lay.split_seq;
    int32_t* split_start = h + lay.split_start;
    int32_t token_acc = 0;
    int32_t split_acc = 0;
    for (uint32_t b = 0; b < num_seqs; ++b) {
        const uint32_t len = context_lens[b];
        const uint32_t needed = (len + tokens_per_block - 1) / tokens_per_block;
        const uint32_t* ids = block_ids + cu_blocks[b];
        int32_t* row = tables + static_cast<size_t>(b) * max_nb;
        for (uint32_t j = 0; j < needed; ++j) row[j] = static_cast<int32_t>(ids[j]);
        for (uint32_t j = needed; j < max_nb; ++j) row[j] = -1;
        seq_lens[b] = static_cast<int32_t>(len);
        cu_seqlens[b] = token_acc;
        cu_splits[b] = split_acc;
        token_acc += static_cast<int32_t>(len);
        const uint32_t nsplit = (len + split_tokens - 1) / split_tokens;
        for (uint32_t s = 0; s < nsplit; ++s) {
            split_seq[split_acc] = static_cast<int32_t>(b);
            split_start[split_acc] = static_cast<int32_t>(s * split_tokens);
            ++split_acc;
        }
    }
    cu_seqlens[num_seqs] = token_acc;
    cu_splits[num_seqs] = split_acc;
    if (with_schedule) qvp::mfma_write_schedule(batch->sched, sin, h + lay.total);

    // The pack before last (same slot) may still be read by a decode on
    // another stream; one upload then carries the arrays and the schedule
    // (now, or left pending for a later decode on `s`).
    int st = qvp::wait_for_reader(batch->readers[slot], s);
    if (st == QVP_OK && !defer_upload) st = qvp::pull_from_pinned(batch->device[slot], h, total * sizeof(int32_t), s);
    if (st != QVP_OK) {
        batch->valid = false;
        batch->sched.valid = false;
        return st;
    }
    if (defer_upload) {
        batch->upload_pending[slot] = true;
        batch->upload_bytes[slot] = total * sizeof(int32_t);
    } else {
        hipError_t err = hipEventRecord(batch->staging_done[slot], s);
        if (err != hipSuccess) {
            batch->valid = false;
            batch->sched.valid = false;
            return qvp::hip_fail(err, "hipEventRecord(pack)");
        }
        batch->staging_pending[slot] = true;
    }
    batch->upload_stream[slot] = s;
    batch->parity ^= 1;
    batch->current = slot;

    int32_t* d = batch->device[slot];
    if (with_schedule) {
        batch->sched.words = d + lay.total;
        batch->sched.in_pack_buffer = true;
        batch->sched.valid = true;
    }
    qvp_packed_view& v = batch->view;
    v.block_tables = d + lay.tables;
    v.seq_lens = d + lay.seq_lens;
    v.cu_seqlens = d + lay.cu_seqlens;
    v.cu_splits = d + lay.cu_splits;
    v.split_seq = d + lay.split_seq;
    v.split_start = d + lay.split_start;
    v.num_seqs = num_seqs;
    v.max_blocks_per_seq = max_nb;
    v.num_splits = static_cast<uint32_t>(num_splits);
    v.split_tokens = split_tokens;
    v.tokens_per_block = tokens_per_block;
    v.num_pool_blocks = num_pool_blocks;
    v.max_seq_len = max_len;
    v.total_tokens = total_tokens;
    if (with_schedule) {
        std::swap(batch->host_seq_lens, batch->lens_scratch);
        std::swap(batch->host_ids, batch->ids_scratch);
        std::swap(batch->host_cu_blocks, batch->cu_scratch);
    } else {
        batch->host_seq_lens.assign(context_lens, context_lens + num_seqs);
        batch->host_ids.clear();
        batch->host_cu_blocks.assign(1, 0);
        for (uint32_t b = 0; b < num_seqs; ++b) {
            const uint32_t needed = (context_lens[b] + tokens_per_block - 1) / tokens_per_block;
            batch->host_ids.insert(batch->host_ids.end(), block_ids + cu_blocks[b],
                                   block_ids + cu_blocks[b] + needed);
            batch->host_cu_blocks.push_back(static_cast<uint32_t>(batch->host_ids.size()));
        }
    }
    batch->generation = generation;
    batch->partition_tiles = explicit_split ? split_tokens / qvp::kScheduleTileTokens : 0u;
    batch->last_plan = qvp_decode_plan{};
    batch->valid = true;
    if (defer_upload) {
        std::lock_guard<std::mutex> lock(g_pending_mutex);
        g_pending.push_back(batch);
    }
    return QVP_OK;
}

}  // namespace

extern "C" {

int qvp_pack_for_decode(qvp_batch* batch, uint32_t num_seqs, const uint32_t* block_ids,
                        const uint32_t* cu_blocks, const uint32_t* context_lens, uint32_t tokens_per_block,
                        uint32_t num_pool_blocks, uint32_t split_tokens, const qvp_decode_args* decode,
                        void* stream) {
    return pack_impl(batch, num_seqs, block_ids, cu_blocks, context_lens, tokens_per_block, num_pool_blocks,
                     split_tokens, decode, stream, false);
}

int qvp_pack_ahead(qvp_batch* batch, uint32_t num_seqs, const uint32_t* block_ids, const uint32_t* cu_blocks,
                   const uint32_t* context_lens, uint32_t tokens_per_block, uint32_t num_pool_blocks,
                   uint32_t split_tokens, const qvp_decode_args* decode, void* stream) {
    return pack_impl(batch, num_seqs, block_ids, cu_blocks, context_lens, tokens_per_block, num_pool_blocks,
                     split_tokens, decode, stream, true);
}

int qvp_batch_upload(qvp_batch* batch, void* stream) {
    if (batch == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "batch is NULL");
    if (!batch->valid) return QVP_OK;
    return qvp::flush_own_upload(batch, qvp::as_stream(stream));
}

}  // extern "C"

namespace qvp {

int wait_for_reader(qvp_reader& r, hipStream_t stream, bool may_allocate) {
    if (!r.pending || r.stream == stream) return QVP_OK;
    if (!r.recorded) {
        // The reader's stream has the read enqueued; an event recorded on it
        // now completes after that read (and whatever followed it there).
        // Without an event object and leave to create one, the host waits
        // for that stream instead.
        if (r.event == nullptr && !may_allocate) {
            QVP_HIP(hipStreamSynchronize(r.stream));
            r.pending = false;
            return QVP_OK;
        }
        if (r.event == nullptr) QVP_HIP(hipEventCreateWithFlags(&r.event, hipEventDisableTiming));
        QVP_HIP(hipEventRecord(r.event, r.stream));
        r.recorded = true;
    }
    QVP_HIP(hipStreamWaitEvent(stream, r.event, 0));
    return QVP_OK;
}

int note_reader(qvp_reader& r, hipStream_t stream, hipStream_t writer, bool may_allocate) {
    // Work captured into a graph reads the buffers whenever the graph is
    // replayed, which no event can stand for; graphs are valid until the
    // pack after next (see qvp_graph_begin_capture).
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    QVP_HIP(hipStreamIsCapturing(stream, &capture));
    if (capture != hipStreamCaptureStatusNone) return QVP_OK;
    r.stream = stream;
    r.pending = true;
    r.recorded = false;
    // Read on another stream than the buffer's writer (an upload pipelined
    // beside the decodes): the event is recorded right after the read, so
    // the next write waits for exactly this read, not for later work on the
    // reader's stream. Reads on the writer's own stream (the one-stream
    // engine loop) record nothing: an event between back-to-back kernels
    // stalls the second one.
    // (Without an event object and leave to create one, the writer records
    // one on this stream when it comes.)
    if (stream != writer && (r.event != nullptr || may_allocate)) {
        if (r.event == nullptr) QVP_HIP(hipEventCreateWithFlags(&r.event, hipEventDisableTiming));
        QVP_HIP(hipEventRecord(r.event, stream));
        r.recorded = true;
    }
    return QVP_OK;
}

void destroy_reader(qvp_reader& r) {
    if (r.event != nullptr) (void)hipEventDestroy(r.event);
    r = qvp_reader{};
}

}  // namespace qvp

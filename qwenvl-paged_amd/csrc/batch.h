// Internal definition of qvp_batch, shared by the packer and the decode
// launcher (the decode caches its work schedule in the batch it runs on).
#pragma once

#include "common.h"

#include <vector>

// One contiguous run of 32-token tiles of one (sequence, kv head) segment that
// a persistent decode workgroup processes: tiles [t0, t1) of segment (b, g),
// whose sequence holds ctx tokens. A piece that is not the whole segment owns
// workspace slot `slot`; the segment's slots are [seg_slot0, seg_slot0 +
// seg_nslots) and counters[seg_slot0] counts the pieces that have finished.
struct qvp_piece {
    int32_t b, g, t0, t1, ctx, slot, seg_slot0, seg_nslots;
};

// A shared-prefix work item of the persistent decode: tiles [t0, t1) of kv
// head g for the nmem sequences of one MFMA column block whose block tables
// hold the same frames over those tiles (member b[0]'s table supplies them),
// decoded once for all of them; member m's own tiles [t1, sfx_t1[m]) (a short
// private suffix, context ctx[m]) run in the item too. With slot[m] = -1 the
// item completes member m's (sequence, kv head) segment and writes its
// output; otherwise its partial result goes to workspace slot slot[m] of the
// segment's nslots[m] slots, whose completion counter is
// counters[seg_slot0[m]]. The segment's other slots are the prefix's other
// chunks and, for a long private suffix, ordinary pieces of the main launch.
constexpr int kPrefixMaxMembers = 8;
struct qvp_prefix_item {
    int32_t g, t0, t1, nmem;
    int32_t b[kPrefixMaxMembers];
    int32_t ctx[kPrefixMaxMembers];
    int32_t sfx_t1[kPrefixMaxMembers];  // end of the member's private tiles run by the item (t1: none)
    int32_t slot[kPrefixMaxMembers];    // -1: the item completes the member's segment
    int32_t seg_slot0[kPrefixMaxMembers];
    int32_t nslots[kPrefixMaxMembers];
};

// The last enqueued consumer of a device buffer: its stream, and an event
// recorded right after the read when it ran beside the buffer's writer. A
// writer on another stream waits for that event on the device (recording one
// on the reader's stream first when none was needed then; that stream must
// still exist).
struct qvp_reader {
    hipEvent_t event{nullptr};
    hipStream_t stream{nullptr};
    bool pending{false};
    bool recorded{false};  // event already marks the read
};

// Balanced schedule of the persistent MFMA decode for one packed batch and one
// kv-head count. Device layout (int32 units, each array 256-byte aligned):
//   wg_begin[num_wgs + 1]  CSR over pieces per workgroup
//   pieces[num_pieces]     qvp_piece
//   counters[num_slots]    completion counters (zero between launches)
//   first[num_wgs][8][8]   per wave: its first tile (piece, tile, kv head, the
//                          two block ids; piece -1 when it has none) and the
//                          workgroup's piece range (begin, end)
//   prefix[num_prefix_items] qvp_prefix_item (shared-prefix launch)
//   suffix[num_suffix]     qvp_piece: short private suffixes of prefix-group
//                          members, decoded by the shared-prefix launch
struct qvp_schedule {
    bool valid{false};
    // Device words of the schedule in use: either the batch's packed buffer
    // (built with the pack) or this schedule's own buffer (built at decode).
    int32_t* words{nullptr};
    bool in_pack_buffer{false};
    // Host plan between planning and writing: per-workgroup piece CSR and pieces.
    std::vector<int32_t> plan_wg_begin;
    std::vector<qvp_piece> plan_pieces;
    std::vector<qvp_prefix_item> plan_prefix;
    std::vector<qvp_piece> plan_suffix;
    uint64_t pack_generation{0};
    uint32_t num_kv_heads{0};
    uint32_t group{0};  // query heads per kv head (sizes the deferred LDS and the slots)
    uint32_t max_wgs{0};
    uint32_t num_wgs{0};
    uint32_t num_pieces{0};
    uint32_t num_slots{0};
    uint32_t max_partial_pieces_per_wg{0};
    uint32_t hps{1};  // kv heads per segment
    uint32_t tile_group{0};  // DecodeGeometry::tile_group the LDS budget was planned for
    uint32_t kv_elem{0};     // DecodeGeometry::kv_elem (only bf16 caches plan shared prefixes)
    uint32_t partition_tiles{0};  // ranges cut only at multiples of this many tiles of a sequence (0: anywhere)
    std::vector<double> weights;  // streaming weight per kv-head group the ranges were cut for
    bool defer{false};            // piece results held in LDS until a range is done
    uint32_t lds_bytes{0};        // dynamic LDS per workgroup for them
    // What the plan was made from besides the geometry fields above: tiles
    // per sequence and the shared-prefix groups found (members, shared
    // tiles). A batch with the same key gets the same plan but for the
    // context lengths it records (qvp_piece::ctx, qvp_prefix_item::ctx).
    bool key_valid{false};
    std::vector<uint32_t> key_tiles;
    std::vector<uint32_t> key_groups;
    // Shared prefixes decoded once for their sequences (a launch before the
    // main one): work items and the sequence groups they came from.
    uint32_t num_prefix_items{0};
    uint32_t num_suffix{0};  // entries of the suffix list (eight per workgroup of that launch)
    uint32_t prefix_groups{0};
    size_t off_wg_begin{0}, off_pieces{0}, off_counters{0}, off_first{0}, off_prefix{0}, off_suffix{0},
        total{0};  // int32 units
    // Two pinned staging buffers, used in turn: rebuilding the schedule for
    // step n + 1 waits only for the upload of the rebuild before last, which
    // the stream reaches once step n - 1's decode is done, so the host can
    // prepare the next step while the current one runs.
    int32_t* staging[2]{nullptr, nullptr};
    size_t staging_cap[2]{0, 0};
    hipEvent_t staging_done[2]{nullptr, nullptr};
    bool staging_pending[2]{false, false};
    int staging_slot{0};
    int32_t* device{nullptr};
    size_t device_cap{0};
    qvp_reader reader;  // last decode that read `device`
};

// Work list of a causal prefill over one packed batch (rebuilt per call: the
// first new position of each sequence is a call argument), and the private
// per-position batch of the prefill's decode-kernel path.
struct qvp_prefill_plan {
    int32_t* staging{nullptr};
    size_t staging_cap{0};  // int32 elements
    hipEvent_t staging_done{nullptr};
    bool staging_pending{false};
    int32_t* device{nullptr};
    size_t device_cap{0};
    qvp_batch* virt{nullptr};
};

// A packed batch. Packs alternate between two slots, each a pinned staging
// buffer and a device buffer (the packed arrays, then optionally the decode
// schedule built with them): packing step n + 1 neither waits for step n's
// upload on the host nor overwrites the arrays step n's decode reads.
struct qvp_batch {
    int32_t* staging[2]{nullptr, nullptr};
    size_t staging_cap[2]{0, 0};  // in int32 elements
    hipEvent_t staging_done[2]{nullptr, nullptr};
    bool staging_pending[2]{false, false};
    int parity{0};                 // slot the next pack fills
    int current{0};                // slot of the last successful pack
    int32_t* device[2]{nullptr, nullptr};
    size_t device_cap[2]{0, 0};    // in int32 elements
    qvp_reader readers[2];         // last decode / prefill that read each slot
    hipStream_t upload_stream[2]{nullptr, nullptr};  // stream of each slot's upload
    // A pack made with qvp_pack_ahead whose upload has not been enqueued yet:
    // its bytes wait in staging[slot] until a decode on upload_stream[slot]
    // carries them, or the batch's own decode / prefill / qvp_batch_upload
    // enqueues them.
    bool upload_pending[2]{false, false};
    size_t upload_bytes[2]{0, 0};
    bool valid{false};
    uint64_t generation{0};            // bumped by every successful pack
    // Partition of the split-K cuts the caller asked for, in 32-token tiles (0:
    // none given -- the persistent kernel then cuts its ranges anywhere).
    uint32_t partition_tiles{0};
    std::vector<int32_t> host_seq_lens;  // host copy of seq_lens for scheduling
    std::vector<uint32_t> host_ids;      // host copy of the needed block ids, CSR over host_cu_blocks
    std::vector<uint32_t> host_cu_blocks;
    // Scratch of a pack that plans a schedule before the batch is replaced.
    std::vector<int32_t> lens_scratch;
    std::vector<uint32_t> ids_scratch;
    std::vector<uint32_t> cu_scratch;
    qvp_packed_view view{};
    qvp_decode_plan last_plan{};       // what the last decode on this pack ran (reset by qvp_pack)
    qvp_schedule sched{};
    qvp_prefill_plan prefill{};
};

namespace qvp {
// A pack's upload taken over by a decode launch: 16-byte words src -> dst
// (src is the device mapping of the pinned staging), then `tail` 4-byte
// words after them.
struct PendingUpload {
    qvp_batch* batch{nullptr};
    int slot{0};
    const void* src{nullptr};
    void* dst{nullptr};
    size_t n16{0};
    uint32_t tail{0};
};
// Enqueues the batch's own pending upload (its current pack) on `stream`,
// after the slot's previous reader when that ran on another stream. Without
// may_allocate no event object is created (the host waits instead).
int flush_own_upload(qvp_batch* batch, hipStream_t stream, bool may_allocate = true);
// Takes one pending upload registered on `stream` by a batch other than
// `exclude`; returns false when there is none. The caller enqueues the copy
// and then calls finish_taken_upload on the same stream.
bool take_pending_upload(hipStream_t stream, const qvp_batch* exclude, PendingUpload* out);
int finish_taken_upload(const PendingUpload& u, hipStream_t stream);
// Makes `stream` wait on the device for a buffer's last reader when that
// reader was enqueued on another stream. Without may_allocate no event object
// is created: the host then waits for the reader's stream.
int wait_for_reader(qvp_reader& r, hipStream_t stream, bool may_allocate = true);
// Records `stream` as a buffer's last reader (call after its kernels);
// `writer` is the stream that wrote the buffer. Without may_allocate no event
// object is created.
int note_reader(qvp_reader& r, hipStream_t stream, hipStream_t writer, bool may_allocate = true);
void destroy_reader(qvp_reader& r);
// Frees the schedule's buffers (called by qvp_batch_destroy).
void destroy_schedule(qvp_schedule& s);
// Frees the prefill plan's buffers and its private batch.
void destroy_prefill_plan(qvp_prefill_plan& p);
}  // namespace qvp

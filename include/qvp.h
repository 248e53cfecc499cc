/*
 * qvp.h - C ABI of the MI355X (gfx950) paged-KV hot path.
 *
 * This is the drop-in boundary below the C++17 host API (allocator, cache
 * manager, scheduler). Everything crossing it is a plain pointer, an integer
 * or a float; there are no C++ types, no exceptions and no torch types.
 *
 * Reference interfaces each group of entry points replaces (paths relative to
 * the QwenVL-Paged source tree):
 *   block pool        include/qwenvl_paged/Block.h:59-70,99-166 (PhysicalBlock
 *                     storage, HostMemoryOptions), src/Block.cpp:21-44
 *                     (alignment rounding), src/MemoryAllocator.cpp:8-26
 *   ragged pack       docs/architecture.md:117-120 (flatten BlockTable::entries()
 *                     into [num_seqs, max_blocks_per_seq]),
 *                     include/qwenvl_paged/PagedAttention.h:15-22 (per-sequence
 *                     context lengths), src/KVCacheManager.cpp:11-25 (unmapped or
 *                     swapped blocks fault)
 *   paged decode      include/qwenvl_paged/PagedAttention.h:53-127
 *                     (paged_attention_decode<T>)
 *   copy-on-write     include/qwenvl_paged/MemoryAllocator.h:116,
 *                     src/MemoryAllocator.cpp:76-85 (copy_block)
 *   swap              include/qwenvl_paged/SwapBackend.h:27-57,
 *                     src/SwapBackend.cpp:10-43 (store/load of whole blocks)
 *   K/V append        tests/PagedAttention.test.cpp:97-127, tests/EndToEnd.test.cpp:157-179
 *   causal prefill    include/qwenvl_paged/PagedAttention.h:43-44 (decode per
 *                     prompt position with context_len = p + 1)
 *   M-RoPE positions  include/qwenvl_paged/KVCacheManager.h:23-78
 *                     (PositionalEncodingSpan metadata)
 *
 * Conventions
 *   - Every entry point returns a qvp_status; QVP_OK is 0. On any other value
 *     nothing was enqueued and no output was touched (the reference's
 *     "return false without touching out", PagedAttention.h:50-51,73-89).
 *     qvp_last_error() returns a thread-local message for the last failure.
 *   - `stream` arguments are hipStream_t values passed as void*; NULL is the
 *     legacy default stream. Work is asynchronous unless stated otherwise.
 *   - Not thread-safe per object: one engine thread drives a pool and a batch,
 *     as the reference's single engine loop does (docs/architecture.md:70-83).
 */
#ifndef QVP_H
#define QVP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Status and element types                                                 */
/* ------------------------------------------------------------------------ */

typedef enum qvp_status {
    QVP_OK = 0,
    /* Shapes, sizes or dtypes are inconsistent (PagedAttention.h:59-68). */
    QVP_ERR_INVALID_ARGUMENT = 1,
    /* A block the call needs is unmapped, swapped out or not in the pool
     * (PagedAttention.h:73-89, KVCacheManager.cpp:11-25). */
    QVP_ERR_UNMAPPED = 2,
    /* Device or pinned-host memory could not be allocated. */
    QVP_ERR_OUT_OF_MEMORY = 3,
    /* A caller-supplied buffer is smaller than the call needs. */
    QVP_ERR_CAPACITY = 4,
    /* A HIP runtime call failed; qvp_last_error() names it. */
    QVP_ERR_DEVICE = 5
} qvp_status;

typedef enum qvp_dtype {
    QVP_DTYPE_F32 = 0,
    QVP_DTYPE_BF16 = 1,
    QVP_DTYPE_F16 = 2
} qvp_dtype;

/* Block-table value for a logical block that has no resident frame (never
 * mapped, or swapped out: BlockTable.h:18-24). Packing refuses it. */
#define QVP_UNMAPPED_BLOCK 0xFFFFFFFFu

/* Returns the message of the last failure on the calling thread ("" if none). */
const char* qvp_last_error(void);
/* Returns a static name for a status value. */
const char* qvp_status_name(int status);
/* Returns the library version as major*10000 + minor*100 + patch. */
int qvp_version(void);

/* ------------------------------------------------------------------------ */
/* Runtime plumbing. No reference counterpart: these give hosts without a   */
/* device runtime of their own (ctypes, cgo, a bare C++ engine) device      */
/* memory, streams and events.                                              */
/* ------------------------------------------------------------------------ */

int qvp_device_count(int* count);
int qvp_set_device(int device);
int qvp_device_synchronize(void);

int qvp_malloc(void** ptr, size_t bytes);
int qvp_free(void* ptr);
/* Pinned (page-locked) host memory that the device can read and write. */
int qvp_host_alloc(void** ptr, size_t bytes);
int qvp_host_free(void* ptr);
/* Device-side address of pinned host memory from qvp_host_alloc. */
int qvp_host_device_pointer(void** device_ptr, void* host_ptr);

int qvp_memcpy_htod(void* dst, const void* src, size_t bytes, void* stream);
int qvp_memcpy_dtoh(void* dst, const void* src, size_t bytes, void* stream);
int qvp_memcpy_dtod(void* dst, const void* src, size_t bytes, void* stream);
/* Fills device memory with a byte value using a fill kernel (safe inside
 * graph capture, unlike a runtime memset node). */
int qvp_fill_bytes(void* dst, uint8_t value, size_t bytes, void* stream);

int qvp_stream_create(void** stream);
int qvp_stream_destroy(void* stream);
int qvp_stream_synchronize(void* stream);
int qvp_event_create(void** event);
int qvp_event_destroy(void* event);
int qvp_event_record(void* event, void* stream);
int qvp_event_synchronize(void* event);
/* *complete = 1 when all work before the event's last record has finished
 * (or it was never recorded), 0 while it is pending. */
int qvp_event_query(void* event, int* complete);
int qvp_stream_wait_event(void* stream, void* event);
int qvp_event_elapsed_ms(float* ms, void* start, void* stop);

/* HIP graph capture of a stream (thread-local mode). Between begin and end,
 * enqueue only calls that touch nothing on the host per call: qvp_paged_decode
 * on a batch that was already decoded once since its last qvp_pack (its
 * schedule is then cached on the device) with a caller workspace,
 * qvp_append_kv, qvp_copy_blocks, qvp_swap_gather / qvp_swap_scatter,
 * qvp_fill_bytes and device-to-device copies. qvp_pack, qvp_paged_prefill and
 * qvp_mrope_positions upload host-built lists on every call and are not
 * captured. The kernels reset their own merge counters, so a graph may be
 * replayed any number of times; it reads and writes the buffers it was
 * captured with, so a captured decode stays valid until the second qvp_pack
 * after the capture on its batch reuses the packed buffer it reads. */
int qvp_graph_begin_capture(void* stream);
int qvp_graph_end_capture(void* stream, void** graph_exec);
int qvp_graph_launch(void* graph_exec, void* stream);
int qvp_graph_destroy(void* graph_exec);

/* ------------------------------------------------------------------------ */
/* Block pool: the physical KV frames in HBM                                */
/* Replaces per-block std::aligned_alloc storage (Block.h:99-166,           */
/* src/Block.cpp:30-44). Frame i lives at base + i * block_stride, where    */
/* block_stride = round_up(block_bytes, alignment) like PhysicalBlock's     */
/* size_bytes() (src/Block.cpp:30-44; alignment 0 means 256, Block.h:17).   */
/* ------------------------------------------------------------------------ */

typedef struct qvp_pool qvp_pool;

int qvp_pool_create(uint32_t num_blocks, size_t block_bytes, size_t alignment, qvp_pool** pool);
int qvp_pool_destroy(qvp_pool* pool);
void* qvp_pool_base(const qvp_pool* pool);
size_t qvp_pool_block_stride(const qvp_pool* pool);
size_t qvp_pool_block_bytes(const qvp_pool* pool);
uint32_t qvp_pool_num_blocks(const qvp_pool* pool);
/* Device address of one frame, or NULL when block >= num_blocks
 * (MemoryAllocator::block returns nullptr for invalid ids,
 * src/MemoryAllocator.cpp:87-99). */
void* qvp_pool_block_ptr(const qvp_pool* pool, uint32_t block);
/* Host <-> frame byte copies at an offset inside one frame (the host writes
 * the reference tests make through PhysicalBlock::data(),
 * tests/PagedAttention.test.cpp:97-127). Asynchronous on `stream`; the host
 * buffer must stay valid until the stream reaches the copy. */
int qvp_pool_write(qvp_pool* pool, uint32_t block, size_t offset, const void* src, size_t bytes,
                   void* stream);
int qvp_pool_read(const qvp_pool* pool, uint32_t block, size_t offset, void* dst, size_t bytes,
                  void* stream);

/* ------------------------------------------------------------------------ */
/* Ragged-batch packing (docs/architecture.md:117-120)                      */
/* ------------------------------------------------------------------------ */

typedef struct qvp_batch qvp_batch;

/* Device-side arrays of the last successful qvp_pack on a batch.
 *   block_tables  int32 [num_seqs][max_blocks_per_seq], row b holds the frames
 *                 of logical blocks 0..ceil(seq_lens[b]/tokens_per_block)-1 in
 *                 logical order, padded with -1
 *   seq_lens      int32 [num_seqs]
 *   cu_seqlens    int32 [num_seqs + 1], exclusive prefix sum of seq_lens
 *   cu_splits     int32 [num_seqs + 1], exclusive prefix sum of each
 *                 sequence's split count ceil(seq_lens[b] / split_tokens)
 *   split_seq     int32 [num_splits], sequence of each split
 *   split_start   int32 [num_splits], first token of each split             */
typedef struct qvp_packed_view {
    const int32_t* block_tables;
    const int32_t* seq_lens;
    const int32_t* cu_seqlens;
    const int32_t* cu_splits;
    const int32_t* split_seq;
    const int32_t* split_start;
    uint32_t num_seqs;
    uint32_t max_blocks_per_seq;
    uint32_t num_splits;
    uint32_t split_tokens;
    uint32_t tokens_per_block;
    uint32_t num_pool_blocks;
    uint32_t max_seq_len;
    uint64_t total_tokens;
} qvp_packed_view;

int qvp_batch_create(qvp_batch** batch);
int qvp_batch_destroy(qvp_batch* batch);

/* Packs a ragged batch given in CSR form: sequence b owns
 * block_ids[cu_blocks[b] .. cu_blocks[b+1]) in logical-block order (what
 * BlockTable::entries() lists, BlockTable.h:105-108) and has context_lens[b]
 * committed tokens. A sequence needs its first ceil(context_lens[b] /
 * tokens_per_block) entries; each must be < num_pool_blocks and not
 * QVP_UNMAPPED_BLOCK. The whole batch is validated before anything is written,
 * so a refused call (QVP_ERR_INVALID_ARGUMENT for context_len == 0 or too few
 * mapped blocks, QVP_ERR_UNMAPPED for a missing frame) leaves the batch's
 * previous contents intact (PagedAttention.h:73-89).
 * split_tokens (0 selects 512) is rounded up to a multiple of 128: the
 * split-K partition (flash-decoding style) of the fp32 and generic decode
 * kernels. The persistent bf16 kernel balances its work in ranges of 32-token
 * tiles cut by cost; when split_tokens is given (non-zero) its ranges are
 * cut only at multiples of split_tokens inside a sequence (or at sequence
 * ends), so every cross-workgroup merge joins whole partitions; with 0 its
 * cuts are free.
 * The arrays are staged in pinned memory and uploaded by one kernel on
 * `stream`. Packs alternate between two device buffers: the arrays of pack n
 * stay valid until pack n + 2, so pack n + 1 may be enqueued on another
 * stream while pack n's decode still runs (the caller makes the decode's
 * stream wait for the pack's). Decodes and prefills enqueued through this
 * library are tracked: pack n + 2 waits on the device for them, whatever
 * stream they ran on. Other readers of qvp_batch_view's pointers must be
 * ordered before pack n + 2 by the caller. */
int qvp_pack(qvp_batch* batch, uint32_t num_seqs, const uint32_t* block_ids,
             const uint32_t* cu_blocks, const uint32_t* context_lens, uint32_t tokens_per_block,
             uint32_t num_pool_blocks, uint32_t split_tokens, void* stream);
int qvp_batch_view(const qvp_batch* batch, qvp_packed_view* view);

/* ------------------------------------------------------------------------ */
/* Paged decode (include/qwenvl_paged/PagedAttention.h:53-127)              */
/* ------------------------------------------------------------------------ */

/* One decode step for every sequence of a packed batch: for each sequence b
 * and query head h, with g = h / (num_query_heads / num_kv_heads),
 *   out[b][h][:] = sum_t w_t * V[b][t][g][:] / sum_t w_t,
 *   w_t = exp(s_t - max_t s_t),  s_t = scale * <query[b][h][:], K[b][t][g][:]>
 * over t < seq_lens[b], with fp32 accumulation (PagedAttention.h:94-124).
 * K and V of token t of sequence b live in frame block_tables[b][t / tpb] at
 * element offset layer * layer_stride + {0 | stream_stride} +
 * (t % tpb) * token_stride + g * head_stride (CacheLayout.cpp:25-38); head_dim
 * elements are contiguous. */
/* Arithmetic of the persistent bf16 decode's 32-token tiles. No reference
 * counterpart (the reference's decode is a scalar loop, PagedAttention.h:
 * 94-124): both engines read each K/V byte once per GQA group. */
typedef enum qvp_tile_engine {
    QVP_TILE_AUTO = 0,    /* the library's choice for the query group */
    QVP_TILE_MATRIX = 1,  /* matrix cores: v_mfma_f32_16x16x32_bf16, the group in the columns */
    QVP_TILE_VECTOR = 2   /* vector ALUs: the group folded into each lane's fp32 dot
                             products (groups of at most 2; refused otherwise) */
} qvp_tile_engine;

typedef struct qvp_decode_args {
    const void* query;          /* device, [num_seqs][num_query_heads][head_dim], kv_dtype */
    void* out;                  /* device, [num_seqs][num_query_heads][head_dim], out_dtype */
    const void* kv_base;        /* device address of frame 0 */
    uint64_t block_stride;      /* bytes between frames */
    const qvp_batch* batch;     /* packed by qvp_pack for this pool */
    uint32_t kv_dtype;          /* qvp_dtype of query and cache elements */
    uint32_t out_dtype;         /* qvp_dtype of out */
    uint32_t layer;
    uint32_t num_layers;
    uint32_t num_query_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t tokens_per_block;
    uint64_t head_stride;       /* elements, KVBlockLayout::head_stride() */
    uint64_t token_stride;      /* elements, KVBlockLayout::token_stride() */
    uint64_t stream_stride;     /* elements, KVBlockLayout::stream_stride() */
    uint64_t layer_stride;      /* elements, KVBlockLayout::layer_stride() */
    float scale;
    void* workspace;            /* device scratch for split partials, or NULL */
    uint64_t workspace_bytes;   /* size of workspace; ignored when it is NULL */
    void* split_event;          /* optional hipEvent_t recorded on `stream` after the
                                   split kernel and before the merge kernel (lets a
                                   caller time the two kernels apart), or NULL */
    uint32_t tile_engine;       /* qvp_tile_engine of the persistent bf16 kernel;
                                   0 (automatic) for the library's choice */
} qvp_decode_args;

/* Bytes of workspace qvp_paged_decode needs for this batch and head shape. */
int qvp_decode_workspace_bytes(const qvp_batch* batch, uint32_t num_query_heads,
                               uint32_t head_dim, uint64_t* bytes);
/* Validates everything on the host, then enqueues the split-K decode kernel
 * and the split-merge kernel on `stream`. With workspace == NULL the library
 * uses a per-device workspace it grows on demand. */
int qvp_paged_decode(const qvp_decode_args* args, void* stream);

/* qvp_pack, plus the work schedule of the decode the pack is for, built now
 * and uploaded with the packed arrays in the same single upload (a later
 * qvp_paged_decode with the same query-head count, kv-head count and cache
 * layout finds it ready and enqueues only its kernel; a decode with other
 * arguments builds its own). `decode` describes that decode exactly as
 * qvp_paged_decode will receive it; its `batch` field is ignored and it is
 * validated by the same rules (a refusal packs nothing). NULL is qvp_pack.
 * A decode the persistent MFMA kernel does not run needs no schedule: the
 * pack then equals qvp_pack. No reference counterpart: the reference
 * resolves blocks per token inside paged_attention_decode
 * (PagedAttention.h:73-89); this moves a step's host work and its upload
 * into the pack. */
int qvp_pack_for_decode(qvp_batch* batch, uint32_t num_seqs, const uint32_t* block_ids,
                        const uint32_t* cu_blocks, const uint32_t* context_lens, uint32_t tokens_per_block,
                        uint32_t num_pool_blocks, uint32_t split_tokens, const qvp_decode_args* decode,
                        void* stream);

/* qvp_pack_for_decode with its upload left pending: the packed arrays and
 * schedule wait in the batch's pinned staging, and the next qvp_paged_decode
 * of ANOTHER batch enqueued on `stream` that runs the persistent bf16 kernel
 * copies them in extra workgroups of its own launch, which get a CU only as
 * that decode's workgroups finish (so the upload runs in the launch's tail
 * instead of as a kernel of its own between two decodes). A decode or
 * prefill of this batch itself, or qvp_batch_upload, enqueues the upload
 * first if it is still pending; a later pack of this batch discards it. For
 * an engine that packs step n + 1 on one batch object while step n decodes
 * from another (two batches used in turn). Until the upload is enqueued the
 * device arrays of qvp_batch_view hold the previous pack's contents. A
 * decode under graph capture carries no pending upload and refuses a batch
 * whose own upload is pending. No reference counterpart (the reference resolves blocks per token,
 * PagedAttention.h:73-89). */
int qvp_pack_ahead(qvp_batch* batch, uint32_t num_seqs, const uint32_t* block_ids, const uint32_t* cu_blocks,
                   const uint32_t* context_lens, uint32_t tokens_per_block, uint32_t num_pool_blocks,
                   uint32_t split_tokens, const qvp_decode_args* decode, void* stream);
/* Enqueues on `stream` the upload a qvp_pack_ahead of this batch left
 * pending (nothing to do otherwise). */
int qvp_batch_upload(qvp_batch* batch, void* stream);

/* qvp_paged_decode for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation). No
 * counterpart in the reference. It calls no hipMalloc, hipHostMalloc,
 * hipFree or other allocating routine: the workspace is a fixed device array
 * of 16 MiB that the library reserves in every device's memory when it loads
 * (held until the process ends), so args->workspace must be NULL, and a
 * decode needing more workspace (e.g. a bf16 config2 batch needs 1.7 MB) is
 * refused with QVP_ERR_CAPACITY. When the bf16 MFMA kernel runs the decode,
 * the batch must already hold its work schedule (packed with
 * qvp_pack_for_decode for this decode, or decoded once by qvp_paged_decode
 * since its last pack), or buffers large enough to rebuild it; otherwise the
 * call is refused with QVP_ERR_CAPACITY before anything is enqueued. Every
 * call on a device shares that device's array: calls that overlap on one
 * device (e.g. on two streams) race and must be ordered by the caller. The
 * array needs no initial contents: every word the kernels read was written
 * earlier in the same call (with shared prefixes, the prefix launch writes
 * slots the main launch then reads; the two run back to back on the stream,
 * so another call on the device must not be enqueued between them, i.e. the
 * caller orders whole calls). */
int qvp_paged_decode_noalloc(const qvp_decode_args* args, void* stream);

/* The work decomposition of the last qvp_paged_decode enqueued on a batch.
 * No reference counterpart (the reference decodes one sequence at a time,
 * PagedAttention.h:53-127): it tells benchmarks and tests which kernel ran
 * and how the batch was divided. */
typedef enum qvp_decode_kernel {
    QVP_DECODE_NONE = 0,        /* nothing decoded since the last qvp_pack */
    QVP_DECODE_MFMA = 1,        /* persistent bf16 MFMA kernel, cost-balanced tile ranges */
    QVP_DECODE_F32_GROUPED = 2, /* fp32 MFMA kernel over split_tokens partitions + merge */
    QVP_DECODE_GENERIC = 3,     /* VALU kernel per query head over split_tokens partitions + merge */
    QVP_DECODE_GROUPED = 4,     /* VALU kernel per kv head (GQA group folded) over split_tokens partitions + merge */
    QVP_DECODE_SPLIT_MFMA = 5   /* bf16/fp16 MFMA kernel per kv head at head_dim 64 over split_tokens partitions + merge */
} qvp_decode_kernel;

typedef struct qvp_decode_plan {
    uint32_t kernel;            /* qvp_decode_kernel */
    uint32_t workgroups;        /* workgroups of the decode kernel */
    uint32_t pieces;            /* MFMA: (sequence, kv-head group, tile range) pieces;
                                   split kernels: token partitions */
    uint32_t slots;             /* partial results merged through the workspace */
    uint32_t kv_heads_per_segment; /* MFMA: kv heads one workgroup decodes side by side */
    uint32_t split_tokens;      /* split kernels: tokens per partition; MFMA: the
                                   partition its range cuts were held to (the pack's
                                   split_tokens when the caller gave one), 0 when the
                                   ranges were cut by cost alone */
    uint32_t deferred_results;  /* MFMA: 1 when piece results wait in LDS until a range ends */
    uint32_t query_group;       /* query heads per kv head of that decode */
    uint32_t tile_engine;       /* MFMA kernel: the qvp_tile_engine that ran (1 or 2) */
    uint32_t shared_prefix_groups; /* MFMA kernel: groups of sequences whose common leading
                                      frames were decoded once for the whole group */
    uint32_t shared_prefix_items;  /* MFMA kernel: work items of that shared-prefix launch */
} qvp_decode_plan;

int qvp_decode_plan_info(const qvp_batch* batch, qvp_decode_plan* plan);

/* ------------------------------------------------------------------------ */
/* Causal paged prefill (PagedAttention.h:43-44: paged_attention_decode<T>  */
/* applied per prompt position p with context_len = p + 1)                  */
/* ------------------------------------------------------------------------ */

/* The new tokens of sequence b are positions q_start[b] .. seq_lens[b] - 1 of
 * the packed batch (their K/V already written, e.g. by qvp_append_kv); their
 * queries and outputs are rows cu_q[b] .. cu_q[b + 1] - 1, with cu_q the
 * exclusive prefix sum of seq_lens[b] - q_start[b]. For each such position p
 * and query head h, with g = h / (num_query_heads / num_kv_heads):
 *   out[row(p)][h][:] = sum_{t <= p} w_t V[b][t][g][:] / sum_{t <= p} w_t,
 *   w_t = exp(s_t - max s),  s_t = scale * <query[row(p)][h][:], K[b][t][g][:]>,
 * i.e. exactly the decode of that position with context p + 1. */
typedef struct qvp_prefill_args {
    const void* query;          /* device, [total_new][num_query_heads][head_dim], kv_dtype */
    void* out;                  /* device, [total_new][num_query_heads][head_dim], out_dtype */
    const void* kv_base;        /* device address of frame 0 */
    uint64_t block_stride;      /* bytes between frames */
    const qvp_batch* batch;     /* packed by qvp_pack with the full context lengths */
    const uint32_t* q_start;    /* host, [num_seqs]: first new position, < seq_lens[b] */
    uint32_t kv_dtype;
    uint32_t out_dtype;
    uint32_t layer;
    uint32_t num_layers;
    uint32_t num_query_heads;
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t tokens_per_block;
    uint64_t head_stride;       /* elements, KVBlockLayout::head_stride() */
    uint64_t token_stride;      /* elements */
    uint64_t stream_stride;     /* elements */
    uint64_t layer_stride;      /* elements */
    float scale;
} qvp_prefill_args;

/* Validates everything on the host (the decode's rules, plus q_start[b] <
 * seq_lens[b]), then enqueues the prefill on `stream`. bf16 caches with
 * head_dim 128, a positive scale, power-of-two tokens_per_block >= 16, and
 * query, out, kv_base and the strides in bytes all multiples of 16 run the
 * MFMA prefill kernel; everything else runs the decode kernels over one
 * virtual sequence per new position (packed in chunks of at most 2^20 block
 * ids, decoded in order on `stream`). */
int qvp_paged_prefill(const qvp_prefill_args* args, void* stream);

/* ------------------------------------------------------------------------ */
/* Copy-on-write (MemoryAllocator::copy_block, src/MemoryAllocator.cpp:76-85)*/
/* ------------------------------------------------------------------------ */

/* Copies bytes [0, copy_bytes) of frame src_ids[i] onto frame dst_ids[i] for
 * every i in one launch. src_ids/dst_ids are host arrays. Refused when an id is
 * >= num_blocks, copy_bytes > block_stride, a destination repeats, or a
 * destination is another pair's source (the result would depend on order).
 * A pair with src == dst is a no-op. */
int qvp_copy_blocks(void* kv_base, uint64_t block_stride, uint32_t num_blocks,
                    const uint32_t* src_ids, const uint32_t* dst_ids, uint32_t num_pairs,
                    uint64_t copy_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Swap (SwapBackend::store / load, src/SwapBackend.cpp:10-39)              */
/* ------------------------------------------------------------------------ */

/* Swap-out gather: frame frame_ids[i] -> arena + arena_offsets[i], copy_bytes
 * each, in one launch. `arena` is pinned host memory from qvp_host_alloc
 * (its host address); offsets + copy_bytes must lie inside arena_bytes, be
 * 16-byte aligned and not overlap each other. */
int qvp_swap_gather(const void* kv_base, uint64_t block_stride, uint32_t num_blocks,
                    const uint32_t* frame_ids, const uint64_t* arena_offsets, uint32_t count,
                    void* arena, uint64_t arena_bytes, uint64_t copy_bytes, void* stream);
/* Swap-in scatter: arena + arena_offsets[i] -> frame frame_ids[i]. Destination
 * frames must be distinct. */
int qvp_swap_scatter(void* kv_base, uint64_t block_stride, uint32_t num_blocks,
                     const uint32_t* frame_ids, const uint64_t* arena_offsets, uint32_t count,
                     const void* arena, uint64_t arena_bytes, uint64_t copy_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* KV append (tests/PagedAttention.test.cpp:97-127,                         */
/* tests/EndToEnd.test.cpp:157-179)                                         */
/* ------------------------------------------------------------------------ */

/* Pool geometry and source tensors of qvp_append_kv. */
typedef struct qvp_append_args {
    void* kv_base;              /* device address of frame 0 */
    uint64_t block_stride;      /* bytes between frames */
    uint32_t num_blocks;        /* frames in the pool */
    uint32_t kv_dtype;          /* qvp_dtype of the cache and of k / v */
    uint32_t num_layers;        /* layers per frame (BlockShape::num_layers) */
    uint32_t first_layer;       /* layers [first_layer, first_layer + layer_count) */
    uint32_t layer_count;       /*   are written */
    uint32_t num_kv_heads;
    uint32_t head_dim;
    uint32_t tokens_per_block;
    uint64_t head_stride;       /* elements, KVBlockLayout::head_stride() */
    uint64_t token_stride;      /* elements, KVBlockLayout::token_stride() */
    uint64_t stream_stride;     /* elements, KVBlockLayout::stream_stride() */
    uint64_t layer_stride;      /* elements, KVBlockLayout::layer_stride() */
    const void* k;              /* device, [count][layer_count][num_kv_heads][head_dim] */
    const void* v;              /* device, same shape */
} qvp_append_args;

/* For every token i < count and every written layer l, stream s (0 = K from
 * k, 1 = V from v) and kv head h, stores the head_dim elements of the source
 * row at element offset (first_layer + l) * layer_stride + s * stream_stride +
 * slots[i] * token_stride + h * head_stride of frame frames[i]
 * (KVBlockLayout::element_offset, src/CacheLayout.cpp:25-38), which is what the
 * reference's harnesses do element by element after
 * KVCacheManager::ensure_token_writable returned the frame. frames / slots are
 * host arrays (slot = token position % tokens_per_block). Refused before
 * anything is enqueued: a frame >= num_blocks (QVP_ERR_UNMAPPED), a slot >=
 * tokens_per_block, a (frame, slot) pair given twice, more than 2^24 tokens,
 * layers outside num_layers or more than 65535 of them, strides under which two elements coincide or the layout
 * exceeds block_stride (QVP_ERR_INVALID_ARGUMENT). */
int qvp_append_kv(const qvp_append_args* args, const uint32_t* frames, const uint32_t* slots,
                  uint32_t count, void* stream);

/* A copy-on-write step in one launch: qvp_copy_blocks(src_ids, dst_ids,
 * num_pairs, copy_bytes) followed by qvp_append_kv(args, frames, slots, count)
 * on the pool args describes, with the same result bytes. This is the order
 * the reference keeps within a step: KVCacheManager::ensure_token_writable
 * copies a shared block (src/KVCacheManager.cpp:141-150, the memcpy of
 * MemoryAllocator::copy_block, src/MemoryAllocator.cpp:76-85) before the
 * harness stores the token's rows into the new frame
 * (tests/PagedAttention.test.cpp:97-127). Every 16-byte unit of a destination
 * frame is written once, from the appended row it lies in or else from the
 * source frame. Refused before anything is enqueued: everything qvp_append_kv
 * and qvp_copy_blocks refuse, more than 128 copies or 128 tokens, more than
 * 64 tokens per block, frames of 2 GiB or more, K and V tensors of 4 GiB or
 * more, copy_bytes not a multiple of 16, pools, rows or strides not 16-byte
 * aligned, and a token row written into a frame that a copy reads (run the
 * two calls apart for that). A pair with src == dst is a no-op. */
int qvp_copy_append_kv(const qvp_append_args* args, const uint32_t* src_ids, const uint32_t* dst_ids,
                       uint32_t num_pairs, uint64_t copy_bytes, const uint32_t* frames, const uint32_t* slots,
                       uint32_t count, void* stream);

/* ------------------------------------------------------------------------ */
/* M-RoPE positions (PositionalEncodingSpan, KVCacheManager.h:23-78)        */
/* ------------------------------------------------------------------------ */

/* One PositionalEncodingSpan of a sequence. `grid` (the span's temporal,
 * height and width extents) is this build's addition: the reference's span
 * carries origin and stride only, which do not say where an image row ends. */
typedef struct qvp_mrope_span {
    uint32_t start_token;
    uint32_t token_count;
    uint32_t kind;              /* 0 Text1D, 1 Image2D, 2 Video3D */
    uint32_t reserved;          /* 0 */
    int64_t origin[3];          /* temporal, height, width */
    int64_t stride[3];
    int64_t grid[3];            /* extents; Image2D / Video3D only */
} qvp_mrope_span;

/* Host staging and device buffers of the position materialisation. */
typedef struct qvp_mrope qvp_mrope;
int qvp_mrope_create(qvp_mrope** out);
int qvp_mrope_destroy(qvp_mrope* m);

/* Writes the (temporal, height, width) position of tokens [begin[b], end[b])
 * of every sequence b to out (device, int64, [3][total_rows], rows in sequence
 * order, axis-major as a model's position_ids). Token i of a Text1D span is
 * origin + i * stride on each axis; token i of an Image2D / Video3D span with
 * grid (T, H, W) is origin + (i / (H W), (i / W) % H, i % W) * stride per
 * axis; a token no span covers takes 1 + the largest position of any axis of
 * the tokens before it on all three axes (0 for the first token), which is
 * the text / decode continuation of Qwen2-VL's get_rope_index. spans: host,
 * CSR over cu_spans[num_seqs + 1], sorted by start_token within a sequence.
 * Refused before anything is enqueued: overlapping or unsorted spans, an
 * empty span, an unknown kind, a grid whose product is not token_count (or
 * an Image2D grid with T != 1), |origin| or |stride| above 2^24, more than
 * 2^24 sequences, begin[b] > end[b], total_rows != sum(end - begin). */
int qvp_mrope_positions(qvp_mrope* m, const qvp_mrope_span* spans, const uint32_t* cu_spans,
                        const uint32_t* begin, const uint32_t* end, uint32_t num_seqs, int64_t* out,
                        uint64_t total_rows, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QVP_H */

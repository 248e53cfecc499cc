#pragma once
// Physical block pool with reference counts, copy-on-write copies and swap
// (include/qwenvl_paged/MemoryAllocator.h:18-198).
//
// Bookkeeping is the reference's exactly: frames 0..N-1 start on a LIFO free
// list so allocate() hands out N-1 first (src/MemoryAllocator.cpp:13-40),
// release() pushes to the back and advances the generation (:42-60), and
// stats() is a point-in-time snapshot. Not thread-safe: one engine thread
// owns the allocator (docs/architecture.md:70-83).
//
// With BlockPlacement::Device the frames are one HBM allocation (qvp_pool), and
// every byte movement is recorded in an ordered queue instead of being done on
// the spot: copy_block() queues a copy-on-write copy, PinnedSwapBackend queues
// gathers (swap-out) and scatters (swap-in). flush() turns each run of
// non-conflicting operations of one kind into a single launch (copy_blocks on
// the engine stream; swap gathers/scatters on a side stream that waits for the
// engine stream and is waited on by it), so results are ordered exactly as the
// synchronous reference orders them. Everything that reads or writes frames on
// the device (decode, block reads/writes) flushes first.

#include "qwenvl_paged/Block.h"
#include "qwenvl_paged/SwapBackend.h"

#include <array>
#include <cstddef>
#include <cstdint>
#include <deque>
#include <functional>
#include <memory>
#include <optional>
#include <string>
#include <vector>

struct qvp_pool;

namespace qwenvl_paged {

struct AllocatorConfig {
    BlockShape block_shape{};
    HostMemoryOptions memory_options{};
    std::uint32_t max_blocks{0};
    // Additions: where frames live and, for the device, the engine stream
    // (a hipStream_t; nullptr lets the allocator create one).
    BlockPlacement placement{BlockPlacement::Host};
    void* stream{nullptr};
};

struct AllocatorStats {
    std::uint32_t total_blocks{0};
    std::uint32_t free_blocks{0};
    std::uint32_t active_blocks{0};
    std::uint32_t shared_blocks{0};
    // Blocks held by the swap backend; they have no frame (MemoryAllocator.h:32-38).
    std::uint32_t swapped_blocks{0};
    std::size_t bytes_reserved{0};
};

struct PhysicalBlockInfo {
    PhysicalBlockId id{0};
    BlockState state{BlockState::Free};
    std::uint32_t ref_count{0};  // non-atomic, engine thread only
    std::uint64_t generation{0};
};

class MemoryAllocator;

// Policy hook naming a block worth evicting; advisory only (MemoryAllocator.h:60-68).
using EvictionCandidateSelector = std::function<std::optional<PhysicalBlockId>(const MemoryAllocator&)>;

class MemoryAllocator {
public:
    explicit MemoryAllocator(AllocatorConfig config);
    ~MemoryAllocator();
    MemoryAllocator(const MemoryAllocator&) = delete;
    MemoryAllocator& operator=(const MemoryAllocator&) = delete;

    [[nodiscard]] std::optional<PhysicalBlockId> allocate();
    void release(PhysicalBlockId id);
    void retain(PhysicalBlockId id);
    // Copies the whole padded frame (src/MemoryAllocator.cpp:76-85); silent on
    // invalid ids. Device placement: queued, executed by flush().
    void copy_block(PhysicalBlockId source, PhysicalBlockId destination);

    [[nodiscard]] PhysicalBlock* block(PhysicalBlockId id) noexcept;
    [[nodiscard]] const PhysicalBlock* block(PhysicalBlockId id) const noexcept;
    [[nodiscard]] const PhysicalBlockInfo* info(PhysicalBlockId id) const noexcept;

    // Non-owning; the backend must outlive the allocator (MemoryAllocator.h:133-139),
    // except a PinnedSwapBackend, which is built on a device allocator and
    // detaches itself when destroyed first.
    void set_swap_backend(SwapBackend* backend) noexcept;
    void detach_swap_backend(const SwapBackend* backend) noexcept;
    [[nodiscard]] std::optional<SwapSlotId> swap_out(PhysicalBlockId id);
    [[nodiscard]] std::optional<PhysicalBlockId> swap_in(SwapSlotId slot);
    void discard_swapped(SwapSlotId slot);

    void set_eviction_selector(EvictionCandidateSelector selector);
    [[nodiscard]] std::optional<PhysicalBlockId> select_eviction_candidate() const;

    [[nodiscard]] AllocatorStats stats() const noexcept;
    [[nodiscard]] bool can_allocate(std::uint32_t block_count) const noexcept;

    // ---- Device placement -------------------------------------------------
    [[nodiscard]] BlockPlacement placement() const noexcept;
    // False when a device allocator could not create its pool or streams.
    [[nodiscard]] bool ok() const noexcept;
    [[nodiscard]] const std::string& last_error() const noexcept;
    [[nodiscard]] void* stream() const noexcept;       // engine stream (hipStream_t)
    [[nodiscard]] void* side_stream() const noexcept;  // swap stream (hipStream_t)
    [[nodiscard]] void* device_base() const noexcept;  // frame 0
    [[nodiscard]] std::size_t block_stride() const noexcept;
    // Runs every queued device operation in order; false on a device error.
    bool flush();
    // flush(), except that a last batch of copies -- at most max_pairs, none
    // reading a frame listed in `written` -- is not launched but handed to the
    // caller (sources in src, destinations in dst, empty when there is none)
    // to run in its own launch on the engine stream, which is already ordered
    // after any swap touching those frames. The handed-out batch counts in
    // copy_launches().
    bool flush_except_last_copies(std::size_t max_pairs, const std::vector<PhysicalBlockId>& written,
                                  std::vector<PhysicalBlockId>& src, std::vector<PhysicalBlockId>& dst);
    // Operations queued and not yet flushed.
    [[nodiscard]] std::size_t pending_operations() const noexcept;
    // Launches issued by flush() so far, by kind (copy, gather, scatter).
    [[nodiscard]] std::uint64_t copy_launches() const noexcept;
    [[nodiscard]] std::uint64_t swap_launches() const noexcept;
    // Swap batches known to have finished (every one after synchronize()):
    // their GPU time on the side stream, start to end of each batch, and the
    // bytes they moved.
    [[nodiscard]] double swap_gpu_ms() const noexcept;
    [[nodiscard]] std::uint64_t swap_bytes_moved() const noexcept;
    // Flush, then copy host bytes into / out of a frame and wait for the copy.
    bool write_block_bytes(PhysicalBlockId id, std::size_t offset, const void* src, std::size_t bytes);
    bool read_block_bytes(PhysicalBlockId id, std::size_t offset, void* dst, std::size_t bytes);
    // Flush, then wait until the engine and side streams are idle.
    bool synchronize();

    // Used by PinnedSwapBackend to record its byte movements in order.
    void enqueue_swap_gather(PhysicalBlockId frame, void* arena, std::size_t arena_bytes, std::size_t offset);
    void enqueue_swap_scatter(PhysicalBlockId frame, void* arena, std::size_t arena_bytes, std::size_t offset);

    // Swap traffic runs on the side stream without holding up the engine
    // stream; work the engine stream enqueues next must be ordered after the
    // swaps it depends on. Call (after flush()) before enqueuing engine work
    // that reads these frames (waits for scatters into them) or writes them
    // (waits for gathers out of them and scatters into them). Only the batches
    // still running are waited for, on the device.
    bool order_frame_reads(const std::vector<PhysicalBlockId>& frames);
    bool order_frame_writes(const std::vector<PhysicalBlockId>& frames);

private:
    enum class OpKind : std::uint8_t { Copy, Gather, Scatter };
    struct DeviceOp {
        OpKind kind;
        PhysicalBlockId frame_a;  // copy source / gather frame / scatter frame
        PhysicalBlockId frame_b;  // copy destination
        void* arena;
        std::size_t arena_bytes;
        std::size_t offset;
    };

    // A swap batch on the side stream: its sequence number and the event
    // recorded after it.
    struct SwapBatchEvent {
        std::uint64_t epoch;
        void* start;  // recorded on the side stream right before the launch
        void* event;  // recorded right after it
        std::uint64_t bytes;
    };

    bool fail(const std::string& what);
    bool run_batch(OpKind kind, const std::vector<DeviceOp>& ops);
    // flush() with an optional hand-out of the last copy batch.
    bool flush_queue(std::size_t max_pairs, const std::vector<PhysicalBlockId>* written,
                     std::vector<PhysicalBlockId>* src, std::vector<PhysicalBlockId>* dst);
    void set_ref_count(PhysicalBlockInfo& info, std::uint32_t count) noexcept;
    // Makes the engine stream wait for the swap batches the frames depend on.
    bool order_engine_after_swaps(const PhysicalBlockId* frames, std::size_t n, bool writes);
    // Drops finished swap batches from the front of swap_events_.
    bool retire_swap_batches();

    AllocatorConfig config_{};
    std::vector<std::unique_ptr<PhysicalBlock>> blocks_;
    std::vector<PhysicalBlockInfo> infos_;
    std::vector<PhysicalBlockId> free_list_;
    std::array<std::uint32_t, 4> state_counts_{};  // blocks per BlockState
    std::size_t bytes_reserved_{0};
    SwapBackend* swap_backend_{nullptr};
    EvictionCandidateSelector eviction_selector_{};

    qvp_pool* pool_{nullptr};
    void* stream_{nullptr};
    void* side_stream_{nullptr};
    void* main_event_{nullptr};
    // Swap batches in launch order (the side stream runs them in order), the
    // last batch that gathered out of / scattered into each frame, and the
    // newest batch known finished or already waited for by the engine.
    std::deque<SwapBatchEvent> swap_events_;
    std::vector<void*> spare_events_;
    std::vector<std::uint64_t> gather_epoch_;
    std::vector<std::uint64_t> scatter_epoch_;
    std::uint64_t swap_epoch_{0};
    std::uint64_t completed_epoch_{0};
    std::uint64_t engine_waited_epoch_{0};
    bool own_stream_{false};
    bool ok_{true};
    std::string last_error_;
    std::vector<DeviceOp> queue_;
    std::uint64_t copy_launches_{0};
    std::uint64_t swap_launches_{0};
    double swap_gpu_ms_{0.0};
    std::uint64_t swap_bytes_{0};
};

}  // namespace qwenvl_paged

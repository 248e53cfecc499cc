// Physical block pool (API: include/qwenvl_paged/MemoryAllocator.h of the
// reference; decisions: src/MemoryAllocator.cpp), with a device placement
// whose byte movements run as batched launches (libqvp): copies on the engine
// stream, swap gathers and scatters on a side stream that runs beside it.
#include "qwenvl_paged/MemoryAllocator.h"

#include "qvp.h"

#include <algorithm>
#include <cstring>
#include <unordered_set>
#include <utility>

namespace qwenvl_paged {

MemoryAllocator::MemoryAllocator(AllocatorConfig config) : config_(config) {
    const std::uint32_t n = config_.max_blocks;
    std::byte* base = nullptr;
    std::size_t stride = 0;
    if (config_.placement == BlockPlacement::Device && n > 0) {
        // One pool allocation; frame i at base + i * stride.
        if (qvp_pool_create(n, config_.block_shape.byte_size(), config_.memory_options.alignment_bytes, &pool_) !=
            QVP_OK) {
            fail(std::string("qvp_pool_create: ") + qvp_last_error());
            return;
        }
        base = static_cast<std::byte*>(qvp_pool_base(pool_));
        stride = qvp_pool_block_stride(pool_);
        own_stream_ = config_.stream == nullptr;
        stream_ = config_.stream;
        const bool streams = (!own_stream_ || qvp_stream_create(&stream_) == QVP_OK) &&
                             qvp_stream_create(&side_stream_) == QVP_OK &&
                             qvp_event_create(&main_event_) == QVP_OK;
        if (!streams) {
            fail(std::string("stream/event setup: ") + qvp_last_error());
            return;
        }
        gather_epoch_.assign(n, 0);
        scatter_epoch_.assign(n, 0);
    } else if (config_.placement == BlockPlacement::Device) {
        // An empty device pool holds nothing to place on the device.
        return;
    }

    // Every frame starts free. The free list is a stack holding 0..N-1, so
    // the first allocate() hands out frame N-1 and a released frame is the
    // next one handed out.
    infos_.resize(n);
    free_list_.resize(n);
    blocks_.reserve(n);
    for (PhysicalBlockId id = 0; id < n; ++id) {
        infos_[id].id = id;
        free_list_[id] = id;
        blocks_.push_back(config_.placement == BlockPlacement::Device
                              ? std::make_unique<PhysicalBlock>(id, config_.block_shape, config_.memory_options,
                                                                base + static_cast<std::size_t>(id) * stride, stride)
                              : std::make_unique<PhysicalBlock>(id, config_.block_shape, config_.memory_options));
        bytes_reserved_ += blocks_.back()->size_bytes();
    }
    state_counts_[static_cast<std::size_t>(BlockState::Free)] = n;
}

MemoryAllocator::~MemoryAllocator() {
    if (config_.placement != BlockPlacement::Device) return;
    // Work already handed to the device must finish before the pool goes;
    // operations still queued are dropped with it.
    if (stream_ != nullptr) (void)qvp_stream_synchronize(stream_);
    if (side_stream_ != nullptr) (void)qvp_stream_synchronize(side_stream_);
    for (SwapBatchEvent& b : swap_events_) {
        (void)qvp_event_destroy(b.start);
        (void)qvp_event_destroy(b.event);
    }
    for (void* e : spare_events_) (void)qvp_event_destroy(e);
    (void)qvp_event_destroy(main_event_);
    (void)qvp_stream_destroy(side_stream_);
    if (own_stream_) (void)qvp_stream_destroy(stream_);
    (void)qvp_pool_destroy(pool_);
}

bool MemoryAllocator::fail(const std::string& what) {
    ok_ = false;
    last_error_ = what;
    return false;
}

// The one place a frame's reference count changes. Its state follows from the
// count (0 free, 1 active, more shared), and the per-state counts behind
// stats() move with it. Dropping to zero returns the frame to the top of the
// free stack under a new generation, so ids held across the free are stale.
void MemoryAllocator::set_ref_count(PhysicalBlockInfo& info, std::uint32_t count) noexcept {
    const BlockState next = count == 0 ? BlockState::Free : (count == 1 ? BlockState::Active : BlockState::Shared);
    --state_counts_[static_cast<std::size_t>(info.state)];
    ++state_counts_[static_cast<std::size_t>(next)];
    if (count == 0 && info.ref_count != 0) {
        ++info.generation;
        free_list_.push_back(info.id);
    }
    info.ref_count = count;
    info.state = next;
}

std::optional<PhysicalBlockId> MemoryAllocator::allocate() {
    if (free_list_.empty()) return std::nullopt;
    const PhysicalBlockId id = free_list_.back();
    free_list_.pop_back();
    set_ref_count(infos_[id], 1);
    return id;
}

void MemoryAllocator::release(PhysicalBlockId id) {
    PhysicalBlockInfo* held = id < infos_.size() ? &infos_[id] : nullptr;
    if (held != nullptr && held->ref_count > 0) set_ref_count(*held, held->ref_count - 1);
}

void MemoryAllocator::retain(PhysicalBlockId id) {
    // Only a frame someone holds can gain a sharer.
    PhysicalBlockInfo* held = id < infos_.size() ? &infos_[id] : nullptr;
    if (held != nullptr && held->ref_count > 0) set_ref_count(*held, held->ref_count + 1);
}

void MemoryAllocator::copy_block(PhysicalBlockId source, PhysicalBlockId destination) {
    PhysicalBlock* from = block(source);
    PhysicalBlock* to = block(destination);
    if (from == nullptr || to == nullptr) return;
    if (config_.placement == BlockPlacement::Device) {
        // Queued; flush() runs the step's copies as one launch.
        if (source != destination) queue_.push_back(DeviceOp{OpKind::Copy, source, destination, nullptr, 0, 0});
        return;
    }
    std::memcpy(to->data(), from->data(), std::min(from->size_bytes(), to->size_bytes()));
}

PhysicalBlock* MemoryAllocator::block(PhysicalBlockId id) noexcept {
    return id < blocks_.size() ? blocks_[id].get() : nullptr;
}

const PhysicalBlock* MemoryAllocator::block(PhysicalBlockId id) const noexcept {
    return id < blocks_.size() ? blocks_[id].get() : nullptr;
}

const PhysicalBlockInfo* MemoryAllocator::info(PhysicalBlockId id) const noexcept {
    return id < infos_.size() ? &infos_[id] : nullptr;
}

void MemoryAllocator::set_swap_backend(SwapBackend* backend) noexcept { swap_backend_ = backend; }

void MemoryAllocator::detach_swap_backend(const SwapBackend* backend) noexcept {
    if (swap_backend_ == backend) swap_backend_ = nullptr;
}

std::optional<SwapSlotId> MemoryAllocator::swap_out(PhysicalBlockId id) {
    // Only a frame held by exactly one sequence can leave the pool: a free
    // frame holds nothing and a shared one is still mapped by a sibling.
    PhysicalBlockInfo* held = (swap_backend_ != nullptr && id < infos_.size()) ? &infos_[id] : nullptr;
    if (held == nullptr || held->ref_count != 1 || block(id) == nullptr) return std::nullopt;
    const std::optional<SwapSlotId> slot = swap_backend_->store(*block(id));
    if (slot) set_ref_count(*held, 0);
    return slot;
}

std::optional<PhysicalBlockId> MemoryAllocator::swap_in(SwapSlotId slot) {
    if (swap_backend_ == nullptr) return std::nullopt;
    // The bytes come back into a freshly allocated frame; the slot is freed
    // only once they are in (a failed load gives the frame back).
    const std::optional<PhysicalBlockId> frame = allocate();
    if (!frame) return std::nullopt;
    if (!swap_backend_->load(slot, *block(*frame))) {
        release(*frame);
        return std::nullopt;
    }
    swap_backend_->discard(slot);
    return frame;
}

void MemoryAllocator::discard_swapped(SwapSlotId slot) {
    if (swap_backend_ != nullptr) swap_backend_->discard(slot);
}

void MemoryAllocator::set_eviction_selector(EvictionCandidateSelector selector) {
    eviction_selector_ = std::move(selector);
}

std::optional<PhysicalBlockId> MemoryAllocator::select_eviction_candidate() const {
    if (!eviction_selector_) return std::nullopt;
    return eviction_selector_(*this);
}

// Same figures as counting every block's state (src/MemoryAllocator.cpp:178-207),
// kept as running counts so the scheduler's per-step calls cost O(1).
AllocatorStats MemoryAllocator::stats() const noexcept {
    AllocatorStats s;
    s.total_blocks = static_cast<std::uint32_t>(infos_.size());
    s.free_blocks = state_counts_[static_cast<std::size_t>(BlockState::Free)];
    s.active_blocks = state_counts_[static_cast<std::size_t>(BlockState::Active)];
    s.shared_blocks = state_counts_[static_cast<std::size_t>(BlockState::Shared)];
    if (swap_backend_ != nullptr) s.swapped_blocks = static_cast<std::uint32_t>(swap_backend_->resident_slots());
    s.bytes_reserved = bytes_reserved_;
    return s;
}

bool MemoryAllocator::can_allocate(std::uint32_t block_count) const noexcept {
    return free_list_.size() >= block_count;
}

// ---------------------------------------------------------------------------
// Device placement
// ---------------------------------------------------------------------------

BlockPlacement MemoryAllocator::placement() const noexcept { return config_.placement; }
bool MemoryAllocator::ok() const noexcept { return ok_; }
const std::string& MemoryAllocator::last_error() const noexcept { return last_error_; }
void* MemoryAllocator::stream() const noexcept { return stream_; }
void* MemoryAllocator::side_stream() const noexcept { return side_stream_; }
void* MemoryAllocator::device_base() const noexcept { return pool_ ? qvp_pool_base(pool_) : nullptr; }
std::size_t MemoryAllocator::block_stride() const noexcept { return pool_ ? qvp_pool_block_stride(pool_) : 0; }
std::size_t MemoryAllocator::pending_operations() const noexcept { return queue_.size(); }
std::uint64_t MemoryAllocator::copy_launches() const noexcept { return copy_launches_; }
std::uint64_t MemoryAllocator::swap_launches() const noexcept { return swap_launches_; }
double MemoryAllocator::swap_gpu_ms() const noexcept { return swap_gpu_ms_; }
std::uint64_t MemoryAllocator::swap_bytes_moved() const noexcept { return swap_bytes_; }

void MemoryAllocator::enqueue_swap_gather(PhysicalBlockId frame, void* arena, std::size_t arena_bytes,
                                          std::size_t offset) {
    queue_.push_back(DeviceOp{OpKind::Gather, frame, 0, arena, arena_bytes, offset});
}

void MemoryAllocator::enqueue_swap_scatter(PhysicalBlockId frame, void* arena, std::size_t arena_bytes,
                                           std::size_t offset) {
    queue_.push_back(DeviceOp{OpKind::Scatter, frame, 0, arena, arena_bytes, offset});
}

bool MemoryAllocator::run_batch(OpKind kind, const std::vector<DeviceOp>& ops) {
    const std::uint32_t n = static_cast<std::uint32_t>(ops.size());
    const std::size_t stride = block_stride();
    std::vector<std::uint32_t> a(n), b(n);
    std::vector<std::uint64_t> off(n);
    for (std::uint32_t i = 0; i < n; ++i) {
        a[i] = ops[i].frame_a;
        b[i] = ops[i].frame_b;
        off[i] = ops[i].offset;
    }
    if (kind == OpKind::Copy) {
        // Copies run on the engine stream: their sources may still be coming
        // back from the swap store, their destinations may still be read by
        // a gather.
        if (!order_engine_after_swaps(a.data(), n, false) || !order_engine_after_swaps(b.data(), n, true)) return false;
        const int st = qvp_copy_blocks(qvp_pool_base(pool_), stride, config_.max_blocks, a.data(), b.data(), n, stride,
                                       stream_);
        if (st != QVP_OK) return fail(std::string("qvp_copy_blocks: ") + qvp_last_error());
        ++copy_launches_;
        return true;
    }
    // Swap traffic runs on the side stream, after everything already on the
    // engine stream (which wrote the frames a gather reads and may still read
    // the frames a scatter overwrites). The engine stream does not wait for
    // it here: a completion event per batch lets later engine work wait only
    // where it touches a frame the batch moved (order_frame_reads / _writes).
    if (qvp_event_record(main_event_, stream_) != QVP_OK || qvp_stream_wait_event(side_stream_, main_event_) != QVP_OK) {
        return fail(std::string("swap ordering: ") + qvp_last_error());
    }
    void* ev[2] = {nullptr, nullptr};
    for (void*& e : ev) {
        if (!spare_events_.empty()) {
            e = spare_events_.back();
            spare_events_.pop_back();
        } else if (qvp_event_create(&e) != QVP_OK) {
            for (void* made : ev) {
                if (made != nullptr) spare_events_.push_back(made);
            }
            return fail(std::string("swap event: ") + qvp_last_error());
        }
    }
    if (qvp_event_record(ev[0], side_stream_) != QVP_OK) {
        spare_events_.insert(spare_events_.end(), ev, ev + 2);
        return fail(std::string("swap ordering: ") + qvp_last_error());
    }
    const int st = kind == OpKind::Gather
                       ? qvp_swap_gather(qvp_pool_base(pool_), stride, config_.max_blocks, a.data(), off.data(), n,
                                         ops[0].arena, ops[0].arena_bytes, stride, side_stream_)
                       : qvp_swap_scatter(qvp_pool_base(pool_), stride, config_.max_blocks, a.data(), off.data(), n,
                                          ops[0].arena, ops[0].arena_bytes, stride, side_stream_);
    if (st != QVP_OK || qvp_event_record(ev[1], side_stream_) != QVP_OK) {
        // The start event may already be recorded on the side stream; the
        // events are only reused once that stream has passed them.
        (void)qvp_stream_synchronize(side_stream_);
        spare_events_.insert(spare_events_.end(), ev, ev + 2);
        return fail(std::string(st != QVP_OK ? "swap launch: " : "swap ordering: ") + qvp_last_error());
    }
    const std::uint64_t epoch = ++swap_epoch_;
    swap_events_.push_back(SwapBatchEvent{epoch, ev[0], ev[1], static_cast<std::uint64_t>(n) * stride});
    std::vector<std::uint64_t>& moved = kind == OpKind::Gather ? gather_epoch_ : scatter_epoch_;
    for (const DeviceOp& op : ops) moved[op.frame_a] = epoch;
    ++swap_launches_;
    return true;
}

bool MemoryAllocator::retire_swap_batches() {
    while (!swap_events_.empty()) {
        int complete = 0;
        if (qvp_event_query(swap_events_.front().event, &complete) != QVP_OK) {
            return fail(std::string("swap event query: ") + qvp_last_error());
        }
        if (complete == 0) break;
        const SwapBatchEvent& b = swap_events_.front();
        float ms = 0.f;
        if (qvp_event_elapsed_ms(&ms, b.start, b.event) == QVP_OK) swap_gpu_ms_ += ms;
        swap_bytes_ += b.bytes;
        completed_epoch_ = b.epoch;
        spare_events_.push_back(b.start);
        spare_events_.push_back(b.event);
        swap_events_.pop_front();
    }
    return true;
}

bool MemoryAllocator::order_engine_after_swaps(const PhysicalBlockId* frames, std::size_t n, bool writes) {
    if (config_.placement != BlockPlacement::Device || swap_events_.empty()) return true;
    // Batches finish in launch order: when the engine stream already waits
    // for (or the host has seen the end of) the newest one, no frame needs a
    // look.
    if (swap_events_.back().epoch <= std::max(completed_epoch_, engine_waited_epoch_)) return true;
    // A read depends on the last scatter into the frame; a write also on the
    // last gather out of it (which must have read the old bytes first).
    std::uint64_t need = 0;
    for (std::size_t k = 0; k < n; ++k) {
        if (frames[k] >= scatter_epoch_.size()) continue;
        need = std::max(need, scatter_epoch_[frames[k]]);
        if (writes) need = std::max(need, gather_epoch_[frames[k]]);
    }
    if (need <= std::max(completed_epoch_, engine_waited_epoch_)) return true;
    if (!retire_swap_batches()) return false;
    if (need <= completed_epoch_) return true;
    // Batches finish in launch order, so waiting for batch `need` covers
    // every earlier one.
    for (const SwapBatchEvent& b : swap_events_) {
        if (b.epoch != need) continue;
        if (qvp_stream_wait_event(stream_, b.event) != QVP_OK) {
            return fail(std::string("swap ordering: ") + qvp_last_error());
        }
        engine_waited_epoch_ = need;
        return true;
    }
    return fail("swap batch event missing");
}

bool MemoryAllocator::order_frame_reads(const std::vector<PhysicalBlockId>& frames) {
    return order_engine_after_swaps(frames.data(), frames.size(), false);
}

bool MemoryAllocator::order_frame_writes(const std::vector<PhysicalBlockId>& frames) {
    return order_engine_after_swaps(frames.data(), frames.size(), true);
}

bool MemoryAllocator::flush() { return flush_queue(0, nullptr, nullptr, nullptr); }

bool MemoryAllocator::flush_except_last_copies(std::size_t max_pairs, const std::vector<PhysicalBlockId>& written,
                                               std::vector<PhysicalBlockId>& src, std::vector<PhysicalBlockId>& dst) {
    src.clear();
    dst.clear();
    return flush_queue(max_pairs, &written, &src, &dst);
}

bool MemoryAllocator::flush_queue(std::size_t max_pairs, const std::vector<PhysicalBlockId>* written,
                                  std::vector<PhysicalBlockId>* src, std::vector<PhysicalBlockId>* dst) {
    if (config_.placement != BlockPlacement::Device) return true;
    if (!ok_) {
        queue_.clear();
        return false;
    }
    bool good = true;
    std::size_t i = 0;
    std::vector<DeviceOp> batch;
    std::unordered_set<PhysicalBlockId> reads, writes;
    std::vector<std::size_t> regions;
    while (i < queue_.size()) {
        const OpKind kind = queue_[i].kind;
        batch.clear();
        reads.clear();
        writes.clear();
        regions.clear();
        // Extend the batch while the next operation is of the same kind and
        // does not touch what the batch reads or writes, so running the batch
        // in parallel gives the same bytes as running it in order.
        for (; i < queue_.size() && queue_[i].kind == kind; ++i) {
            const DeviceOp& op = queue_[i];
            bool hazard = false;
            if (kind == OpKind::Copy) {
                hazard = writes.count(op.frame_b) || reads.count(op.frame_b) || writes.count(op.frame_a);
            } else if (kind == OpKind::Gather) {
                hazard = !batch.empty() && op.arena != batch.front().arena;
                for (std::size_t r : regions) hazard = hazard || r == op.offset;
            } else {
                hazard = writes.count(op.frame_a) || (!batch.empty() && op.arena != batch.front().arena);
            }
            if (hazard) break;
            batch.push_back(op);
            if (kind == OpKind::Copy) {
                reads.insert(op.frame_a);
                writes.insert(op.frame_b);
            } else if (kind == OpKind::Gather) {
                regions.push_back(op.offset);
            } else {
                writes.insert(op.frame_a);
            }
        }
        if (src != nullptr && kind == OpKind::Copy && i == queue_.size() && batch.size() <= max_pairs) {
            bool reads_written = false;
            for (PhysicalBlockId w : *written) reads_written = reads_written || reads.count(w) != 0;
            if (!reads_written) {
                for (const DeviceOp& op : batch) {
                    src->push_back(op.frame_a);
                    dst->push_back(op.frame_b);
                }
                good = order_engine_after_swaps(src->data(), src->size(), false) &&
                       order_engine_after_swaps(dst->data(), dst->size(), true);
                if (good) ++copy_launches_;
                break;
            }
        }
        if (!run_batch(kind, batch)) {
            good = false;
            break;
        }
    }
    queue_.clear();
    return good;
}

bool MemoryAllocator::write_block_bytes(PhysicalBlockId id, std::size_t offset, const void* src, std::size_t bytes) {
    PhysicalBlock* b = block(id);
    if (b == nullptr || offset > b->size_bytes() || bytes > b->size_bytes() - offset) return false;
    if (config_.placement == BlockPlacement::Host) {
        std::memcpy(b->data() + offset, src, bytes);
        return true;
    }
    if (!flush() || !order_engine_after_swaps(&id, 1, true)) return false;
    if (qvp_pool_write(pool_, id, offset, src, bytes, stream_) != QVP_OK || qvp_stream_synchronize(stream_) != QVP_OK) {
        return fail(std::string("block write: ") + qvp_last_error());
    }
    return true;
}

bool MemoryAllocator::read_block_bytes(PhysicalBlockId id, std::size_t offset, void* dst, std::size_t bytes) {
    const PhysicalBlock* b = block(id);
    if (b == nullptr || offset > b->size_bytes() || bytes > b->size_bytes() - offset) return false;
    if (config_.placement == BlockPlacement::Host) {
        std::memcpy(dst, b->data() + offset, bytes);
        return true;
    }
    if (!flush() || !order_engine_after_swaps(&id, 1, false)) return false;
    if (qvp_pool_read(pool_, id, offset, dst, bytes, stream_) != QVP_OK || qvp_stream_synchronize(stream_) != QVP_OK) {
        return fail(std::string("block read: ") + qvp_last_error());
    }
    return true;
}

bool MemoryAllocator::synchronize() {
    if (config_.placement != BlockPlacement::Device) return true;
    const bool flushed = flush();
    if (stream_ != nullptr && qvp_stream_synchronize(stream_) != QVP_OK) return fail(qvp_last_error());
    if (side_stream_ != nullptr && qvp_stream_synchronize(side_stream_) != QVP_OK) return fail(qvp_last_error());
    return retire_swap_batches() && flushed;
}

}  // namespace qwenvl_paged

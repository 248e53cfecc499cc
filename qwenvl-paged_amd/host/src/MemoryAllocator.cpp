// Physical block pool (src/MemoryAllocator.cpp of the reference), with a
// device placement whose byte movements run as batched launches (libqvp).
#include "qwenvl_paged/MemoryAllocator.h"

#include "qvp.h"

#include <algorithm>
#include <cstring>
#include <unordered_set>
#include <utility>

namespace qwenvl_paged {

MemoryAllocator::MemoryAllocator(AllocatorConfig config) : config_(config) {
    std::byte* base = nullptr;
    std::size_t stride = 0;
    if (config_.placement == BlockPlacement::Device) {
        if (config_.max_blocks == 0) {
            // An empty device pool holds nothing to place on the device.
            return;
        }
        const int st = qvp_pool_create(config_.max_blocks, config_.block_shape.byte_size(),
                                       config_.memory_options.alignment_bytes, &pool_);
        if (st != QVP_OK) {
            fail(std::string("qvp_pool_create: ") + qvp_last_error());
            return;
        }
        base = static_cast<std::byte*>(qvp_pool_base(pool_));
        stride = qvp_pool_block_stride(pool_);
        if (config_.stream != nullptr) {
            stream_ = config_.stream;
        } else if (qvp_stream_create(&stream_) == QVP_OK) {
            own_stream_ = true;
        } else {
            fail(std::string("qvp_stream_create: ") + qvp_last_error());
            return;
        }
        if (qvp_stream_create(&side_stream_) != QVP_OK || qvp_event_create(&main_event_) != QVP_OK ||
            qvp_event_create(&side_event_) != QVP_OK) {
            fail(std::string("stream/event setup: ") + qvp_last_error());
            return;
        }
    }

    blocks_.reserve(config_.max_blocks);
    infos_.reserve(config_.max_blocks);
    free_list_.reserve(config_.max_blocks);
    for (std::uint32_t i = 0; i < config_.max_blocks; ++i) {
        if (config_.placement == BlockPlacement::Device) {
            blocks_.push_back(std::make_unique<PhysicalBlock>(i, config_.block_shape, config_.memory_options,
                                                              base + static_cast<std::size_t>(i) * stride, stride));
        } else {
            blocks_.push_back(std::make_unique<PhysicalBlock>(i, config_.block_shape, config_.memory_options));
        }
        PhysicalBlockInfo info;
        info.id = i;
        ++state_counts_[static_cast<std::size_t>(info.state)];
        bytes_reserved_ += blocks_.back()->size_bytes();
        infos_.push_back(info);
        // Free list 0..N-1, so allocate() pops N-1 first.
        free_list_.push_back(i);
    }
}

MemoryAllocator::~MemoryAllocator() {
    if (config_.placement != BlockPlacement::Device) return;
    // Work already handed to the device must finish before the pool goes;
    // operations still queued are dropped with it.
    if (stream_ != nullptr) (void)qvp_stream_synchronize(stream_);
    if (side_stream_ != nullptr) (void)qvp_stream_synchronize(side_stream_);
    (void)qvp_event_destroy(main_event_);
    (void)qvp_event_destroy(side_event_);
    (void)qvp_stream_destroy(side_stream_);
    if (own_stream_) (void)qvp_stream_destroy(stream_);
    (void)qvp_pool_destroy(pool_);
}

void MemoryAllocator::set_state(PhysicalBlockInfo& info, BlockState state) noexcept {
    --state_counts_[static_cast<std::size_t>(info.state)];
    ++state_counts_[static_cast<std::size_t>(state)];
    info.state = state;
}

bool MemoryAllocator::fail(const std::string& what) {
    ok_ = false;
    last_error_ = what;
    return false;
}

std::optional<PhysicalBlockId> MemoryAllocator::allocate() {
    if (free_list_.empty()) return std::nullopt;
    const PhysicalBlockId id = free_list_.back();
    free_list_.pop_back();
    PhysicalBlockInfo& info = infos_[id];
    set_state(info, BlockState::Active);
    info.ref_count = 1;
    return id;
}

void MemoryAllocator::release(PhysicalBlockId id) {
    if (id >= infos_.size()) return;
    PhysicalBlockInfo& info = infos_[id];
    if (info.ref_count == 0) return;
    --info.ref_count;
    if (info.ref_count == 0) {
        set_state(info, BlockState::Free);
        ++info.generation;
        free_list_.push_back(id);
    } else if (info.ref_count == 1) {
        set_state(info, BlockState::Active);
    }
}

void MemoryAllocator::retain(PhysicalBlockId id) {
    if (id >= infos_.size()) return;
    PhysicalBlockInfo& info = infos_[id];
    if (info.ref_count == 0) return;
    ++info.ref_count;
    set_state(info, BlockState::Shared);
}

void MemoryAllocator::copy_block(PhysicalBlockId source, PhysicalBlockId destination) {
    PhysicalBlock* src = block(source);
    PhysicalBlock* dst = block(destination);
    if (src == nullptr || dst == nullptr) return;
    if (config_.placement == BlockPlacement::Device) {
        if (source != destination) queue_.push_back(DeviceOp{OpKind::Copy, source, destination, nullptr, 0, 0});
        return;
    }
    const std::size_t bytes = std::min(src->size_bytes(), dst->size_bytes());
    std::memcpy(dst->data(), src->data(), bytes);
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
    if (swap_backend_ == nullptr || id >= infos_.size()) return std::nullopt;
    PhysicalBlockInfo& info = infos_[id];
    // A free block has nothing to evict; a shared one is still mapped by a
    // sibling (src/MemoryAllocator.cpp:113-116).
    if (info.ref_count != 1) return std::nullopt;
    PhysicalBlock* frame = block(id);
    if (frame == nullptr) return std::nullopt;
    const std::optional<SwapSlotId> slot = swap_backend_->store(*frame);
    if (!slot) return std::nullopt;
    info.ref_count = 0;
    set_state(info, BlockState::Free);
    ++info.generation;
    free_list_.push_back(id);
    return slot;
}

std::optional<PhysicalBlockId> MemoryAllocator::swap_in(SwapSlotId slot) {
    if (swap_backend_ == nullptr) return std::nullopt;
    const std::optional<PhysicalBlockId> id = allocate();
    if (!id) return std::nullopt;
    PhysicalBlock* frame = block(*id);
    if (frame == nullptr || !swap_backend_->load(slot, *frame)) {
        release(*id);
        return std::nullopt;
    }
    swap_backend_->discard(slot);
    return id;
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
        const int st = qvp_copy_blocks(qvp_pool_base(pool_), stride, config_.max_blocks, a.data(), b.data(), n, stride,
                                       stream_);
        if (st != QVP_OK) return fail(std::string("qvp_copy_blocks: ") + qvp_last_error());
        ++copy_launches_;
        return true;
    }
    // Swap traffic runs on the side stream, after everything already on the
    // engine stream, and the engine stream waits for it.
    if (qvp_event_record(main_event_, stream_) != QVP_OK || qvp_stream_wait_event(side_stream_, main_event_) != QVP_OK) {
        return fail(std::string("swap ordering: ") + qvp_last_error());
    }
    const int st = kind == OpKind::Gather
                       ? qvp_swap_gather(qvp_pool_base(pool_), stride, config_.max_blocks, a.data(), off.data(), n,
                                         ops[0].arena, ops[0].arena_bytes, stride, side_stream_)
                       : qvp_swap_scatter(qvp_pool_base(pool_), stride, config_.max_blocks, a.data(), off.data(), n,
                                          ops[0].arena, ops[0].arena_bytes, stride, side_stream_);
    if (st != QVP_OK) return fail(std::string("swap launch: ") + qvp_last_error());
    if (qvp_event_record(side_event_, side_stream_) != QVP_OK || qvp_stream_wait_event(stream_, side_event_) != QVP_OK) {
        return fail(std::string("swap ordering: ") + qvp_last_error());
    }
    ++swap_launches_;
    return true;
}

bool MemoryAllocator::flush() {
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
    if (!flush()) return false;
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
    if (!flush()) return false;
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
    return flushed;
}

}  // namespace qwenvl_paged

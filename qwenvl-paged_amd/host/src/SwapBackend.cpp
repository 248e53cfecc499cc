// Swap stores: host memory (API: include/qwenvl_paged/SwapBackend.h of the
// reference; slot numbering and capacity rules: src/SwapBackend.cpp) and the
// pinned-arena backend of the device allocator.
#include "qwenvl_paged/SwapBackend.h"

#include "qvp.h"
#include "qwenvl_paged/MemoryAllocator.h"

#include <algorithm>
#include <cstring>
#include <utility>

namespace qwenvl_paged {

HostSwapBackend::HostSwapBackend(std::size_t max_slots) : max_slots_(max_slots) {}

std::optional<SwapSlotId> HostSwapBackend::store(const PhysicalBlock& block) {
    // Capacity counts resident slots; slot ids count up from 1 and are never
    // reused, so a stale id can never name newer bytes.
    if (slot_buffer_.size() >= max_slots_) return std::nullopt;
    std::size_t buf = buffers_.size();
    if (idle_buffers_.empty()) {
        buffers_.emplace_back();
    } else {
        buf = idle_buffers_.back();
        idle_buffers_.pop_back();
    }
    std::vector<std::byte>& bytes = buffers_[buf];
    bytes.assign(block.data(), block.data() + block.size_bytes());
    slot_buffer_.emplace(next_slot_, buf);
    return next_slot_++;
}

bool HostSwapBackend::load(SwapSlotId slot, PhysicalBlock& block) {
    // The slot stays resident after a load; discard() frees it.
    const auto it = slot_buffer_.find(slot);
    if (it == slot_buffer_.end()) return false;
    const std::vector<std::byte>& bytes = buffers_[it->second];
    if (bytes.size() > block.size_bytes()) return false;
    std::copy(bytes.begin(), bytes.end(), block.data());
    return true;
}

void HostSwapBackend::discard(SwapSlotId slot) {
    const auto it = slot_buffer_.find(slot);
    if (it == slot_buffer_.end()) return;
    idle_buffers_.push_back(it->second);
    slot_buffer_.erase(it);
}

std::size_t HostSwapBackend::resident_slots() const noexcept { return slot_buffer_.size(); }
std::size_t HostSwapBackend::capacity_slots() const noexcept { return max_slots_; }

// ---------------------------------------------------------------------------

PinnedSwapBackend::PinnedSwapBackend(MemoryAllocator& device_allocator, std::size_t max_slots)
    : allocator_(&device_allocator), max_slots_(max_slots), slot_stride_(device_allocator.block_stride()) {
    if (device_allocator.placement() != BlockPlacement::Device || max_slots_ == 0 || slot_stride_ == 0) return;
    void* p = nullptr;
    if (qvp_host_alloc(&p, max_slots_ * slot_stride_) != QVP_OK) return;
    arena_ = static_cast<std::byte*>(p);
    free_regions_.reserve(max_slots_);
    // Hand out low regions first.
    for (std::size_t i = max_slots_; i > 0; --i) free_regions_.push_back(i - 1);
}

PinnedSwapBackend::~PinnedSwapBackend() {
    // Destroy the backend before its allocator. Queued gathers or scatters may
    // still target the arena, so they run (and finish) before it is freed.
    if (arena_ != nullptr) {
        allocator_->synchronize();
        (void)qvp_host_free(arena_);
    }
    allocator_->detach_swap_backend(this);
}

bool PinnedSwapBackend::ok() const noexcept { return arena_ != nullptr; }

// Only frames of the allocator the backend was built on can be gathered from
// or scattered to: the queued operation names the frame by id.
bool PinnedSwapBackend::owns(const PhysicalBlock& block) const noexcept {
    return block.placement() == BlockPlacement::Device && allocator_->block(block.id()) == &block;
}

std::optional<SwapSlotId> PinnedSwapBackend::store(const PhysicalBlock& block) {
    if (arena_ == nullptr || slots_.size() >= max_slots_ || free_regions_.empty()) return std::nullopt;
    if (!owns(block) || block.size_bytes() > slot_stride_) return std::nullopt;
    const std::size_t region = free_regions_.back();
    free_regions_.pop_back();
    const SwapSlotId slot = next_slot_++;
    slots_.emplace(slot, region);
    allocator_->enqueue_swap_gather(block.id(), arena_, max_slots_ * slot_stride_, region * slot_stride_);
    return slot;
}

bool PinnedSwapBackend::load(SwapSlotId slot, PhysicalBlock& block) {
    auto it = slots_.find(slot);
    if (it == slots_.end()) return false;
    if (!owns(block) || block.size_bytes() < slot_stride_) return false;
    allocator_->enqueue_swap_scatter(block.id(), arena_, max_slots_ * slot_stride_, it->second * slot_stride_);
    return true;
}

void PinnedSwapBackend::discard(SwapSlotId slot) {
    auto it = slots_.find(slot);
    if (it == slots_.end()) return;
    // A later store may gather into this region; the allocator's queue keeps
    // that gather after any scatter already queued from it.
    free_regions_.push_back(it->second);
    slots_.erase(it);
}

std::size_t PinnedSwapBackend::resident_slots() const noexcept { return slots_.size(); }
std::size_t PinnedSwapBackend::capacity_slots() const noexcept { return max_slots_; }
std::size_t PinnedSwapBackend::slot_stride() const noexcept { return slot_stride_; }

const std::byte* PinnedSwapBackend::slot_bytes(SwapSlotId slot) {
    auto it = slots_.find(slot);
    if (it == slots_.end()) return nullptr;
    if (!allocator_->synchronize()) return nullptr;
    return arena_ + it->second * slot_stride_;
}

}  // namespace qwenvl_paged

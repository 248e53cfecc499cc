#pragma once
// Store for the bytes of evicted blocks (include/qwenvl_paged/SwapBackend.h:27-93).
//
// HostSwapBackend keeps the reference behaviour (whole-block copies in host
// memory, slot ids counting up from 1, fixed capacity). PinnedSwapBackend is
// the device counterpart: slots are regions of one pinned host arena, and
// store/load only record a gather (frame -> arena) or scatter (arena -> frame)
// in the device allocator's ordered operation queue; MemoryAllocator::flush()
// runs each batch as one kernel launch on the allocator's side stream.

#include "qwenvl_paged/Block.h"

#include <cstddef>
#include <optional>
#include <unordered_map>
#include <vector>

namespace qwenvl_paged {

class MemoryAllocator;

class SwapBackend {
public:
    virtual ~SwapBackend() = default;
    // Copies a block's bytes into a new slot; nullopt when full (SwapBackend.h:36-41).
    [[nodiscard]] virtual std::optional<SwapSlotId> store(const PhysicalBlock& block) = 0;
    // Copies a slot back into a block; the slot stays resident. False for an
    // unknown slot or a block too small for it (SwapBackend.h:43-52).
    [[nodiscard]] virtual bool load(SwapSlotId slot, PhysicalBlock& block) = 0;
    virtual void discard(SwapSlotId slot) = 0;
    [[nodiscard]] virtual std::size_t resident_slots() const noexcept = 0;
};

class HostSwapBackend final : public SwapBackend {
public:
    explicit HostSwapBackend(std::size_t max_slots);

    [[nodiscard]] std::optional<SwapSlotId> store(const PhysicalBlock& block) override;
    [[nodiscard]] bool load(SwapSlotId slot, PhysicalBlock& block) override;
    void discard(SwapSlotId slot) override;
    [[nodiscard]] std::size_t resident_slots() const noexcept override;
    [[nodiscard]] std::size_t capacity_slots() const noexcept;

private:
    std::size_t max_slots_{0};
    SwapSlotId next_slot_{1};
    // Slot id -> buffer holding its bytes. Buffers of discarded slots are
    // kept and reused by later stores (a swap store cycles through the same
    // frame size), so a store allocates only while the store grows.
    std::unordered_map<SwapSlotId, std::size_t> slot_buffer_;
    std::vector<std::vector<std::byte>> buffers_;
    std::vector<std::size_t> idle_buffers_;
};

// Swap space for a device-placement MemoryAllocator: max_slots frames of
// pinned host memory. Slot numbering and capacity follow HostSwapBackend.
class PinnedSwapBackend final : public SwapBackend {
public:
    // Destroy the backend before the allocator it was built on.
    PinnedSwapBackend(MemoryAllocator& device_allocator, std::size_t max_slots);
    ~PinnedSwapBackend() override;
    PinnedSwapBackend(const PinnedSwapBackend&) = delete;
    PinnedSwapBackend& operator=(const PinnedSwapBackend&) = delete;

    [[nodiscard]] std::optional<SwapSlotId> store(const PhysicalBlock& block) override;
    [[nodiscard]] bool load(SwapSlotId slot, PhysicalBlock& block) override;
    void discard(SwapSlotId slot) override;
    [[nodiscard]] std::size_t resident_slots() const noexcept override;
    [[nodiscard]] std::size_t capacity_slots() const noexcept;

    // Host address of a slot's bytes after flushing and waiting for the device
    // (for inspection); nullptr for an unknown slot.
    [[nodiscard]] const std::byte* slot_bytes(SwapSlotId slot);
    [[nodiscard]] std::size_t slot_stride() const noexcept;
    // True when the arena could be allocated.
    [[nodiscard]] bool ok() const noexcept;

private:
    [[nodiscard]] bool owns(const PhysicalBlock& block) const noexcept;

    MemoryAllocator* allocator_{nullptr};
    std::size_t max_slots_{0};
    std::size_t slot_stride_{0};
    std::byte* arena_{nullptr};
    SwapSlotId next_slot_{1};
    std::unordered_map<SwapSlotId, std::size_t> slots_;  // slot id -> arena index
    std::vector<std::size_t> free_regions_;
};

}  // namespace qwenvl_paged

#pragma once
// Page table of one sequence and cache stream (include/qwenvl_paged/BlockTable.h:14-122).
// Entries stay sorted by logical index; entries() is what the ragged-batch
// packer flattens into the device block table (docs/architecture.md:117-120).

#include "qwenvl_paged/Block.h"

#include <cstddef>
#include <optional>
#include <vector>

namespace qwenvl_paged {

struct BlockTableEntry {
    LogicalBlock logical{};
    PhysicalBlockId physical_id{0};
    bool writable{true};
    // Engaged while the block's bytes live in the swap backend; physical_id is
    // then stale (BlockTable.h:18-24).
    std::optional<SwapSlotId> swap_slot{};
};

class BlockTable {
public:
    explicit BlockTable(SequenceId sequence_id, CacheKind cache_kind = CacheKind::TextKV);

    [[nodiscard]] SequenceId sequence_id() const noexcept;
    [[nodiscard]] CacheKind cache_kind() const noexcept;
    [[nodiscard]] std::size_t size() const noexcept;
    [[nodiscard]] bool empty() const noexcept;

    // Adds or replaces (clearing any swap slot) one mapping.
    void map(LogicalBlock logical, PhysicalBlockId physical_id, bool writable);
    [[nodiscard]] std::optional<PhysicalBlockId> unmap(LogicalBlockIndex index);
    // nullopt for an unmapped or swapped-out index (BlockTable.h:82-88).
    [[nodiscard]] std::optional<PhysicalBlockId> lookup(LogicalBlockIndex index) const;
    [[nodiscard]] const BlockTableEntry* entry(LogicalBlockIndex index) const noexcept;
    [[nodiscard]] BlockTableEntry* mutable_entry(LogicalBlockIndex index) noexcept;
    void set_writable(LogicalBlockIndex index, bool writable);
    [[nodiscard]] const std::vector<BlockTableEntry>& entries() const noexcept;
    // Child table sharing every frame, all entries read-only (BlockTable.h:110-116).
    [[nodiscard]] BlockTable fork(SequenceId child_sequence_id) const;

private:
    SequenceId sequence_id_{0};
    CacheKind cache_kind_{CacheKind::TextKV};
    std::vector<BlockTableEntry> entries_;
};

}  // namespace qwenvl_paged

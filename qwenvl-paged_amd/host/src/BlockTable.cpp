// Sorted page table of one sequence (src/BlockTable.cpp of the reference).
#include "qwenvl_paged/BlockTable.h"

#include <algorithm>

namespace qwenvl_paged {

namespace {

template <typename Vec>
auto find_index(Vec& entries, LogicalBlockIndex index) {
    return std::lower_bound(entries.begin(), entries.end(), index,
                            [](const BlockTableEntry& e, LogicalBlockIndex v) { return e.logical.index < v; });
}

}  // namespace

BlockTable::BlockTable(SequenceId sequence_id, CacheKind cache_kind)
    : sequence_id_(sequence_id), cache_kind_(cache_kind) {}

SequenceId BlockTable::sequence_id() const noexcept { return sequence_id_; }
CacheKind BlockTable::cache_kind() const noexcept { return cache_kind_; }
std::size_t BlockTable::size() const noexcept { return entries_.size(); }
bool BlockTable::empty() const noexcept { return entries_.empty(); }

void BlockTable::map(LogicalBlock logical, PhysicalBlockId physical_id, bool writable) {
    auto it = find_index(entries_, logical.index);
    if (it != entries_.end() && it->logical.index == logical.index) {
        it->logical = logical;
        it->physical_id = physical_id;
        it->writable = writable;
        it->swap_slot.reset();
        return;
    }
    BlockTableEntry entry;
    entry.logical = logical;
    entry.physical_id = physical_id;
    entry.writable = writable;
    entries_.insert(it, entry);
}

std::optional<PhysicalBlockId> BlockTable::unmap(LogicalBlockIndex index) {
    auto it = find_index(entries_, index);
    if (it == entries_.end() || it->logical.index != index) return std::nullopt;
    const PhysicalBlockId id = it->physical_id;
    entries_.erase(it);
    return id;
}

std::optional<PhysicalBlockId> BlockTable::lookup(LogicalBlockIndex index) const {
    const BlockTableEntry* e = entry(index);
    if (e == nullptr || e->swap_slot.has_value()) return std::nullopt;
    return e->physical_id;
}

const BlockTableEntry* BlockTable::entry(LogicalBlockIndex index) const noexcept {
    auto it = find_index(entries_, index);
    return (it == entries_.end() || it->logical.index != index) ? nullptr : &*it;
}

BlockTableEntry* BlockTable::mutable_entry(LogicalBlockIndex index) noexcept {
    auto it = find_index(entries_, index);
    return (it == entries_.end() || it->logical.index != index) ? nullptr : &*it;
}

void BlockTable::set_writable(LogicalBlockIndex index, bool writable) {
    if (BlockTableEntry* e = mutable_entry(index)) e->writable = writable;
}

const std::vector<BlockTableEntry>& BlockTable::entries() const noexcept { return entries_; }

BlockTable BlockTable::fork(SequenceId child_sequence_id) const {
    BlockTable child(*this);
    child.sequence_id_ = child_sequence_id;
    for (BlockTableEntry& e : child.entries_) {
        e.writable = false;
        e.logical.sequence_id = child_sequence_id;
    }
    return child;
}

}  // namespace qwenvl_paged

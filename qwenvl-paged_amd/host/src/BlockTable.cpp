// Page table of one sequence and cache stream (API: include/qwenvl_paged/
// BlockTable.h:38-122 of the reference; semantics: src/BlockTable.cpp).
//
// Entries are kept sorted by logical index, which is what entries() returns
// and the ragged-batch packer flattens. A sequence's table grows by appending
// the next logical index (KVCacheManager::reserve_tokens), so in practice
// entry k holds logical block k: every lookup first tests that position and
// only a table with holes (unmapped indices) falls back to a binary search.
// The packer and the copy-on-write point therefore resolve a block in O(1).
#include "qwenvl_paged/BlockTable.h"

namespace qwenvl_paged {

namespace {

// Position of the first entry whose logical index is not below `index` (the
// insertion point that keeps the entries sorted).
std::size_t slot_for(const std::vector<BlockTableEntry>& entries, LogicalBlockIndex index) {
    const std::size_t n = entries.size();
    if (index < n && entries[index].logical.index == index) return index;  // dense table
    if (n == 0 || entries[n - 1].logical.index < index) return n;          // beyond the last
    std::size_t lo = 0;
    std::size_t hi = n;
    while (lo < hi) {
        const std::size_t mid = lo + (hi - lo) / 2;
        if (entries[mid].logical.index < index) {
            lo = mid + 1;
        } else {
            hi = mid;
        }
    }
    return lo;
}

bool holds(const std::vector<BlockTableEntry>& entries, std::size_t pos, LogicalBlockIndex index) {
    return pos < entries.size() && entries[pos].logical.index == index;
}

}  // namespace

BlockTable::BlockTable(SequenceId sequence_id, CacheKind cache_kind)
    : sequence_id_(sequence_id), cache_kind_(cache_kind) {}

SequenceId BlockTable::sequence_id() const noexcept { return sequence_id_; }
CacheKind BlockTable::cache_kind() const noexcept { return cache_kind_; }
std::size_t BlockTable::size() const noexcept { return entries_.size(); }
bool BlockTable::empty() const noexcept { return entries_.empty(); }
const std::vector<BlockTableEntry>& BlockTable::entries() const noexcept { return entries_; }

void BlockTable::map(LogicalBlock logical, PhysicalBlockId physical_id, bool writable) {
    // A (re)mapped entry points at a resident frame: no swap slot.
    const BlockTableEntry fresh{logical, physical_id, writable, std::nullopt};
    const std::size_t pos = slot_for(entries_, logical.index);
    if (holds(entries_, pos, logical.index)) {
        entries_[pos] = fresh;
    } else {
        entries_.insert(entries_.begin() + static_cast<std::ptrdiff_t>(pos), fresh);
    }
}

std::optional<PhysicalBlockId> BlockTable::unmap(LogicalBlockIndex index) {
    const std::size_t pos = slot_for(entries_, index);
    if (!holds(entries_, pos, index)) return std::nullopt;
    const PhysicalBlockId frame = entries_[pos].physical_id;
    entries_.erase(entries_.begin() + static_cast<std::ptrdiff_t>(pos));
    return frame;
}

const BlockTableEntry* BlockTable::entry(LogicalBlockIndex index) const noexcept {
    const std::size_t pos = slot_for(entries_, index);
    return holds(entries_, pos, index) ? entries_.data() + pos : nullptr;
}

BlockTableEntry* BlockTable::mutable_entry(LogicalBlockIndex index) noexcept {
    const std::size_t pos = slot_for(entries_, index);
    return holds(entries_, pos, index) ? entries_.data() + pos : nullptr;
}

std::optional<PhysicalBlockId> BlockTable::lookup(LogicalBlockIndex index) const {
    // A swapped-out entry's frame went back to the allocator: it faults like
    // an unmapped one.
    const BlockTableEntry* e = entry(index);
    if (e != nullptr && !e->swap_slot) return e->physical_id;
    return std::nullopt;
}

void BlockTable::set_writable(LogicalBlockIndex index, bool writable) {
    BlockTableEntry* e = mutable_entry(index);
    if (e != nullptr) e->writable = writable;
}

BlockTable BlockTable::fork(SequenceId child_sequence_id) const {
    // The child maps the same frames, owned by its own sequence, and every
    // shared frame is read-only until copy-on-write gives it a private one.
    BlockTable child(child_sequence_id, cache_kind_);
    child.entries_.reserve(entries_.size());
    for (BlockTableEntry e : entries_) {
        e.logical.sequence_id = child_sequence_id;
        e.writable = false;
        child.entries_.push_back(e);
    }
    return child;
}

}  // namespace qwenvl_paged

// Sequence cache lifecycle and CacheView (src/KVCacheManager.cpp of the
// reference). Identical decisions; on a device allocator the copy-on-write and
// swap byte movements are queued by the allocator and batched on flush.
#include "qwenvl_paged/KVCacheManager.h"

#include <utility>

namespace qwenvl_paged {

bool CacheView::valid() const noexcept {
    return block_table != nullptr && allocator != nullptr && layout.element_count() > 0;
}

const std::byte* CacheView::block_bytes(LogicalBlockIndex index) const noexcept {
    if (!valid()) return nullptr;
    // lookup() already refuses a swapped-out entry, whose frame may belong to
    // another sequence by now.
    const std::optional<PhysicalBlockId> physical = block_table->lookup(index);
    if (!physical) return nullptr;
    const PhysicalBlock* b = allocator->block(*physical);
    return b == nullptr ? nullptr : b->data();
}

KVCacheManager::KVCacheManager(MemoryAllocator& allocator) : allocator_(&allocator) {}

bool KVCacheManager::create_sequence(SequenceMetadata metadata) {
    const SequenceId id = metadata.sequence_id;
    if (sequences_.count(id) != 0) return false;
    sequences_.emplace(id, SequenceState{std::move(metadata), BlockTable(id)});
    return true;
}

bool KVCacheManager::fork_sequence(SequenceId parent_id, SequenceMetadata child_metadata) {
    auto parent = sequences_.find(parent_id);
    if (parent == sequences_.end()) return false;
    const SequenceId child_id = child_metadata.sequence_id;
    if (sequences_.count(child_id) != 0) return false;
    // A swapped-out block has no frame to share.
    for (const BlockTableEntry& e : parent->second.text_table.entries()) {
        if (e.swap_slot.has_value()) return false;
    }
    BlockTable child = parent->second.text_table.fork(child_id);
    for (const BlockTableEntry& e : child.entries()) allocator_->retain(e.physical_id);
    sequences_.emplace(child_id, SequenceState{std::move(child_metadata), std::move(child)});
    return true;
}

bool KVCacheManager::reserve_tokens(SequenceId sequence_id, std::uint32_t token_count) {
    auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return false;
    const PhysicalBlock* first = allocator_->block(0);
    const std::uint32_t tpb = first != nullptr ? first->shape().tokens_per_block : 0;
    if (tpb == 0) return false;
    const std::uint32_t needed = (token_count + tpb - 1) / tpb;
    if (!allocator_->can_allocate(needed)) return false;
    BlockTable& table = it->second.text_table;
    const LogicalBlockIndex base = static_cast<LogicalBlockIndex>(table.size());
    for (std::uint32_t k = 0; k < needed; ++k) {
        const std::optional<PhysicalBlockId> physical = allocator_->allocate();
        if (!physical) return false;
        LogicalBlock logical;
        logical.sequence_id = sequence_id;
        logical.index = base + k;
        logical.cache_kind = table.cache_kind();
        logical.start_token = (base + k) * tpb;
        logical.token_count = tpb;
        table.map(logical, *physical, true);
    }
    return true;
}

std::optional<PhysicalBlockId> KVCacheManager::ensure_token_writable(SequenceId sequence_id,
                                                                     TokenPosition token_position,
                                                                     CacheKind /*cache_kind*/) {
    auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return std::nullopt;
    BlockTable& table = it->second.text_table;
    if (table.empty()) return std::nullopt;
    const std::uint32_t tpb = table.entries().front().logical.token_count;
    if (tpb == 0) return std::nullopt;
    BlockTableEntry* entry = table.mutable_entry(static_cast<LogicalBlockIndex>(token_position / tpb));
    if (entry == nullptr || entry->swap_slot.has_value()) return std::nullopt;
    const PhysicalBlockInfo* info = allocator_->info(entry->physical_id);
    if (info == nullptr) return std::nullopt;
    // Sole owner: write in place. Shared (ref_count > 1, not the writable
    // flag, decides): materialise a private copy (src/KVCacheManager.cpp:136-150).
    if (info->ref_count <= 1) {
        entry->writable = true;
        return entry->physical_id;
    }
    const std::optional<PhysicalBlockId> copy = allocator_->allocate();
    if (!copy) return std::nullopt;
    allocator_->copy_block(entry->physical_id, *copy);
    allocator_->release(entry->physical_id);
    entry->physical_id = *copy;
    entry->writable = true;
    return *copy;
}

std::uint32_t KVCacheManager::swap_out_sequence(SequenceId sequence_id) {
    auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return 0;
    BlockTable& table = it->second.text_table;
    std::vector<LogicalBlockIndex> resident;
    for (const BlockTableEntry& e : table.entries()) {
        if (!e.swap_slot.has_value()) resident.push_back(e.logical.index);
    }
    std::uint32_t swapped = 0;
    for (const LogicalBlockIndex index : resident) {
        BlockTableEntry* e = table.mutable_entry(index);
        if (e == nullptr) continue;
        // Shared blocks are refused by the allocator and stay resident.
        const std::optional<SwapSlotId> slot = allocator_->swap_out(e->physical_id);
        if (!slot) continue;
        e->swap_slot = slot;
        ++swapped;
    }
    return swapped;
}

bool KVCacheManager::swap_in_sequence(SequenceId sequence_id) {
    auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return false;
    BlockTable& table = it->second.text_table;
    std::vector<LogicalBlockIndex> swapped;
    for (const BlockTableEntry& e : table.entries()) {
        if (e.swap_slot.has_value()) swapped.push_back(e.logical.index);
    }
    if (swapped.empty()) return true;
    // All-or-nothing through the capacity precheck (src/KVCacheManager.cpp:203-205).
    if (!allocator_->can_allocate(static_cast<std::uint32_t>(swapped.size()))) return false;
    for (const LogicalBlockIndex index : swapped) {
        BlockTableEntry* e = table.mutable_entry(index);
        if (e == nullptr) continue;
        const std::optional<PhysicalBlockId> restored = allocator_->swap_in(*e->swap_slot);
        if (!restored) return false;
        e->physical_id = *restored;
        e->swap_slot.reset();
    }
    return true;
}

void KVCacheManager::release_sequence(SequenceId sequence_id) {
    auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return;
    for (const BlockTableEntry& e : it->second.text_table.entries()) {
        if (e.swap_slot.has_value()) {
            allocator_->discard_swapped(*e.swap_slot);
        } else {
            allocator_->release(e.physical_id);
        }
    }
    sequences_.erase(it);
}

std::optional<CacheView> KVCacheManager::cache_view(SequenceId sequence_id, CacheKind cache_kind) const {
    auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return std::nullopt;
    CacheView view;
    view.sequence_id = sequence_id;
    view.cache_kind = cache_kind;
    view.block_table = &it->second.text_table;
    view.allocator = allocator_;
    if (const PhysicalBlock* b = allocator_->block(0)) view.layout.shape = b->shape();
    return view;
}

bool KVCacheManager::contains(SequenceId sequence_id) const noexcept { return sequences_.count(sequence_id) != 0; }

const SequenceMetadata* KVCacheManager::metadata(SequenceId sequence_id) const noexcept {
    auto it = sequences_.find(sequence_id);
    return it == sequences_.end() ? nullptr : &it->second.metadata;
}

}  // namespace qwenvl_paged

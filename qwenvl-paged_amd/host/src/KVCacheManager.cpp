// Sequence cache lifecycle above the allocator, and the CacheView read
// contract (API: include/qwenvl_paged/KVCacheManager.h:94-253 of the
// reference; decisions: src/KVCacheManager.cpp).
//
// Every operation works on the sequence's text page table through two small
// helpers: `state(id)` finds a sequence, and each table walk visits entries by
// position (the table's structure never changes during a walk; only frames
// and swap slots are rewritten in place). On a device allocator the
// copy-on-write and swap byte movements are queued by the allocator and run
// as batched launches on its next flush.
#include "qwenvl_paged/KVCacheManager.h"

#include <utility>

namespace qwenvl_paged {

bool CacheView::valid() const noexcept {
    return block_table != nullptr && allocator != nullptr && layout.element_count() > 0;
}

const std::byte* CacheView::block_bytes(LogicalBlockIndex index) const noexcept {
    if (!valid()) return nullptr;
    // A swapped-out entry owns no frame (its bytes sit in a swap slot, and
    // the frame id it last had is free for the allocator to reuse), so
    // lookup() answers nullopt for it as for an unmapped one.
    const std::optional<PhysicalBlockId> frame = block_table->lookup(index);
    const PhysicalBlock* b = frame ? allocator->block(*frame) : nullptr;
    return b != nullptr ? b->data() : nullptr;
}

KVCacheManager::KVCacheManager(MemoryAllocator& allocator) : allocator_(&allocator) {}

namespace {

// Tokens per block of the allocator's pool (0 for an empty pool).
std::uint32_t pool_tokens_per_block(const MemoryAllocator& allocator) {
    const PhysicalBlock* first = allocator.block(0);
    return first == nullptr ? 0u : first->shape().tokens_per_block;
}

}  // namespace

bool KVCacheManager::create_sequence(SequenceMetadata metadata) {
    const SequenceId id = metadata.sequence_id;
    return sequences_.try_emplace(id, SequenceState{std::move(metadata), BlockTable(id)}).second;
}

bool KVCacheManager::fork_sequence(SequenceId parent_id, SequenceMetadata child_metadata) {
    const auto parent = sequences_.find(parent_id);
    const SequenceId child_id = child_metadata.sequence_id;
    if (parent == sequences_.end() || contains(child_id)) return false;
    const BlockTable& source = parent->second.text_table;
    // Sharing needs resident frames: a parent with any block in the swap
    // store cannot be forked until it is swapped back in.
    for (std::size_t k = 0; k < source.size(); ++k) {
        if (source.entries()[k].swap_slot) return false;
    }
    BlockTable child = source.fork(child_id);
    for (std::size_t k = 0; k < child.size(); ++k) allocator_->retain(child.entries()[k].physical_id);
    sequences_.try_emplace(child_id, SequenceState{std::move(child_metadata), std::move(child)});
    return true;
}

bool KVCacheManager::reserve_tokens(SequenceId sequence_id, std::uint32_t token_count) {
    const auto it = sequences_.find(sequence_id);
    const std::uint32_t tpb = pool_tokens_per_block(*allocator_);
    if (it == sequences_.end() || tpb == 0) return false;
    const std::uint32_t blocks = (token_count + tpb - 1) / tpb;
    // All or nothing: the capacity check comes before the first allocation.
    if (!allocator_->can_allocate(blocks)) return false;
    BlockTable& table = it->second.text_table;
    // New blocks continue the table's logical numbering.
    LogicalBlock next;
    next.sequence_id = sequence_id;
    next.cache_kind = table.cache_kind();
    next.token_count = tpb;
    next.index = static_cast<LogicalBlockIndex>(table.size());
    for (std::uint32_t k = 0; k < blocks; ++k, ++next.index) {
        const std::optional<PhysicalBlockId> frame = allocator_->allocate();
        if (!frame) return false;
        next.start_token = next.index * tpb;
        table.map(next, *frame, true);
    }
    return true;
}

std::optional<PhysicalBlockId> KVCacheManager::ensure_token_writable(SequenceId sequence_id,
                                                                     TokenPosition token_position,
                                                                     CacheKind /*cache_kind*/) {
    const auto it = sequences_.find(sequence_id);
    if (it == sequences_.end() || it->second.text_table.empty()) return std::nullopt;
    BlockTable& table = it->second.text_table;
    // The block size recorded with the table's own entries.
    const std::uint32_t tpb = table.entries().front().logical.token_count;
    BlockTableEntry* entry = tpb == 0 ? nullptr : table.mutable_entry(static_cast<LogicalBlockIndex>(token_position / tpb));
    if (entry == nullptr || entry->swap_slot) return std::nullopt;
    const PhysicalBlockInfo* held = allocator_->info(entry->physical_id);
    if (held == nullptr) return std::nullopt;
    // The frame's reference count decides, not the entry's writable flag: a
    // frame this sequence owns alone is written in place; a shared one is
    // first copied to a private frame, whose reference the sequence then
    // holds instead of the shared one.
    if (held->ref_count > 1) {
        const std::optional<PhysicalBlockId> own = allocator_->allocate();
        if (!own) return std::nullopt;
        allocator_->copy_block(entry->physical_id, *own);
        allocator_->release(std::exchange(entry->physical_id, *own));
    }
    entry->writable = true;
    return entry->physical_id;
}

std::uint32_t KVCacheManager::swap_out_sequence(SequenceId sequence_id) {
    const auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return 0;
    BlockTable& table = it->second.text_table;
    std::uint32_t moved = 0;
    for (std::size_t k = 0; k < table.size(); ++k) {
        BlockTableEntry& e = *table.mutable_entry(table.entries()[k].logical.index);
        if (e.swap_slot) continue;
        // The allocator keeps shared frames resident (a sibling still maps
        // them), so such entries stay as they are.
        e.swap_slot = allocator_->swap_out(e.physical_id);
        if (e.swap_slot) ++moved;
    }
    return moved;
}

bool KVCacheManager::swap_in_sequence(SequenceId sequence_id) {
    const auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return false;
    BlockTable& table = it->second.text_table;
    std::uint32_t missing = 0;
    for (std::size_t k = 0; k < table.size(); ++k) missing += table.entries()[k].swap_slot ? 1u : 0u;
    if (missing == 0) return true;
    // All or nothing, decided up front: enough free frames for every block.
    if (!allocator_->can_allocate(missing)) return false;
    for (std::size_t k = 0; k < table.size(); ++k) {
        BlockTableEntry& e = *table.mutable_entry(table.entries()[k].logical.index);
        if (!e.swap_slot) continue;
        const std::optional<PhysicalBlockId> frame = allocator_->swap_in(*e.swap_slot);
        if (!frame) return false;
        e.physical_id = *frame;
        e.swap_slot.reset();
    }
    return true;
}

void KVCacheManager::release_sequence(SequenceId sequence_id) {
    const auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return;
    // Resident blocks drop their frame reference; swapped ones free their slot.
    for (const BlockTableEntry& e : it->second.text_table.entries()) {
        if (e.swap_slot) {
            allocator_->discard_swapped(*e.swap_slot);
        } else {
            allocator_->release(e.physical_id);
        }
    }
    sequences_.erase(it);
}

std::optional<CacheView> KVCacheManager::cache_view(SequenceId sequence_id, CacheKind cache_kind) const {
    const auto it = sequences_.find(sequence_id);
    if (it == sequences_.end()) return std::nullopt;
    CacheView view;
    view.sequence_id = sequence_id;
    view.cache_kind = cache_kind;  // echoed; only the text stream has a table
    view.block_table = &it->second.text_table;
    view.allocator = allocator_;
    // Every frame of a pool has the same shape; an empty pool gives a view
    // whose layout is empty (and which is therefore not valid()).
    if (const PhysicalBlock* frame = allocator_->block(0)) view.layout.shape = frame->shape();
    return view;
}

bool KVCacheManager::contains(SequenceId sequence_id) const noexcept { return sequences_.count(sequence_id) != 0; }

const SequenceMetadata* KVCacheManager::metadata(SequenceId sequence_id) const noexcept {
    const auto it = sequences_.find(sequence_id);
    return it == sequences_.end() ? nullptr : &it->second.metadata;
}

}  // namespace qwenvl_paged

#pragma once
// Sequence cache lifecycle above the allocator, and the backend read contract
// CacheView (include/qwenvl_paged/KVCacheManager.h:23-253).

#include "qwenvl_paged/Block.h"
#include "qwenvl_paged/BlockTable.h"
#include "qwenvl_paged/CacheLayout.h"
#include "qwenvl_paged/MemoryAllocator.h"

#include <cstddef>
#include <cstdint>
#include <optional>
#include <unordered_map>
#include <vector>

namespace qwenvl_paged {

// Multimodal / M-RoPE metadata carried with a sequence (KVCacheManager.h:23-78).
struct MultimodalSpan {
    TokenPosition start_token{0};
    std::uint32_t token_count{0};
    std::uint32_t feature_index{0};
};

enum class PositionEncodingKind : std::uint8_t { Text1D, Image2D, Video3D };

struct Position3D {
    std::int64_t temporal{0};
    std::int64_t height{0};
    std::int64_t width{0};
};

struct PositionalEncodingSpan {
    TokenPosition start_token{0};
    std::uint32_t token_count{0};
    PositionEncodingKind kind{PositionEncodingKind::Text1D};
    Position3D origin{};
    Position3D stride{};
    // Addition (trailing, defaulted, so the reference's aggregate
    // initialisations still compile): the temporal, height and width extents
    // of an Image2D / Video3D span, needed to place its token i (row-major
    // over the grid); unused for Text1D.
    Position3D grid{};
};

struct PositionalEncodingMetadata {
    std::vector<PositionalEncodingSpan> spans;
};

struct SequenceMetadata {
    SequenceId sequence_id{0};
    RequestId request_id{0};
    std::vector<MultimodalSpan> multimodal_spans;
    PositionalEncodingMetadata positional_encoding;
};

// Read-only view of one sequence's cache: page table, allocator, layout.
// Borrowed: any cache mutation invalidates it (KVCacheManager.h:80-129).
struct CacheView {
    SequenceId sequence_id{0};
    CacheKind cache_kind{CacheKind::TextKV};
    const BlockTable* block_table{nullptr};
    const MemoryAllocator* allocator{nullptr};
    KVBlockLayout layout{};

    [[nodiscard]] bool valid() const noexcept;
    // Frame bytes of a logical block (device address for a device allocator),
    // or nullptr when unmapped or swapped out (src/KVCacheManager.cpp:11-25).
    [[nodiscard]] const std::byte* block_bytes(LogicalBlockIndex index) const noexcept;

    template <typename T>
    [[nodiscard]] const T* slot(KVStream stream, std::uint32_t layer, TokenPosition token,
                                std::uint32_t kv_head) const noexcept;
};

template <typename T>
const T* CacheView::slot(KVStream stream, std::uint32_t layer, TokenPosition token,
                         std::uint32_t kv_head) const noexcept {
    if (!valid() || sizeof(T) != layout.shape.bytes_per_element) return nullptr;
    const std::uint32_t tpb = layout.shape.tokens_per_block;
    const std::optional<std::size_t> offset = layout.element_offset(layer, stream, token % tpb, kv_head);
    if (!offset) return nullptr;
    const std::byte* bytes = block_bytes(static_cast<LogicalBlockIndex>(token / tpb));
    if (bytes == nullptr) return nullptr;
    return reinterpret_cast<const T*>(bytes) + *offset;
}

class KVCacheManager {
public:
    explicit KVCacheManager(MemoryAllocator& allocator);
    KVCacheManager(const KVCacheManager&) = delete;
    KVCacheManager& operator=(const KVCacheManager&) = delete;

    bool create_sequence(SequenceMetadata metadata);
    // Fails for an unknown parent, a taken child id, or a parent with swapped
    // blocks (KVCacheManager.h:185-192).
    bool fork_sequence(SequenceId parent_id, SequenceMetadata child_metadata);
    bool reserve_tokens(SequenceId sequence_id, std::uint32_t token_count);
    // Copy-on-write point (src/KVCacheManager.cpp:104-151).
    [[nodiscard]] std::optional<PhysicalBlockId> ensure_token_writable(SequenceId sequence_id,
                                                                       TokenPosition token_position,
                                                                       CacheKind cache_kind = CacheKind::TextKV);
    std::uint32_t swap_out_sequence(SequenceId sequence_id);
    bool swap_in_sequence(SequenceId sequence_id);
    void release_sequence(SequenceId sequence_id);
    [[nodiscard]] std::optional<CacheView> cache_view(SequenceId sequence_id,
                                                      CacheKind cache_kind = CacheKind::TextKV) const;
    [[nodiscard]] bool contains(SequenceId sequence_id) const noexcept;

    // Addition: the metadata a sequence was created with (the reference stores
    // it without a getter), for M-RoPE position materialisation.
    [[nodiscard]] const SequenceMetadata* metadata(SequenceId sequence_id) const noexcept;

private:
    struct SequenceState {
        SequenceMetadata metadata{};
        BlockTable text_table;
    };

    MemoryAllocator* allocator_{nullptr};
    std::unordered_map<SequenceId, SequenceState> sequences_;
};

}  // namespace qwenvl_paged

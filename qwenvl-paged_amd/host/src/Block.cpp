// Block shape and physical block storage (src/Block.cpp of the reference).
#include "qwenvl_paged/Block.h"

#include <cstdlib>
#include <utility>

namespace qwenvl_paged {

std::size_t BlockShape::byte_size() const noexcept {
    // K and V for every layer, head and token slot: the factor of two.
    return static_cast<std::size_t>(tokens_per_block) * num_layers * num_kv_heads * head_dim * bytes_per_element *
           2u;
}

bool LogicalBlock::empty() const noexcept { return token_count == 0; }

namespace {

std::size_t round_up(std::size_t value, std::size_t alignment) noexcept {
    return alignment == 0 ? value : (value + alignment - 1) / alignment * alignment;
}

}  // namespace

void PhysicalBlock::Release::operator()(std::byte* p) const noexcept {
    if (owned) std::free(p);
}

PhysicalBlock::PhysicalBlock(PhysicalBlockId id, BlockShape shape, HostMemoryOptions memory_options)
    : id_(id), shape_(shape), memory_options_(memory_options) {
    const std::size_t alignment =
        memory_options_.alignment_bytes == 0 ? kDefaultBlockAlignmentBytes : memory_options_.alignment_bytes;
    // aligned_alloc wants a size that is a multiple of the alignment, and
    // never zero.
    std::size_t bytes = round_up(shape_.byte_size(), alignment);
    if (bytes == 0) bytes = alignment;
    storage_ = std::unique_ptr<std::byte, Release>(static_cast<std::byte*>(std::aligned_alloc(alignment, bytes)),
                                                   Release{true});
    size_bytes_ = bytes;
}

PhysicalBlock::PhysicalBlock(PhysicalBlockId id, BlockShape shape, HostMemoryOptions memory_options,
                             std::byte* frame, std::size_t size_bytes)
    : id_(id),
      shape_(shape),
      memory_options_(memory_options),
      size_bytes_(size_bytes),
      placement_(BlockPlacement::Device),
      storage_(frame, Release{false}) {}

PhysicalBlockId PhysicalBlock::id() const noexcept { return id_; }
const BlockShape& PhysicalBlock::shape() const noexcept { return shape_; }
std::byte* PhysicalBlock::data() noexcept { return storage_.get(); }
const std::byte* PhysicalBlock::data() const noexcept { return storage_.get(); }
std::size_t PhysicalBlock::size_bytes() const noexcept { return size_bytes_; }
std::size_t PhysicalBlock::alignment_bytes() const noexcept { return memory_options_.alignment_bytes; }
bool PhysicalBlock::pinned_memory_requested() const noexcept { return memory_options_.prefer_pinned_memory; }
BlockPlacement PhysicalBlock::placement() const noexcept { return placement_; }

void PhysicalBlock::swap(PhysicalBlock& other) noexcept {
    // The id stays with the block; the storage and what describes it move.
    std::swap(shape_, other.shape_);
    std::swap(memory_options_, other.memory_options_);
    std::swap(size_bytes_, other.size_bytes_);
    std::swap(placement_, other.placement_);
    storage_.swap(other.storage_);
}

}  // namespace qwenvl_paged

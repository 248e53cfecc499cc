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

// Bytes of a host frame for `shape`: whole alignment units, at least one, so
// the request is one std::aligned_alloc accepts and data() is never null,
// even for a shape with a zero extent.
std::size_t host_frame_bytes(const BlockShape& shape, std::size_t alignment) noexcept {
    const std::size_t units = (shape.byte_size() + alignment - 1) / alignment;
    return (units == 0 ? 1 : units) * alignment;
}

}  // namespace

void PhysicalBlock::Release::operator()(std::byte* p) const noexcept {
    if (owned) std::free(p);
}

PhysicalBlock::PhysicalBlock(PhysicalBlockId id, BlockShape shape, HostMemoryOptions memory_options)
    : id_(id), shape_(shape), memory_options_(memory_options) {
    // An alignment of 0 in the options means the library default; the options
    // themselves are kept as given (alignment_bytes() reports them).
    const std::size_t alignment =
        memory_options_.alignment_bytes == 0 ? kDefaultBlockAlignmentBytes : memory_options_.alignment_bytes;
    size_bytes_ = host_frame_bytes(shape_, alignment);
    storage_ = std::unique_ptr<std::byte, Release>(
        static_cast<std::byte*>(std::aligned_alloc(alignment, size_bytes_)), Release{true});
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
    // Exchanges frames: storage, padded size, placement, and the shape and
    // options that describe the bytes. Ids are not exchanged, so each object
    // still answers to the slot the allocator keeps it in.
    std::swap(shape_, other.shape_);
    std::swap(memory_options_, other.memory_options_);
    std::swap(size_bytes_, other.size_bytes_);
    std::swap(placement_, other.placement_);
    storage_.swap(other.storage_);
}

}  // namespace qwenvl_paged

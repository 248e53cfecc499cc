#pragma once
// Core identifiers, block shape and physical block storage.
//
// Public API of include/qwenvl_paged/Block.h in the QwenVL-Paged tree
// (Block.h:10-166), with one addition: a PhysicalBlock can also be a view of a
// frame of the HBM block pool (BlockPlacement::Device), in which case data()
// is a device address. Host blocks behave exactly like the reference's
// (std::aligned_alloc storage, size rounded up to the alignment).

#include <cstddef>
#include <cstdint>
#include <memory>

namespace qwenvl_paged {

using RequestId = std::uint64_t;
using SequenceId = std::uint64_t;
using TokenPosition = std::uint32_t;
using LogicalBlockIndex = std::uint32_t;
using PhysicalBlockId = std::uint32_t;
using SwapSlotId = std::uint64_t;

inline constexpr std::size_t kDefaultBlockAlignmentBytes = 256;

// Kind of cache data held by a block (Block.h:26-31).
enum class CacheKind : std::uint8_t { TextKV, VisionKV, RopeState, Auxiliary };

// Lifecycle state of a frame in the pool (Block.h:36-41).
enum class BlockState : std::uint8_t { Free, Active, Shared, Swapped };

// Where a block's bytes live.
enum class BlockPlacement : std::uint8_t {
    Host,   // std::aligned_alloc storage, host-dereferenceable (the reference's)
    Device  // a frame of the HBM pool; data() is a device address
};

// Static shape of one cache block (Block.h:46-57).
struct BlockShape {
    std::uint32_t tokens_per_block{0};
    std::uint32_t num_layers{0};
    std::uint32_t num_kv_heads{0};
    std::uint32_t head_dim{0};
    std::uint32_t bytes_per_element{0};

    // Bytes of K and V for every layer, kv head and token slot (src/Block.cpp:8-13).
    [[nodiscard]] std::size_t byte_size() const noexcept;
};

// Host allocation policy (Block.h:67-70). prefer_pinned_memory is recorded and
// reported, as in the reference; pinned host memory for swapped blocks is the
// job of PinnedSwapBackend.
struct HostMemoryOptions {
    std::size_t alignment_bytes{kDefaultBlockAlignmentBytes};
    bool prefer_pinned_memory{false};
};

// Virtual page of a sequence (Block.h:78-89).
struct LogicalBlock {
    SequenceId sequence_id{0};
    LogicalBlockIndex index{0};
    CacheKind cache_kind{CacheKind::TextKV};
    TokenPosition start_token{0};
    std::uint32_t token_count{0};

    [[nodiscard]] bool empty() const noexcept;
};

// Storage of one physical block (Block.h:99-166).
class PhysicalBlock {
public:
    // Host block: aligned host allocation of byte_size() rounded up to the
    // alignment (0 selects 256), never zero bytes (src/Block.cpp:30-44).
    PhysicalBlock(PhysicalBlockId id, BlockShape shape, HostMemoryOptions memory_options = {});

    // Device frame view: `frame` is the frame's device address inside a pool
    // owned elsewhere, `size_bytes` the pool stride. The block does not own it.
    PhysicalBlock(PhysicalBlockId id, BlockShape shape, HostMemoryOptions memory_options, std::byte* frame,
                  std::size_t size_bytes);

    ~PhysicalBlock() = default;
    PhysicalBlock(const PhysicalBlock&) = delete;
    PhysicalBlock& operator=(const PhysicalBlock&) = delete;
    PhysicalBlock(PhysicalBlock&&) noexcept = default;
    PhysicalBlock& operator=(PhysicalBlock&&) noexcept = default;

    [[nodiscard]] PhysicalBlockId id() const noexcept;
    [[nodiscard]] const BlockShape& shape() const noexcept;
    [[nodiscard]] std::byte* data() noexcept;
    [[nodiscard]] const std::byte* data() const noexcept;
    [[nodiscard]] std::size_t size_bytes() const noexcept;
    // The alignment as requested in the options (0 stays 0, like the reference).
    [[nodiscard]] std::size_t alignment_bytes() const noexcept;
    [[nodiscard]] bool pinned_memory_requested() const noexcept;
    [[nodiscard]] BlockPlacement placement() const noexcept;

    // Exchanges storage (and its description) with another block; ids stay.
    void swap(PhysicalBlock& other) noexcept;

private:
    struct Release {
        bool owned{true};
        void operator()(std::byte* p) const noexcept;
    };

    PhysicalBlockId id_{0};
    BlockShape shape_{};
    HostMemoryOptions memory_options_{};
    std::size_t size_bytes_{0};
    BlockPlacement placement_{BlockPlacement::Host};
    std::unique_ptr<std::byte, Release> storage_{nullptr, Release{}};
};

}  // namespace qwenvl_paged

#pragma once
// Element order inside a block (include/qwenvl_paged/CacheLayout.h:14-79):
//
//     [layer][K|V][token_in_block][kv_head][head_dim]
//
// Strides and offsets are in elements. The decode kernels take exactly these
// four strides as arguments (qvp_decode_args head/token/stream/layer_stride).

#include "qwenvl_paged/Block.h"

#include <cstddef>
#include <cstdint>
#include <optional>

namespace qwenvl_paged {

enum class KVStream : std::uint8_t { Key, Value };

inline constexpr std::uint32_t kKVStreamCount = 2;

struct KVBlockLayout {
    BlockShape shape{};

    [[nodiscard]] std::size_t head_stride() const noexcept;
    [[nodiscard]] std::size_t token_stride() const noexcept;
    [[nodiscard]] std::size_t stream_stride() const noexcept;
    [[nodiscard]] std::size_t layer_stride() const noexcept;
    [[nodiscard]] std::size_t element_count() const noexcept;

    // Offset of one (layer, stream, token, head) vector, or nullopt when a
    // coordinate is outside the shape (src/CacheLayout.cpp:25-38).
    [[nodiscard]] std::optional<std::size_t> element_offset(std::uint32_t layer, KVStream stream,
                                                            std::uint32_t token_in_block,
                                                            std::uint32_t kv_head) const noexcept;
};

}  // namespace qwenvl_paged

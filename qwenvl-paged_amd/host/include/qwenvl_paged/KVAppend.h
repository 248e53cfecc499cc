#pragma once
// Writes a decode step's new K and V rows into the paged cache.
//
// The reference leaves this step to its callers: its harnesses ask
// KVCacheManager::ensure_token_writable for the token's frame (copying a shared
// block first, src/KVCacheManager.cpp:104-151) and store head_dim elements per
// (layer, stream, kv head) at KVBlockLayout::element_offset
// (tests/PagedAttention.test.cpp:97-127, tests/EndToEnd.test.cpp:157-179).
// KVAppendBatch does the same for a whole step: the copy-on-write decisions on
// the host, then, for device-placed frames, one launch of the stores
// (qvp_append_kv) on the allocator's engine stream, ordered after the step's
// queued block copies and before any later decode on that stream. A decode
// step's copies (up to 128, with up to 128 tokens, none written into a frame
// a copy reads) run in that same launch (qvp_copy_append_kv). For host-placed
// frames the stores are memcpy calls, as in the harnesses.

#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"

#include <cstdint>
#include <string>
#include <vector>

namespace qwenvl_paged {

class KVAppendBatch {
public:
    // Token positions[i] of sequence sequences[i] receives row i of k and v:
    // [n][layer_count][num_kv_heads][head_dim] elements of the cache's element
    // size, in device memory for a device-placement allocator and in host
    // memory for a host-placement one; layers [first_layer, first_layer +
    // layer_count) of the frame are written. Positions must already be
    // reserved (KVCacheManager::reserve_tokens).
    //
    // Refused (false, no K/V written, nothing enqueued) for unequal list
    // sizes, a null pointer, a layer range outside the block shape, an unknown
    // sequence, a position whose block is unmapped or swapped out, or a
    // (sequence, position) pair given twice. If ensure_token_writable itself
    // fails (a shared block with no free frame for its copy) the call returns
    // false after the tokens before it were made writable: those sequences
    // then own private copies of their blocks, with unchanged contents, and
    // still no K/V has been written.
    bool append(KVCacheManager& cache, MemoryAllocator& allocator, const std::vector<SequenceId>& sequences,
                const std::vector<TokenPosition>& positions, std::uint32_t first_layer, std::uint32_t layer_count,
                const void* k, const void* v);

    [[nodiscard]] const std::string& last_error() const noexcept;

private:
    bool fail(std::string msg);

    std::vector<std::uint32_t> frames_;
    std::vector<std::uint32_t> slots_;
    std::vector<PhysicalBlockId> cow_src_;  // the step's copies run in the append's launch
    std::vector<PhysicalBlockId> cow_dst_;
    std::string last_error_;
};

}  // namespace qwenvl_paged

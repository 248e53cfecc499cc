// One step's K/V stores (the write_head_vector / write_token loops of the
// reference's harnesses, tests/PagedAttention.test.cpp:97-127 and
// tests/EndToEnd.test.cpp:157-179), batched.
#include "qwenvl_paged/KVAppend.h"

#include "qvp.h"

#include <algorithm>
#include <cstring>
#include <utility>

namespace qwenvl_paged {

namespace {

// Limits of qvp_copy_append_kv (one decode step): list lengths, tokens per
// block and the frame stride.
constexpr std::size_t kFusedCopyLimit = 128;
constexpr std::size_t kFusedRowLimit = 128;
constexpr std::uint32_t kFusedSlotLimit = 64;
constexpr std::uint64_t kFusedStrideLimit = 0x80000000ull - 8192;

}  // namespace


bool KVAppendBatch::fail(std::string msg) {
    last_error_ = std::move(msg);
    return false;
}

const std::string& KVAppendBatch::last_error() const noexcept { return last_error_; }

bool KVAppendBatch::append(KVCacheManager& cache, MemoryAllocator& allocator, const std::vector<SequenceId>& sequences,
                           const std::vector<TokenPosition>& positions, std::uint32_t first_layer,
                           std::uint32_t layer_count, const void* k, const void* v) {
    if (sequences.size() != positions.size()) return fail("sequences and positions differ in size");
    if (sequences.empty()) return true;
    if (k == nullptr || v == nullptr) return fail("null k or v");
    const std::optional<CacheView> first_view = cache.cache_view(sequences.front());
    if (!first_view || !first_view->valid()) return fail("unknown sequence");
    const KVBlockLayout layout = first_view->layout;
    const BlockShape shape = layout.shape;
    if (layer_count == 0 || static_cast<std::uint64_t>(first_layer) + layer_count > shape.num_layers) {
        return fail("layer range outside the block shape");
    }
    if (shape.tokens_per_block == 0) return fail("zero tokens per block");
    const bool device = allocator.placement() == BlockPlacement::Device;
    if (device && shape.bytes_per_element != 4 && shape.bytes_per_element != 2) {
        return fail("element size must be 2 or 4 bytes");
    }
    if (device && !allocator.ok()) return fail("allocator: " + allocator.last_error());

    // Everything that can be checked without side effects is checked before
    // the first copy-on-write decision.
    // A prompt's rows come as runs of one sequence: its view is looked up once
    // per run.
    std::vector<std::pair<SequenceId, TokenPosition>> keys(sequences.size());
    std::optional<CacheView> view;
    for (std::size_t i = 0; i < sequences.size(); ++i) {
        if (i == 0 || sequences[i] != sequences[i - 1]) {
            view = cache.cache_view(sequences[i]);
            if (!view || !view->valid()) return fail("unknown sequence " + std::to_string(sequences[i]));
        }
        const LogicalBlockIndex index = positions[i] / shape.tokens_per_block;
        if (!view->block_table->lookup(index)) {
            return fail("position " + std::to_string(positions[i]) + " of sequence " + std::to_string(sequences[i]) +
                        " has no mapped block");
        }
        keys[i] = {sequences[i], positions[i]};
    }
    std::sort(keys.begin(), keys.end());
    if (std::adjacent_find(keys.begin(), keys.end()) != keys.end()) return fail("a token is given twice");

    // After ensure_token_writable returned a frame for a token, the block is
    // the sequence's own (KVCacheManager.cpp:104-151 copies a shared block
    // and remaps it), so the next token of the same (sequence, block) gets the
    // same frame without a second call.
    frames_.resize(sequences.size());
    slots_.resize(sequences.size());
    for (std::size_t i = 0; i < sequences.size(); ++i) {
        const LogicalBlockIndex index = positions[i] / shape.tokens_per_block;
        if (i > 0 && sequences[i] == sequences[i - 1] && index == positions[i - 1] / shape.tokens_per_block) {
            frames_[i] = frames_[i - 1];
        } else {
            const std::optional<PhysicalBlockId> frame = cache.ensure_token_writable(sequences[i], positions[i]);
            if (!frame) {
                return fail("no writable frame for position " + std::to_string(positions[i]) + " of sequence " +
                            std::to_string(sequences[i]));
            }
            frames_[i] = *frame;
        }
        slots_[i] = positions[i] % shape.tokens_per_block;
    }

    const std::size_t bpe = shape.bytes_per_element;
    const std::size_t row = static_cast<std::size_t>(shape.head_dim) * bpe;
    if (!device) {
        const auto* ks = static_cast<const std::byte*>(k);
        const auto* vs = static_cast<const std::byte*>(v);
        for (std::size_t i = 0; i < frames_.size(); ++i) {
            std::byte* base = allocator.block(frames_[i])->data();
            for (std::uint32_t l = 0; l < layer_count; ++l) {
                for (const KVStream stream : {KVStream::Key, KVStream::Value}) {
                    const std::byte* src = (stream == KVStream::Key ? ks : vs) +
                                           (i * layer_count + l) * static_cast<std::size_t>(shape.num_kv_heads) * row;
                    for (std::uint32_t h = 0; h < shape.num_kv_heads; ++h) {
                        const std::optional<std::size_t> off =
                            layout.element_offset(first_layer + l, stream, slots_[i], h);
                        std::memcpy(base + *off * bpe, src + h * row, row);
                    }
                }
            }
        }
        return true;
    }

    // The copies ensure_token_writable queued run first, on the same stream,
    // and the frames written here wait for any swap still moving them. A
    // step's copies (the last queued batch, when no token row goes into a
    // frame one of them reads) run in the append's own launch: each chunk of a
    // destination frame is copied and then overwritten by its rows by one
    // workgroup, so the bytes equal those of the two launches in order.
    const std::uint64_t align = reinterpret_cast<std::uintptr_t>(allocator.device_base()) |
                                reinterpret_cast<std::uintptr_t>(k) | reinterpret_cast<std::uintptr_t>(v) |
                                allocator.block_stride() | row | layout.head_stride() * bpe |
                                layout.token_stride() * bpe | layout.stream_stride() * bpe |
                                layout.layer_stride() * bpe;
    const bool fuse = frames_.size() <= kFusedRowLimit && align % 16 == 0 &&
                      shape.tokens_per_block <= kFusedSlotLimit && allocator.block_stride() <= kFusedStrideLimit;
    if (fuse ? !allocator.flush_except_last_copies(kFusedCopyLimit, frames_, cow_src_, cow_dst_)
             : !allocator.flush()) {
        return fail("flush: " + allocator.last_error());
    }
    if (!fuse) {
        cow_src_.clear();
        cow_dst_.clear();
    }
    if (!allocator.order_frame_writes(frames_)) return fail("flush: " + allocator.last_error());
    qvp_append_args a{};
    a.kv_base = allocator.device_base();
    a.block_stride = allocator.block_stride();
    a.num_blocks = allocator.stats().total_blocks;
    a.kv_dtype = bpe == 4 ? QVP_DTYPE_F32 : QVP_DTYPE_BF16;  // a byte copy: only the size matters
    a.num_layers = shape.num_layers;
    a.first_layer = first_layer;
    a.layer_count = layer_count;
    a.num_kv_heads = shape.num_kv_heads;
    a.head_dim = shape.head_dim;
    a.tokens_per_block = shape.tokens_per_block;
    a.head_stride = layout.head_stride();
    a.token_stride = layout.token_stride();
    a.stream_stride = layout.stream_stride();
    a.layer_stride = layout.layer_stride();
    a.k = k;
    a.v = v;
    if (!cow_src_.empty()) {
        if (qvp_copy_append_kv(&a, cow_src_.data(), cow_dst_.data(), static_cast<std::uint32_t>(cow_src_.size()),
                               allocator.block_stride(), frames_.data(), slots_.data(),
                               static_cast<std::uint32_t>(frames_.size()), allocator.stream()) != QVP_OK) {
            return fail(std::string("copy + append: ") + qvp_last_error());
        }
        return true;
    }
    if (qvp_append_kv(&a, frames_.data(), slots_.data(), static_cast<std::uint32_t>(frames_.size()),
                      allocator.stream()) != QVP_OK) {
        return fail(std::string("append: ") + qvp_last_error());
    }
    return true;
}

}  // namespace qwenvl_paged

// GPU paged-attention decode behind the reference interface
// (include/qwenvl_paged/PagedAttention.h:53-127): the checks are the
// reference's, the arithmetic is libqvp's (qvp_pack + qvp_paged_decode).
#include "qwenvl_paged/PagedAttention.h"

#include "qvp.h"

#include <algorithm>
#include <cstring>
#include <type_traits>
#include <utility>

namespace qwenvl_paged {

bf16::bf16(float f) noexcept {
    std::uint32_t u;
    std::memcpy(&u, &f, sizeof u);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        bits = static_cast<std::uint16_t>((u >> 16) | 0x40u);
    } else {
        bits = static_cast<std::uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
    }
}

bf16::operator float() const noexcept {
    const std::uint32_t u = static_cast<std::uint32_t>(bits) << 16;
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
}

// binary16 from float, rounding to nearest even at the 13 dropped mantissa
// bits (normal results) or at the bits below 2^-24 (subnormal results).
f16::f16(float f) noexcept {
    std::uint32_t u;
    std::memcpy(&u, &f, sizeof u);
    const std::uint32_t sign = (u >> 16) & 0x8000u;
    const std::uint32_t mag = u & 0x7fffffffu;
    if (mag > 0x7f800000u) {
        bits = static_cast<std::uint16_t>(sign | 0x7e00u | ((mag >> 13) & 0x3ffu));  // quiet NaN
    } else if (mag >= 0x477ff000u) {
        bits = static_cast<std::uint16_t>(sign | 0x7c00u);  // at or past 65520: infinity
    } else if (mag >= 0x38800000u) {
        // Normal: rebias the exponent (127 -> 15) after rounding; a carry out
        // of the mantissa moves into the exponent, as it should.
        const std::uint32_t r = mag + 0xfffu + ((mag >> 13) & 1u);
        bits = static_cast<std::uint16_t>(sign | ((r - 0x38000000u) >> 13));
    } else {
        // Subnormal or zero: the value in units of 2^-24 is the full
        // mantissa shifted right by 126 - exponent.
        const std::uint32_t e = mag >> 23;
        const std::uint32_t shift = 126u - e;
        std::uint32_t m = 0;
        if (shift < 25u) {
            const std::uint32_t full = (mag & 0x7fffffu) | 0x800000u;
            m = full >> shift;
            const std::uint32_t rem = full & ((1u << shift) - 1u);
            const std::uint32_t half = 1u << (shift - 1u);
            if (rem > half || (rem == half && (m & 1u))) ++m;
        }
        bits = static_cast<std::uint16_t>(sign | m);
    }
}

f16::operator float() const noexcept {
    const std::uint32_t sign = static_cast<std::uint32_t>(bits & 0x8000u) << 16;
    const std::uint32_t e = (bits >> 10) & 0x1fu;
    const std::uint32_t m = bits & 0x3ffu;
    std::uint32_t u;
    if (e == 0x1fu) {
        u = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        u = sign | ((e + 112u) << 23) | (m << 13);
    } else {
        // Subnormal: m x 2^-24, exact in float.
        const float v = static_cast<float>(m) * 5.9604644775390625e-8f;
        std::memcpy(&u, &v, sizeof u);
        u |= sign;
    }
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
}

namespace {

thread_local std::string g_last_error;

bool refuse(std::string msg) {
    g_last_error = std::move(msg);
    return false;
}

// Frames of logical blocks 0 .. ceil(ctx / tpb) - 1, QVP_UNMAPPED_BLOCK for a
// block that is unmapped or swapped out (the packer then refuses the batch).
// A table that grew by appending (entry k holds logical block k, the usual
// case) is read in one pass over its entries; one with holes goes through
// entry() per block.
void collect_blocks(const CacheView& view, std::uint32_t context_len, std::vector<std::uint32_t>& ids) {
    const std::uint32_t tpb = view.layout.shape.tokens_per_block;
    const std::uint32_t needed = (context_len + tpb - 1) / tpb;
    const std::vector<BlockTableEntry>& entries = view.block_table->entries();
    const std::size_t base = ids.size();
    ids.resize(base + needed);
    std::uint32_t* out = ids.data() + base;
    std::uint32_t j = 0;
    const std::uint32_t dense = static_cast<std::uint32_t>(std::min<std::size_t>(needed, entries.size()));
    for (; j < dense; ++j) {
        const BlockTableEntry& e = entries[j];
        if (e.logical.index != j) break;
        out[j] = e.swap_slot.has_value() ? QVP_UNMAPPED_BLOCK : e.physical_id;
    }
    for (; j < needed; ++j) {
        const BlockTableEntry* e = view.block_table->entry(j);
        out[j] = (e == nullptr || e->swap_slot.has_value()) ? QVP_UNMAPPED_BLOCK : e->physical_id;
    }
}

// Grows a device (or pinned host) buffer to at least `bytes`.
bool grow(void*& ptr, std::size_t& have, std::size_t bytes, bool pinned) {
    if (have >= bytes) return true;
    (void)(pinned ? qvp_host_free(ptr) : qvp_free(ptr));
    ptr = nullptr;
    have = 0;
    if ((pinned ? qvp_host_alloc(&ptr, bytes) : qvp_malloc(&ptr, bytes)) != QVP_OK) return false;
    have = bytes;
    return true;
}

// Device staging for the single-sequence entry point, one per thread: query
// and output buffers, and for views over host-placed frames a pinned and a
// device copy of the frames' layer slices, their packed batch and a stream.
struct SingleScratch {
    PagedAttentionBatch batch;
    void* dq{nullptr};
    void* dout{nullptr};
    std::size_t dq_bytes{0};
    std::size_t dout_bytes{0};
    void* host_slices{nullptr};
    void* dev_slices{nullptr};
    std::size_t host_slice_bytes{0};
    std::size_t dev_slice_bytes{0};
    qvp_batch* staged{nullptr};
    void* stream{nullptr};

    ~SingleScratch() {
        if (stream != nullptr) (void)qvp_stream_synchronize(stream);
        (void)qvp_batch_destroy(staged);
        (void)qvp_free(dq);
        (void)qvp_free(dout);
        (void)qvp_host_free(host_slices);
        (void)qvp_free(dev_slices);
        if (stream != nullptr) (void)qvp_stream_destroy(stream);
    }

    bool ensure(std::size_t q_bytes, std::size_t o_bytes) {
        return grow(dq, dq_bytes, q_bytes, false) && grow(dout, dout_bytes, o_bytes, false);
    }
};

template <typename T>
constexpr ElementType element_type_of() {
    return std::is_same<T, float>::value ? ElementType::F32
                                         : (std::is_same<T, f16>::value ? ElementType::F16 : ElementType::BF16);
}

// Decode over host-placed frames: the layer's K/V slice of every block the
// context needs (one contiguous run per block in the [layer][K|V][token]
// [head][dim] order) is copied into pinned memory, uploaded in one transfer
// and decoded as a pool of those slices (block i of the context is slice i,
// one layer per slice). The checks already ran; every block is resolved
// before anything is copied, so a refusal leaves `out` untouched.
template <typename T>
bool decode_host_frames(const CacheView& view, const T* query, const PagedAttentionParams& params, T* out,
                        SingleScratch& scratch) {
    const KVBlockLayout& layout = view.layout;
    const BlockShape& shape = layout.shape;
    const std::uint32_t tpb = shape.tokens_per_block;
    const std::uint32_t needed = (params.context_len + tpb - 1) / tpb;
    const std::size_t slice = layout.layer_stride() * shape.bytes_per_element;
    const std::size_t layer_offset = static_cast<std::size_t>(params.layer) * slice;
    std::vector<const std::byte*> frames(needed, nullptr);
    for (std::uint32_t j = 0; j < needed; ++j) {
        const BlockTableEntry* e = view.block_table->entry(j);
        const PhysicalBlock* b = (e == nullptr || e->swap_slot) ? nullptr : view.allocator->block(e->physical_id);
        if (b == nullptr || b->data() == nullptr || b->size_bytes() < layer_offset + slice) {
            return refuse("a block of the context is unmapped or swapped out");
        }
        frames[j] = b->data() + layer_offset;
    }
    if (scratch.stream == nullptr && qvp_stream_create(&scratch.stream) != QVP_OK) {
        return refuse(std::string("stream: ") + qvp_last_error());
    }
    if (scratch.staged == nullptr && qvp_batch_create(&scratch.staged) != QVP_OK) {
        return refuse(std::string("batch: ") + qvp_last_error());
    }
    const std::size_t total = slice * needed;
    if (!grow(scratch.host_slices, scratch.host_slice_bytes, total, true) ||
        !grow(scratch.dev_slices, scratch.dev_slice_bytes, total, false)) {
        return refuse(std::string("frame staging: ") + qvp_last_error());
    }
    // The previous call synchronized its stream before returning, so the
    // pinned buffer is free to refill.
    auto* staging = static_cast<std::byte*>(scratch.host_slices);
    for (std::uint32_t j = 0; j < needed; ++j) std::memcpy(staging + j * slice, frames[j], slice);
    const std::size_t bytes = static_cast<std::size_t>(params.num_query_heads) * shape.head_dim * sizeof(T);
    void* stream = scratch.stream;
    if (qvp_memcpy_htod(scratch.dev_slices, staging, total, stream) != QVP_OK ||
        qvp_memcpy_htod(scratch.dq, query, bytes, stream) != QVP_OK) {
        // A first copy may be under way: the staging is reused by the next call.
        const std::string why = std::string("upload: ") + qvp_last_error();
        (void)qvp_stream_synchronize(stream);
        return refuse(why);
    }
    std::vector<std::uint32_t> ids(needed);
    for (std::uint32_t j = 0; j < needed; ++j) ids[j] = j;
    const std::uint32_t cu[2] = {0, needed};
    const std::uint32_t lens[1] = {params.context_len};
    qvp_decode_args args{};
    args.query = scratch.dq;
    args.out = scratch.dout;
    args.kv_base = scratch.dev_slices;
    args.block_stride = slice;
    args.batch = scratch.staged;
    args.kv_dtype = static_cast<std::uint32_t>(element_type_of<T>());
    args.out_dtype = args.kv_dtype;
    args.layer = 0;
    args.num_layers = 1;
    args.num_query_heads = params.num_query_heads;
    args.num_kv_heads = shape.num_kv_heads;
    args.head_dim = shape.head_dim;
    args.tokens_per_block = tpb;
    args.head_stride = layout.head_stride();
    args.token_stride = layout.token_stride();
    args.stream_stride = layout.stream_stride();
    args.layer_stride = layout.layer_stride();
    args.scale = params.scale;
    if (qvp_pack_for_decode(scratch.staged, 1, ids.data(), cu, lens, tpb, needed, 0, &args, stream) != QVP_OK ||
        qvp_paged_decode(&args, stream) != QVP_OK) {
        (void)qvp_stream_synchronize(stream);
        return refuse(std::string("decode: ") + qvp_last_error());
    }
    if (qvp_memcpy_dtoh(out, scratch.dout, bytes, stream) != QVP_OK || qvp_stream_synchronize(stream) != QVP_OK) {
        return refuse(std::string("result download: ") + qvp_last_error());
    }
    return true;
}

}  // namespace

const std::string& paged_attention_last_error() { return g_last_error; }

template <typename T>
bool paged_attention_decode(const CacheView& view, const T* query, const PagedAttentionParams& params, T* out) {
    // Argument checks of the reference, in its order (PagedAttention.h:59-68).
    if (!view.valid() || query == nullptr || out == nullptr) return refuse("invalid view or null query/output");
    const BlockShape& shape = view.layout.shape;
    if (sizeof(T) != shape.bytes_per_element) return refuse("element size does not match the cache");
    if (params.context_len == 0) return refuse("context_len is 0");
    if (params.layer >= shape.num_layers) return refuse("layer outside the block shape");
    if (params.num_query_heads == 0 || params.num_query_heads % shape.num_kv_heads != 0) {
        return refuse("query heads do not group onto the kv heads");
    }
    thread_local SingleScratch scratch;
    const std::size_t bytes = static_cast<std::size_t>(params.num_query_heads) * shape.head_dim * sizeof(T);
    if (!scratch.ensure(bytes, bytes)) return refuse(std::string("device staging: ") + qvp_last_error());
    if (view.allocator->placement() != BlockPlacement::Device) {
        return decode_host_frames(view, query, params, out, scratch);
    }
    scratch.batch.set_cache_element_type(element_type_of<T>());
    void* stream = view.allocator->stream();
    if (qvp_memcpy_htod(scratch.dq, query, bytes, stream) != QVP_OK) {
        return refuse(std::string("query upload: ") + qvp_last_error());
    }
    if (!scratch.batch.decode({view}, {params.context_len}, params.layer, params.num_query_heads, params.scale,
                              scratch.dq, scratch.dout, element_type_of<T>())) {
        return refuse(scratch.batch.last_error());
    }
    if (qvp_memcpy_dtoh(out, scratch.dout, bytes, stream) != QVP_OK || qvp_stream_synchronize(stream) != QVP_OK) {
        return refuse(std::string("result download: ") + qvp_last_error());
    }
    return true;
}

template bool paged_attention_decode<float>(const CacheView&, const float*, const PagedAttentionParams&, float*);
template bool paged_attention_decode<bf16>(const CacheView&, const bf16*, const PagedAttentionParams&, bf16*);
template bool paged_attention_decode<f16>(const CacheView&, const f16*, const PagedAttentionParams&, f16*);

// ---------------------------------------------------------------------------

PagedAttentionBatch::PagedAttentionBatch() { (void)qvp_batch_create(&batch_); }

PagedAttentionBatch::~PagedAttentionBatch() { (void)qvp_batch_destroy(batch_); }

bool PagedAttentionBatch::fail(std::string msg) {
    last_error_ = std::move(msg);
    return false;
}

const std::string& PagedAttentionBatch::last_error() const noexcept { return last_error_; }
qvp_batch* PagedAttentionBatch::packed() const noexcept { return batch_; }
void PagedAttentionBatch::set_split_tokens(std::uint32_t tokens) noexcept { split_tokens_ = tokens; }
void PagedAttentionBatch::set_cache_element_type(ElementType type) noexcept {
    cache_type_override_ = static_cast<int>(type);
}

bool PagedAttentionBatch::pack(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                               std::uint32_t layer, std::uint32_t num_query_heads, const void* device_query,
                               void* device_out, int& cache_type, void*& stream) {
    if (batch_ == nullptr) return fail("no packed-batch object (device unavailable?)");
    if (views.empty() || views.size() != context_lens.size()) return fail("views and context_lens differ in size");
    if (device_query == nullptr || device_out == nullptr) return fail("null query or output buffer");
    const MemoryAllocator* allocator = views.front().allocator;
    if (allocator == nullptr) return fail("invalid view");
    const BlockShape shape = views.front().layout.shape;
    for (const CacheView& v : views) {
        if (!v.valid()) return fail("invalid view");
        if (v.allocator != allocator) return fail("views over different allocators");
        if (std::memcmp(&v.layout.shape, &shape, sizeof shape) != 0) return fail("views with different shapes");
    }
    if (allocator->placement() != BlockPlacement::Device || !allocator->ok()) {
        return fail("the decode needs a working device-placement allocator");
    }
    if (layer >= shape.num_layers) return fail("layer outside the block shape");
    if (num_query_heads == 0 || shape.num_kv_heads == 0 || num_query_heads % shape.num_kv_heads != 0) {
        return fail("query heads do not group onto the kv heads");
    }
    cache_type = shape.bytes_per_element == 4 ? QVP_DTYPE_F32 : QVP_DTYPE_BF16;
    if (cache_type_override_ >= 0) cache_type = cache_type_override_;
    if (qvp_dtype(cache_type) == QVP_DTYPE_F32 ? shape.bytes_per_element != 4 : shape.bytes_per_element != 2) {
        return fail("element type does not match the cache's element size");
    }

    ids_.clear();
    cu_.assign(1, 0);
    for (std::size_t b = 0; b < views.size(); ++b) {
        if (context_lens[b] == 0) return fail("context_len is 0");
        collect_blocks(views[b], context_lens[b], ids_);
        cu_.push_back(static_cast<std::uint32_t>(ids_.size()));
    }

    // Queued copy-on-write copies and swap traffic land before the kernels
    // read any frame.
    MemoryAllocator* mut = const_cast<MemoryAllocator*>(allocator);
    // The frames read here may still be coming back from the swap store.
    if (!mut->flush() || !mut->order_frame_reads(ids_)) return fail("flush: " + mut->last_error());
    stream = allocator->stream();
    const PhysicalBlock* frame0 = allocator->block(0);
    const std::uint32_t num_blocks = static_cast<std::uint32_t>(allocator->stats().total_blocks);
    if (frame0 == nullptr) return fail("empty pool");
    num_pool_blocks_ = num_blocks;
    return true;
}

bool PagedAttentionBatch::upload(const std::vector<std::uint32_t>& context_lens, std::uint32_t tokens_per_block,
                                 const qvp_decode_args* decode, void* stream) {
    // One upload per step: with the decode's arguments the pack also carries
    // that decode's work schedule.
    if (qvp_pack_for_decode(batch_, static_cast<std::uint32_t>(context_lens.size()),
                            ids_.empty() ? nullptr : ids_.data(), cu_.data(), context_lens.data(), tokens_per_block,
                            num_pool_blocks_, split_tokens_, decode, stream) != QVP_OK) {
        return fail(std::string("pack: ") + qvp_last_error());
    }
    return true;
}

bool PagedAttentionBatch::prepare(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                                  std::uint32_t layer, std::uint32_t num_query_heads, float scale,
                                  const void* device_query, void* device_out, ElementType out_type, void*& stream) {
    int cache_type = 0;
    if (!pack(views, context_lens, layer, num_query_heads, device_query, device_out, cache_type, stream)) return false;
    const KVBlockLayout& layout = views.front().layout;
    const BlockShape& shape = layout.shape;
    const MemoryAllocator* allocator = views.front().allocator;
    if (!args_) args_ = std::make_unique<qvp_decode_args>();
    qvp_decode_args& args = *args_;
    args = qvp_decode_args{};
    args.query = device_query;
    args.out = device_out;
    args.kv_base = allocator->device_base();
    args.block_stride = allocator->block_stride();
    args.batch = batch_;
    args.kv_dtype = static_cast<std::uint32_t>(cache_type);
    args.out_dtype = static_cast<std::uint32_t>(out_type);
    args.layer = layer;
    args.num_layers = shape.num_layers;
    args.num_query_heads = num_query_heads;
    args.num_kv_heads = shape.num_kv_heads;
    args.head_dim = shape.head_dim;
    args.tokens_per_block = shape.tokens_per_block;
    args.head_stride = layout.head_stride();
    args.token_stride = layout.token_stride();
    args.stream_stride = layout.stream_stride();
    args.layer_stride = layout.layer_stride();
    args.scale = scale;
    return true;
}

bool PagedAttentionBatch::decode(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                                 std::uint32_t layer, std::uint32_t num_query_heads, float scale,
                                 const void* device_query, void* device_out, ElementType out_type) {
    void* stream = nullptr;
    packed_ready_ = false;
    if (!prepare(views, context_lens, layer, num_query_heads, scale, device_query, device_out, out_type, stream)) {
        return false;
    }
    const qvp_decode_args* args = args_.get();
    if (!upload(context_lens, views.front().layout.shape.tokens_per_block, args, stream)) return false;
    if (qvp_paged_decode(args, stream) != QVP_OK) return fail(std::string("decode: ") + qvp_last_error());
    return true;
}

bool PagedAttentionBatch::pack_ahead(const std::vector<CacheView>& views,
                                     const std::vector<std::uint32_t>& context_lens, std::uint32_t layer,
                                     std::uint32_t num_query_heads, float scale, const void* device_query,
                                     void* device_out, ElementType out_type) {
    void* stream = nullptr;
    packed_ready_ = false;
    if (!prepare(views, context_lens, layer, num_query_heads, scale, device_query, device_out, out_type, stream)) {
        return false;
    }
    const qvp_decode_args* args = args_.get();
    if (qvp_pack_ahead(batch_, static_cast<std::uint32_t>(context_lens.size()), ids_.empty() ? nullptr : ids_.data(),
                       cu_.data(), context_lens.data(), views.front().layout.shape.tokens_per_block, num_pool_blocks_,
                       split_tokens_, args, stream) != QVP_OK) {
        return fail(std::string("pack: ") + qvp_last_error());
    }
    packed_stream_ = stream;
    packed_ready_ = true;
    return true;
}

bool PagedAttentionBatch::decode_packed() {
    if (!packed_ready_) return fail("nothing packed: call pack_ahead() first");
    packed_ready_ = false;
    const qvp_decode_args* args = args_.get();
    if (qvp_paged_decode(args, packed_stream_) != QVP_OK) return fail(std::string("decode: ") + qvp_last_error());
    return true;
}

bool PagedAttentionBatch::prefill(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                                  const std::vector<std::uint32_t>& first_new, std::uint32_t layer,
                                  std::uint32_t num_query_heads, float scale, const void* device_query,
                                  void* device_out, ElementType out_type) {
    packed_ready_ = false;
    if (first_new.size() != views.size()) return fail("views and first_new differ in size");
    for (std::size_t b = 0; b < first_new.size() && b < context_lens.size(); ++b) {
        if (first_new[b] >= context_lens[b]) return fail("first new position is not below the context length");
    }
    int cache_type = 0;
    void* stream = nullptr;
    if (!pack(views, context_lens, layer, num_query_heads, device_query, device_out, cache_type, stream)) return false;
    const KVBlockLayout& layout = views.front().layout;
    const BlockShape& shape = layout.shape;
    const MemoryAllocator* allocator = views.front().allocator;
    qvp_prefill_args args{};
    args.query = device_query;
    args.out = device_out;
    args.kv_base = allocator->device_base();
    args.block_stride = allocator->block_stride();
    args.batch = batch_;
    args.q_start = first_new.data();
    args.kv_dtype = static_cast<std::uint32_t>(cache_type);
    args.out_dtype = static_cast<std::uint32_t>(out_type);
    args.layer = layer;
    args.num_layers = shape.num_layers;
    args.num_query_heads = num_query_heads;
    args.num_kv_heads = shape.num_kv_heads;
    args.head_dim = shape.head_dim;
    args.tokens_per_block = shape.tokens_per_block;
    args.head_stride = layout.head_stride();
    args.token_stride = layout.token_stride();
    args.stream_stride = layout.stream_stride();
    args.layer_stride = layout.layer_stride();
    args.scale = scale;
    if (!upload(context_lens, shape.tokens_per_block, nullptr, stream)) return false;
    if (qvp_paged_prefill(&args, stream) != QVP_OK) return fail(std::string("prefill: ") + qvp_last_error());
    return true;
}

}  // namespace qwenvl_paged

// GPU paged-attention decode behind the reference interface
// (include/qwenvl_paged/PagedAttention.h:53-127): the checks are the
// reference's, the arithmetic is libqvp's (qvp_pack + qvp_paged_decode).
#include "qwenvl_paged/PagedAttention.h"

#include "qvp.h"

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

namespace {

thread_local std::string g_last_error;

bool refuse(std::string msg) {
    g_last_error = std::move(msg);
    return false;
}

// Frames of logical blocks 0 .. ceil(ctx / tpb) - 1, QVP_UNMAPPED_BLOCK for a
// block that is unmapped or swapped out (the packer then refuses the batch).
void collect_blocks(const CacheView& view, std::uint32_t context_len, std::vector<std::uint32_t>& ids) {
    const std::uint32_t tpb = view.layout.shape.tokens_per_block;
    const std::uint32_t needed = (context_len + tpb - 1) / tpb;
    for (std::uint32_t j = 0; j < needed; ++j) {
        const BlockTableEntry* e = view.block_table->entry(j);
        ids.push_back((e == nullptr || e->swap_slot.has_value()) ? QVP_UNMAPPED_BLOCK : e->physical_id);
    }
}

// Device staging for the single-sequence entry point, one per thread.
struct SingleScratch {
    PagedAttentionBatch batch;
    void* dq{nullptr};
    void* dout{nullptr};
    std::size_t dq_bytes{0};
    std::size_t dout_bytes{0};

    ~SingleScratch() {
        (void)qvp_free(dq);
        (void)qvp_free(dout);
    }

    bool ensure(std::size_t q_bytes, std::size_t o_bytes) {
        if (dq_bytes < q_bytes) {
            (void)qvp_free(dq);
            dq = nullptr;
            dq_bytes = 0;
            if (qvp_malloc(&dq, q_bytes) != QVP_OK) return false;
            dq_bytes = q_bytes;
        }
        if (dout_bytes < o_bytes) {
            (void)qvp_free(dout);
            dout = nullptr;
            dout_bytes = 0;
            if (qvp_malloc(&dout, o_bytes) != QVP_OK) return false;
            dout_bytes = o_bytes;
        }
        return true;
    }
};

template <typename T>
constexpr ElementType element_type_of() {
    return std::is_same<T, float>::value ? ElementType::F32 : ElementType::BF16;
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
    if (view.allocator->placement() != BlockPlacement::Device) {
        return refuse("the view's frames are host memory; the decode runs on the GPU only");
    }
    thread_local SingleScratch scratch;
    const std::size_t bytes = static_cast<std::size_t>(params.num_query_heads) * shape.head_dim * sizeof(T);
    if (!scratch.ensure(bytes, bytes)) return refuse(std::string("device staging: ") + qvp_last_error());
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

bool PagedAttentionBatch::decode(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                                 std::uint32_t layer, std::uint32_t num_query_heads, float scale,
                                 const void* device_query, void* device_out, ElementType out_type) {
    int cache_type = 0;
    void* stream = nullptr;
    if (!pack(views, context_lens, layer, num_query_heads, device_query, device_out, cache_type, stream)) return false;
    const KVBlockLayout& layout = views.front().layout;
    const BlockShape& shape = layout.shape;
    const MemoryAllocator* allocator = views.front().allocator;
    qvp_decode_args args{};
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
    if (!upload(context_lens, shape.tokens_per_block, &args, stream)) return false;
    if (qvp_paged_decode(&args, stream) != QVP_OK) return fail(std::string("decode: ") + qvp_last_error());
    return true;
}

bool PagedAttentionBatch::prefill(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                                  const std::vector<std::uint32_t>& first_new, std::uint32_t layer,
                                  std::uint32_t num_query_heads, float scale, const void* device_query,
                                  void* device_out, ElementType out_type) {
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

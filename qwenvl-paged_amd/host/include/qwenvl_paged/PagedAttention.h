#pragma once
// Paged-attention decode on the GPU behind the reference's interface
// (include/qwenvl_paged/PagedAttention.h:23-127).
//
// paged_attention_decode<T> keeps the reference signature and refusal rules:
// it returns false, leaving `out` untouched, for an invalid view, a null
// pointer, sizeof(T) != bytes_per_element, context_len == 0, a layer outside
// the shape, query heads that do not group onto the kv heads, or a needed block
// that is unmapped or swapped out (PagedAttention.h:50-89). Otherwise the
// computation runs on the GPU (libqvp: pack, then the decode) and the result
// is copied back. A view over host-placed frames (the reference's own
// allocator) is decoded the same way: the layer's K/V slice of each block the
// context needs is staged through pinned memory into device frames first.
// There is no CPU path. PagedAttentionBatch decodes many sequences in one
// launch from device buffers; that is the engine's per-step entry point.

#include "qwenvl_paged/CacheLayout.h"
#include "qwenvl_paged/KVCacheManager.h"

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

struct qvp_batch;
struct qvp_decode_args;

namespace qwenvl_paged {

struct PagedAttentionParams {
    std::uint32_t layer{0};
    std::uint32_t num_query_heads{0};
    std::uint32_t context_len{0};
    float scale{1.0F};
};

// bfloat16 cache element: two bytes, explicit conversions (float -> bf16
// rounds to nearest, ties to even; NaN stays NaN).
struct bf16 {
    std::uint16_t bits{0};
    bf16() = default;
    explicit bf16(float f) noexcept;
    explicit operator float() const noexcept;
};
static_assert(sizeof(bf16) == 2, "bf16 must be two bytes");

// IEEE binary16 cache element: two bytes, explicit conversions (float -> f16
// rounds to nearest, ties to even, overflowing to infinity, with subnormal
// results; NaN stays NaN).
struct f16 {
    std::uint16_t bits{0};
    f16() = default;
    explicit f16(float f) noexcept;
    explicit operator float() const noexcept;
};
static_assert(sizeof(f16) == 2, "f16 must be two bytes");

// Element type codes (values of qvp_dtype).
enum class ElementType : int { F32 = 0, BF16 = 1, F16 = 2 };

// Decodes one query token (query, out: host arrays of num_query_heads *
// head_dim elements, head-major). T is float, bf16 or f16; a two-byte T also
// names how the cache's elements are read.
template <typename T>
[[nodiscard]] bool paged_attention_decode(const CacheView& view, const T* query, const PagedAttentionParams& params,
                                          T* out);

// The calling thread's message for the last refusal of paged_attention_decode.
[[nodiscard]] const std::string& paged_attention_last_error();

class PagedAttentionBatch {
public:
    PagedAttentionBatch();
    ~PagedAttentionBatch();
    PagedAttentionBatch(const PagedAttentionBatch&) = delete;
    PagedAttentionBatch& operator=(const PagedAttentionBatch&) = delete;

    // Packs the sequences of `views` (context_lens[b] committed tokens each,
    // all views over the same device allocator), validates every argument and
    // block, and enqueues the decode on the allocator's engine stream.
    // device_query / device_out: [B][num_query_heads][head_dim], the cache
    // element type for the query; out_type selects the output element type.
    // Refused calls return false with nothing enqueued.
    bool decode(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                std::uint32_t layer, std::uint32_t num_query_heads, float scale, const void* device_query,
                void* device_out, ElementType out_type);
    // Pipelined steps (two objects used in turn): pack_ahead() does all of
    // decode()'s host work for the next step -- checks, the page-table walk,
    // the pack and the decode's work schedule -- but leaves the step's upload
    // waiting in pinned staging, to be carried by the next decode that
    // another PagedAttentionBatch (or qvp_paged_decode on another batch)
    // enqueues on the allocator's stream, in the tail of that launch;
    // decode_packed() then enqueues this object's decode (and the upload
    // itself if no launch carried it). The engine loop:
    //     b.pack_ahead(step n + 1); a.decode_packed();  // step n carries n + 1's upload
    //     a.pack_ahead(step n + 2); b.decode_packed();  // ...
    // The views are read at pack_ahead(); the cache must not move or rewrite
    // the frames they name before decode_packed() has been enqueued, and a
    // frame the previous step's decode reads must not be released or swapped
    // out by the next step's bookkeeping before that decode is enqueued.
    // Refused calls return false with nothing enqueued (decode_packed()
    // refuses when nothing is packed).
    bool pack_ahead(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                    std::uint32_t layer, std::uint32_t num_query_heads, float scale, const void* device_query,
                    void* device_out, ElementType out_type);
    bool decode_packed();
    // Causal prefill: for every sequence b the new positions p in
    // [first_new[b], context_lens[b]) each attend to tokens [0, p] -- the
    // reference's decode applied per position with context_len = p + 1
    // (PagedAttention.h:43-44), in one enqueued call. The K/V of the new
    // positions must already be in the cache (KVAppendBatch). device_query /
    // device_out: [sum_b (context_lens[b] - first_new[b])][num_query_heads]
    // [head_dim], sequence-major then position order. Refused like decode,
    // and for first_new[b] >= context_lens[b].
    bool prefill(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                 const std::vector<std::uint32_t>& first_new, std::uint32_t layer, std::uint32_t num_query_heads,
                 float scale, const void* device_query, void* device_out, ElementType out_type);
    // Element type of the cache from its element size (4: F32, 2: BF16 unless
    // set_cache_element_type(F16) was called).
    void set_cache_element_type(ElementType type) noexcept;
    [[nodiscard]] const std::string& last_error() const noexcept;
    // The packed batch of the last successful decode or prefill (device arrays).
    [[nodiscard]] qvp_batch* packed() const noexcept;
    // Split-K partition in tokens (0: library default).
    void set_split_tokens(std::uint32_t tokens) noexcept;

private:
    bool fail(std::string msg);
    // Checks shared by decode and prefill and the batch's block ids in CSR
    // form (flushing queued copies first); fills the launch's element type
    // and the allocator's stream.
    bool pack(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
              std::uint32_t layer, std::uint32_t num_query_heads, const void* device_query, void* device_out,
              int& cache_type, void*& stream);
    // Packs the collected batch on `stream`, with the schedule of `decode`
    // when given (qvp_pack_for_decode).
    bool upload(const std::vector<std::uint32_t>& context_lens, std::uint32_t tokens_per_block,
                const qvp_decode_args* decode, void* stream);
    // Checks, walk and the decode's arguments (into args_) shared by decode()
    // and pack_ahead().
    bool prepare(const std::vector<CacheView>& views, const std::vector<std::uint32_t>& context_lens,
                 std::uint32_t layer, std::uint32_t num_query_heads, float scale, const void* device_query,
                 void* device_out, ElementType out_type, void*& stream);

    qvp_batch* batch_{nullptr};
    std::uint32_t num_pool_blocks_{0};
    std::vector<std::uint32_t> ids_;
    std::vector<std::uint32_t> cu_;
    std::string last_error_;
    std::uint32_t split_tokens_{0};
    int cache_type_override_{-1};
    // The decode's arguments of the last decode() / pack_ahead(), and the
    // stream of the last pack_ahead().
    std::unique_ptr<qvp_decode_args> args_;
    void* packed_stream_{nullptr};
    bool packed_ready_{false};
};

}  // namespace qwenvl_paged

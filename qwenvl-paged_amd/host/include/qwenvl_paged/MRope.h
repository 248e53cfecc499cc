#pragma once
// M-RoPE position ids of a step's tokens, from the sequences' positional
// metadata (PositionalEncodingSpan, include/qwenvl_paged/KVCacheManager.h:
// 23-78), written on the GPU.
//
// The reference stores the spans with each sequence and leaves their use to
// model code ("model-specific code reconstruct[s] the correct positional IDs",
// KVCacheManager.h:49-53). MRopePositionBatch implements Qwen2-VL's rule
// (get_rope_index in Hugging Face transformers; Qwen2.5-VL differs only in the
// temporal stride of videos, which the span's stride carries): token i of a
// span sits at origin + stride * (its grid coordinates) per axis -- i itself
// on every axis for Text1D, (i / (H W), (i / W) % H, i % W) for an image or
// video span of grid (T, H, W) -- and a token outside every span continues at
// 1 + the largest position of the tokens before it, which numbers decode
// tokens as p + rope_delta. For a prompt laid out as get_rope_index lays it
// out (a Text1D span per text run at the running position, a vision span per
// image / video with that origin) the positions equal transformers' own.

#include "qwenvl_paged/KVCacheManager.h"

#include <cstdint>
#include <string>
#include <vector>

struct qvp_mrope;
struct qvp_mrope_span;

namespace qwenvl_paged {

class MRopePositionBatch {
public:
    MRopePositionBatch();
    ~MRopePositionBatch();
    MRopePositionBatch(const MRopePositionBatch&) = delete;
    MRopePositionBatch& operator=(const MRopePositionBatch&) = delete;

    // Enqueues on `stream` the positions of tokens [begin[i], end[i]) of
    // sequences[i] (their metadata as given to create_sequence /
    // fork_sequence) into device_out: int64 [3][rows], rows = sum of
    // end[i] - begin[i] in list order, axis-major (temporal, height, width) as
    // a model's position_ids. Refused (false, nothing enqueued) for unequal
    // list sizes, an unknown sequence, begin > end, or spans that are
    // unsorted, overlapping, empty, of an image / video kind without a grid
    // whose product is the token count, or with |origin| or |stride| above
    // 2^24.
    bool materialise(const KVCacheManager& cache, const std::vector<SequenceId>& sequences,
                     const std::vector<TokenPosition>& begin, const std::vector<TokenPosition>& end,
                     std::int64_t* device_out, void* stream);

    [[nodiscard]] const std::string& last_error() const noexcept;

private:
    bool fail(std::string msg);

    qvp_mrope* handle_{nullptr};
    std::vector<qvp_mrope_span> spans_;
    std::vector<std::uint32_t> cu_;
    std::string last_error_;
};

}  // namespace qwenvl_paged

// M-RoPE position ids from PositionalEncodingSpan metadata (the reference's
// include/qwenvl_paged/KVCacheManager.h:23-78), one qvp_mrope_positions call
// per step.
#include "qwenvl_paged/MRope.h"

#include "qvp.h"

#include <utility>

namespace qwenvl_paged {

MRopePositionBatch::MRopePositionBatch() { (void)qvp_mrope_create(&handle_); }

MRopePositionBatch::~MRopePositionBatch() { (void)qvp_mrope_destroy(handle_); }

bool MRopePositionBatch::fail(std::string msg) {
    last_error_ = std::move(msg);
    return false;
}

const std::string& MRopePositionBatch::last_error() const noexcept { return last_error_; }

bool MRopePositionBatch::materialise(const KVCacheManager& cache, const std::vector<SequenceId>& sequences,
                                     const std::vector<TokenPosition>& begin, const std::vector<TokenPosition>& end,
                                     std::int64_t* device_out, void* stream) {
    if (handle_ == nullptr) return fail("no position object");
    if (sequences.size() != begin.size() || sequences.size() != end.size()) {
        return fail("sequences, begin and end differ in size");
    }
    spans_.clear();
    cu_.assign(1, 0);
    std::uint64_t rows = 0;
    for (std::size_t i = 0; i < sequences.size(); ++i) {
        const SequenceMetadata* m = cache.metadata(sequences[i]);
        if (m == nullptr) return fail("unknown sequence " + std::to_string(sequences[i]));
        if (begin[i] > end[i]) return fail("begin > end for sequence " + std::to_string(sequences[i]));
        for (const PositionalEncodingSpan& s : m->positional_encoding.spans) {
            qvp_mrope_span d{};
            d.start_token = s.start_token;
            d.token_count = s.token_count;
            d.kind = static_cast<std::uint32_t>(s.kind);
            const Position3D* src[3] = {&s.origin, &s.stride, &s.grid};
            std::int64_t* dst[3] = {d.origin, d.stride, d.grid};
            for (int f = 0; f < 3; ++f) {
                dst[f][0] = src[f]->temporal;
                dst[f][1] = src[f]->height;
                dst[f][2] = src[f]->width;
            }
            spans_.push_back(d);
        }
        cu_.push_back(static_cast<std::uint32_t>(spans_.size()));
        rows += end[i] - begin[i];
    }
    if (qvp_mrope_positions(handle_, spans_.empty() ? nullptr : spans_.data(), cu_.data(), begin.data(), end.data(),
                            static_cast<std::uint32_t>(sequences.size()), device_out, rows, stream) != QVP_OK) {
        return fail(std::string("positions: ") + qvp_last_error());
    }
    return true;
}

}  // namespace qwenvl_paged

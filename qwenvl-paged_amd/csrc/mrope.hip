// M-RoPE positions: the (temporal, height, width) position id of every token
// of a packed batch, from the sequences' positional spans.
//
// The reference carries the metadata (PositionalEncodingSpan: start, count,
// kind, origin, stride; include/qwenvl_paged/KVCacheManager.h:23-78) and
// leaves its use to model code. The rule implemented here is Qwen2-VL's
// (get_rope_index / get_vision_position_ids in Hugging Face transformers'
// modeling_qwen2_vl.py; Qwen2.5-VL only changes the temporal stride of
// videos): token i of a span is origin + its grid coordinates times stride,
// and a token outside every span continues one-dimensionally after the
// largest position seen so far, which is also how decode tokens are numbered
// (p + rope_delta). Image and video spans need their grid extents, which the
// reference's span does not carry: qvp_mrope_span adds them.
//
// The host validates the spans and turns each into a 12-word descriptor that
// includes R, the largest position of any token before the span's end (R_k =
// max(R_{k-1} + gap_k, largest position inside span k), gap_k = the uncovered
// tokens between spans k-1 and k). With R, a token after span k and before
// span k+1 sits at R_k + 1 + (p - end_k) without looking at earlier tokens.
// A workgroup takes up to 256 consecutive rows of one sequence; the host gives
// it the window of spans that can matter to those rows (those overlapping its
// token range plus the one before), which the workgroup stages in LDS with one
// coalesced read. Each thread then finds its token's span by a binary search
// in LDS and writes three coalesced int64 stores: two dependent global reads
// per workgroup. Only the windows are uploaded, so a decode step (one row per
// sequence) sends a few spans per sequence, not the whole prompt's.
#include "common.h"

#include <algorithm>
#include <cstring>
#include <vector>

struct qvp_mrope {
    int64_t* staging[2]{nullptr, nullptr};
    size_t staging_cap[2]{0, 0};  // int64 elements
    hipEvent_t staging_done[2]{nullptr, nullptr};
    bool staging_pending[2]{false, false};
    int parity{0};
    int64_t* device{nullptr};
    size_t device_cap{0};
};

namespace {

using qvp::fail;

constexpr int kRowsPerGroup = 256;      // rows (threads) per workgroup
constexpr int kGroupWords = 6;          // first output row, first token, rows, first span, span count, 0
constexpr int kSpanWords = 12;          // start, end, kind, origin[3], stride[3], grid h, grid w, R
constexpr int kMaxWindow = kRowsPerGroup + 1;   // spans one group can need
// |origin| and |stride| bound: every position and running maximum stays far
// inside int64 (|position| < 2^24 + 2^32 * 2^24).
constexpr int64_t kCoordLimit = int64_t{1} << 24;

__global__ void __launch_bounds__(kRowsPerGroup) mrope_rows(const int64_t* __restrict__ groups,
                                                            const int64_t* __restrict__ spans, int64_t total,
                                                            int64_t* __restrict__ out) {
    // Sized per launch to the largest window of the call (a few spans for
    // typical prompts), so LDS does not limit how many groups a CU holds.
    extern __shared__ int64_t win[];
    const int64_t* g = groups + static_cast<int64_t>(kGroupWords) * blockIdx.x;
    const int64_t row0 = g[0];
    const int64_t p0 = g[1];
    const int n = static_cast<int>(g[2]);
    const int ns = static_cast<int>(g[4]);
    const int64_t* src = spans + kSpanWords * g[3];
    for (int w = threadIdx.x; w < ns * kSpanWords; w += kRowsPerGroup) win[w] = src[w];
    __syncthreads();
    const int t = threadIdx.x;
    if (t >= n) return;
    const int64_t p = p0 + t;
    // Number of window spans starting at or before p.
    int a = 0;
    int b = ns;
    while (a < b) {
        const int mid = (a + b) >> 1;
        if (win[kSpanWords * mid] <= p) {
            a = mid + 1;
        } else {
            b = mid;
        }
    }
    int64_t pos[3];
    if (a == 0) {
        pos[0] = pos[1] = pos[2] = p;  // no span starts before p in the sequence
    } else {
        const int64_t* sp = win + kSpanWords * (a - 1);
        if (p < sp[1]) {
            const uint32_t i = static_cast<uint32_t>(p - sp[0]);
            uint32_t c[3] = {i, i, i};
            if (sp[2] != 0) {
                const uint32_t gh = static_cast<uint32_t>(sp[9]);
                const uint32_t gw = static_cast<uint32_t>(sp[10]);
                const uint32_t r = i / gw;
                c[0] = r / gh;
                c[1] = r - c[0] * gh;
                c[2] = i - r * gw;
            }
#pragma unroll
            for (int x = 0; x < 3; ++x) pos[x] = sp[3 + x] + static_cast<int64_t>(c[x]) * sp[6 + x];
        } else {
            pos[0] = pos[1] = pos[2] = sp[11] + 1 + (p - sp[1]);
        }
    }
    const int64_t row = row0 + t;
    out[row] = pos[0];
    out[total + row] = pos[1];
    out[2 * total + row] = pos[2];
}

// Largest position inside a validated span.
int64_t span_max(const qvp_mrope_span& s) {
    int64_t m = INT64_MIN;
    for (int x = 0; x < 3; ++x) {
        const int64_t n = s.kind == 0 ? static_cast<int64_t>(s.token_count) : s.grid[x];
        m = std::max(m, std::max(s.origin[x], s.origin[x] + (n - 1) * s.stride[x]));
    }
    return m;
}

int check_span(const qvp_mrope_span& s, uint32_t seq, uint32_t k) {
    if (s.token_count == 0) return fail(QVP_ERR_INVALID_ARGUMENT, "sequence %u span %u is empty", seq, k);
    if (s.kind > 2) return fail(QVP_ERR_INVALID_ARGUMENT, "sequence %u span %u: unknown kind %u", seq, k, s.kind);
    for (int x = 0; x < 3; ++x) {
        if (s.origin[x] > kCoordLimit || s.origin[x] < -kCoordLimit || s.stride[x] > kCoordLimit ||
            s.stride[x] < -kCoordLimit) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "sequence %u span %u: |origin| or |stride| above 2^24", seq, k);
        }
    }
    if (s.kind == 0) return QVP_OK;
    for (int x = 0; x < 3; ++x) {
        if (s.grid[x] < 1 || s.grid[x] > static_cast<int64_t>(s.token_count)) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "sequence %u span %u: grid extent outside [1, token_count]", seq, k);
        }
    }
    if (s.kind == 1 && s.grid[0] != 1) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "sequence %u span %u: Image2D grid with temporal extent != 1", seq, k);
    }
    if (s.grid[0] * s.grid[1] * s.grid[2] != static_cast<int64_t>(s.token_count)) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "sequence %u span %u: grid product != token_count", seq, k);
    }
    return QVP_OK;
}

int64_t span_end(const qvp_mrope_span& s) { return static_cast<int64_t>(s.start_token) + s.token_count; }

// Window of spans [first, last) of one sequence that matters to tokens
// [q0, q1): the spans overlapping it and the last one ending at or before q0.
void window(const qvp_mrope_span* sp, uint32_t ns, int64_t q0, int64_t q1, uint32_t& first, uint32_t& last) {
    const qvp_mrope_span* ov = std::partition_point(sp, sp + ns, [&](const qvp_mrope_span& s) {
        return span_end(s) <= q0;
    });
    const qvp_mrope_span* stop = std::partition_point(sp, sp + ns, [&](const qvp_mrope_span& s) {
        return static_cast<int64_t>(s.start_token) < q1;
    });
    first = static_cast<uint32_t>(ov - sp);
    if (first > 0) --first;
    last = std::max(first, static_cast<uint32_t>(stop - sp));
}

}  // namespace

extern "C" int qvp_mrope_create(qvp_mrope** out) {
    if (out == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "out is NULL");
    *out = new qvp_mrope();
    return QVP_OK;
}

extern "C" int qvp_mrope_destroy(qvp_mrope* m) {
    if (m == nullptr) return QVP_OK;
    for (int i = 0; i < 2; ++i) {
        if (m->staging_pending[i]) (void)hipEventSynchronize(m->staging_done[i]);
        if (m->staging[i] != nullptr) (void)hipHostFree(m->staging[i]);
        if (m->staging_done[i] != nullptr) (void)hipEventDestroy(m->staging_done[i]);
    }
    if (m->device != nullptr) (void)hipFree(m->device);
    delete m;
    return QVP_OK;
}

extern "C" int qvp_mrope_positions(qvp_mrope* m, const qvp_mrope_span* spans, const uint32_t* cu_spans,
                                   const uint32_t* begin, const uint32_t* end, uint32_t num_seqs, int64_t* out,
                                   uint64_t total_rows, void* stream) {
    qvp::clear_error();
    if (m == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "mrope object is NULL");
    if (num_seqs > 0 && (cu_spans == nullptr || begin == nullptr || end == nullptr)) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "cu_spans, begin or end is NULL");
    }
    if (num_seqs > (1u << 24)) return fail(QVP_ERR_INVALID_ARGUMENT, "more than 2^24 sequences");
    if (num_seqs > 0 && cu_spans[0] != 0) return fail(QVP_ERR_INVALID_ARGUMENT, "cu_spans[0] != 0");
    const uint32_t nspans = num_seqs > 0 ? cu_spans[num_seqs] : 0;
    if (nspans > 0 && spans == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "spans is NULL");

    // Pass 1: validate, count workgroups and uploaded spans.
    uint64_t rows = 0;
    uint64_t groups = 0;
    uint64_t uploaded = 0;
    for (uint32_t b = 0; b < num_seqs; ++b) {
        if (cu_spans[b + 1] < cu_spans[b] || cu_spans[b + 1] > nspans) {
            return fail(QVP_ERR_INVALID_ARGUMENT, "cu_spans is not a non-decreasing CSR offset array");
        }
        if (begin[b] > end[b]) return fail(QVP_ERR_INVALID_ARGUMENT, "begin[%u] > end[%u]", b, b);
        const qvp_mrope_span* sp = spans + cu_spans[b];
        const uint32_t ns = cu_spans[b + 1] - cu_spans[b];
        int64_t prev_end = 0;
        for (uint32_t k = 0; k < ns; ++k) {
            QVP_TRY(check_span(sp[k], b, k));
            if (static_cast<int64_t>(sp[k].start_token) < prev_end) {
                return fail(QVP_ERR_INVALID_ARGUMENT, "sequence %u: spans unsorted or overlapping at span %u", b, k);
            }
            prev_end = span_end(sp[k]);
        }
        const uint64_t r = end[b] - begin[b];
        if (r == 0) continue;
        rows += r;
        groups += (r + kRowsPerGroup - 1) / kRowsPerGroup;
        uint32_t first = 0;
        uint32_t last = 0;
        window(sp, ns, begin[b], end[b], first, last);
        uploaded += last - first;
    }
    if (rows != total_rows) {
        return fail(QVP_ERR_INVALID_ARGUMENT, "total_rows %llu != sum of end - begin (%llu)",
                    static_cast<unsigned long long>(total_rows), static_cast<unsigned long long>(rows));
    }
    if (rows == 0) return QVP_OK;
    if (out == nullptr) return fail(QVP_ERR_INVALID_ARGUMENT, "out is NULL");
    if (groups > 0x7fffffffu) return fail(QVP_ERR_INVALID_ARGUMENT, "too many rows");

    const size_t span_base = groups * kGroupWords;
    const size_t words = span_base + uploaded * kSpanWords;
    hipStream_t s = qvp::as_stream(stream);
    const int slot = m->parity;
    if (m->staging_done[slot] == nullptr) {
        // Host-side reuse of pinned staging only: no system-scope release.
        QVP_HIP(hipEventCreateWithFlags(&m->staging_done[slot], hipEventDisableTiming | hipEventDisableSystemFence));
    }
    // The staging buffer about to be refilled may still be read by the copy of
    // the call before last.
    if (m->staging_pending[slot]) {
        QVP_HIP(hipEventSynchronize(m->staging_done[slot]));
        m->staging_pending[slot] = false;
    }
    if (m->staging_cap[slot] < words) {
        if (m->staging[slot] != nullptr) QVP_HIP(hipHostFree(m->staging[slot]));
        m->staging[slot] = nullptr;
        m->staging_cap[slot] = 0;
        const size_t cap = std::max<size_t>(words, 4096);
        QVP_HIP(hipHostMalloc(reinterpret_cast<void**>(&m->staging[slot]), cap * sizeof(int64_t),
                              hipHostMallocCoherent));
        m->staging_cap[slot] = cap;
    }
    if (m->device_cap < words) {
        // An earlier call on this stream may still read the descriptors.
        if (m->device != nullptr) {
            QVP_HIP(hipStreamSynchronize(s));
            QVP_HIP(hipFree(m->device));
        }
        m->device = nullptr;
        m->device_cap = 0;
        const size_t cap = std::max<size_t>(words, 4096);
        QVP_HIP(hipMalloc(reinterpret_cast<void**>(&m->device), cap * sizeof(int64_t)));
        m->device_cap = cap;
    }

    // Pass 2: workgroup descriptors and span windows, straight into staging.
    int64_t* gd = m->staging[slot];
    int64_t* sd = gd + span_base;
    uint64_t row = 0;
    uint64_t sent = 0;
    uint32_t max_window = 1;
    for (uint32_t b = 0; b < num_seqs; ++b) {
        const uint64_t r = end[b] - begin[b];
        if (r == 0) continue;
        const qvp_mrope_span* sp = spans + cu_spans[b];
        const uint32_t ns = cu_spans[b + 1] - cu_spans[b];
        uint32_t wfirst = 0;
        uint32_t wlast = 0;
        window(sp, ns, begin[b], end[b], wfirst, wlast);
        // R of every span up to the window's end; descriptors of the window.
        int64_t running = -1;
        int64_t prev_end = 0;
        for (uint32_t k = 0; k < wlast; ++k) {
            running = std::max(running + (static_cast<int64_t>(sp[k].start_token) - prev_end), span_max(sp[k]));
            prev_end = span_end(sp[k]);
            if (k < wfirst) continue;
            int64_t* d = sd + (sent + (k - wfirst)) * kSpanWords;
            d[0] = sp[k].start_token;
            d[1] = prev_end;
            d[2] = sp[k].kind;
            for (int x = 0; x < 3; ++x) {
                d[3 + x] = sp[k].origin[x];
                d[6 + x] = sp[k].stride[x];
            }
            d[9] = sp[k].kind == 0 ? 1 : sp[k].grid[1];
            d[10] = sp[k].kind == 0 ? 1 : sp[k].grid[2];
            d[11] = running;
        }
        for (uint64_t q0 = begin[b]; q0 < end[b]; q0 += kRowsPerGroup) {
            const uint64_t q1 = std::min<uint64_t>(q0 + kRowsPerGroup, end[b]);
            uint32_t first = 0;
            uint32_t last = 0;
            window(sp, ns, static_cast<int64_t>(q0), static_cast<int64_t>(q1), first, last);
            gd[0] = static_cast<int64_t>(row);
            gd[1] = static_cast<int64_t>(q0);
            gd[2] = static_cast<int64_t>(q1 - q0);
            gd[3] = static_cast<int64_t>(sent + (first - wfirst));
            gd[4] = static_cast<int64_t>(last - first);
            gd[5] = 0;
            max_window = std::max(max_window, last - first);
            gd += kGroupWords;
            row += q1 - q0;
        }
        sent += wlast - wfirst;
    }

    QVP_TRY(qvp::pull_from_pinned(m->device, m->staging[slot], words * sizeof(int64_t), s));
    QVP_HIP(hipEventRecord(m->staging_done[slot], s));
    m->staging_pending[slot] = true;
    m->parity ^= 1;
    if (max_window > kMaxWindow) return fail(QVP_ERR_INVALID_ARGUMENT, "internal: span window of %u", max_window);
    const size_t lds = static_cast<size_t>(max_window) * kSpanWords * sizeof(int64_t);
    hipLaunchKernelGGL(mrope_rows, dim3(static_cast<unsigned>(groups)), dim3(kRowsPerGroup), lds, s, m->device,
                       m->device + span_base, static_cast<int64_t>(rows), out);
    QVP_HIP(hipGetLastError());
    return QVP_OK;
}

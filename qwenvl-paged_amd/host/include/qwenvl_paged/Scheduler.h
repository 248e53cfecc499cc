#pragma once
// Continuous-batching admission, preemption and resume
// (include/qwenvl_paged/Scheduler.h:18-199). Policy and results match the
// reference: FIFO admission with a head-of-line stop, optional watermark
// preemption of the newest pre-existing active request, preemption by
// sequence swap-out, resume by all-or-nothing swap-in.

#include "qwenvl_paged/KVCacheManager.h"
#include "qwenvl_paged/MemoryAllocator.h"

#include <cstdint>
#include <deque>
#include <optional>
#include <string>
#include <unordered_map>
#include <vector>

namespace qwenvl_paged {

enum class RequestState : std::uint8_t { Pending, Prefill, Decode, Preempted, Finished, Cancelled };

struct SamplingConfig {
    std::uint32_t num_parallel_samples{1};
    std::uint32_t max_decode_tokens{0};
};

struct Request {
    RequestId request_id{0};
    SequenceId root_sequence_id{0};
    std::uint32_t prompt_tokens{0};
    SamplingConfig sampling{};
    std::vector<MultimodalSpan> multimodal_spans;
    PositionalEncodingMetadata positional_encoding;
    RequestState state{RequestState::Pending};
};

struct SchedulerConfig {
    std::uint32_t max_active_requests{0};
    std::uint32_t max_batch_tokens{0};
    // Free blocks to keep after admitting; 0 disables automatic preemption.
    std::uint32_t preemption_watermark_blocks{0};
};

struct PreemptionInfo {
    std::string reason;
    std::uint32_t swapped_blocks{0};
};

struct BatchPlan {
    std::vector<RequestId> prefill_requests;
    std::vector<RequestId> decode_requests;
    std::uint32_t scheduled_tokens{0};
};

class Scheduler {
public:
    Scheduler(SchedulerConfig config, KVCacheManager& cache_manager, MemoryAllocator& allocator);
    Scheduler(const Scheduler&) = delete;
    Scheduler& operator=(const Scheduler&) = delete;

    void enqueue(Request request);
    [[nodiscard]] BatchPlan schedule_next();
    void complete_step(RequestId request_id, std::uint32_t produced_tokens);
    void cancel(RequestId request_id);
    bool preempt(RequestId request_id, std::string reason);
    bool resume(RequestId request_id);
    [[nodiscard]] std::optional<PreemptionInfo> preemption_info(RequestId request_id) const;
    [[nodiscard]] std::optional<RequestState> state(RequestId request_id) const;
    [[nodiscard]] std::size_t active_size() const noexcept;

private:
    // Every known request lives in `requests_`, found by id in O(1); the three
    // order lists hold ids only: FIFO admission order, admission/resume order
    // of the running set, and preemption order.
    struct Tracked {
        Request request;
        std::optional<PreemptionInfo> preemption;
    };

    [[nodiscard]] std::uint32_t frames_for(std::uint32_t tokens) const noexcept;
    void make_room(std::uint32_t prompt_tokens, std::size_t admitted_now);
    void forget(RequestId id);

    SchedulerConfig config_{};
    KVCacheManager* cache_manager_{nullptr};
    MemoryAllocator* allocator_{nullptr};
    std::unordered_map<RequestId, Tracked> requests_;
    std::deque<RequestId> waiting_;
    std::vector<RequestId> running_;
    std::vector<RequestId> parked_;
};

}  // namespace qwenvl_paged

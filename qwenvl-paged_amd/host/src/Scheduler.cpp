// Continuous-batching scheduler. Decisions follow src/Scheduler.cpp of the
// reference (admission :41-73, preempt/resume :100-135, watermark :173-208);
// the bookkeeping is an id-indexed table plus three id order lists.
#include "qwenvl_paged/Scheduler.h"

#include <algorithm>
#include <utility>

namespace qwenvl_paged {

namespace {

void erase_id(std::vector<RequestId>& ids, RequestId id) {
    auto it = std::find(ids.begin(), ids.end(), id);
    if (it != ids.end()) ids.erase(it);
}

void erase_id(std::deque<RequestId>& ids, RequestId id) {
    auto it = std::find(ids.begin(), ids.end(), id);
    if (it != ids.end()) ids.erase(it);
}

}  // namespace

Scheduler::Scheduler(SchedulerConfig config, KVCacheManager& cache_manager, MemoryAllocator& allocator)
    : config_(config), cache_manager_(&cache_manager), allocator_(&allocator) {}

void Scheduler::enqueue(Request request) {
    const RequestId id = request.request_id;
    // Request ids are unique; a second enqueue of a live id is ignored.
    if (requests_.count(id) != 0) return;
    request.state = RequestState::Pending;
    requests_.emplace(id, Tracked{std::move(request), std::nullopt});
    waiting_.push_back(id);
}

BatchPlan Scheduler::schedule_next() {
    BatchPlan plan;
    while (!waiting_.empty() && running_.size() < config_.max_active_requests) {
        Request& next = requests_.at(waiting_.front()).request;
        if (plan.scheduled_tokens + next.prompt_tokens > config_.max_batch_tokens) break;
        make_room(next.prompt_tokens, plan.prefill_requests.size());

        SequenceMetadata meta;
        meta.sequence_id = next.root_sequence_id;
        meta.request_id = next.request_id;
        meta.multimodal_spans = next.multimodal_spans;
        meta.positional_encoding = next.positional_encoding;
        if (!cache_manager_->create_sequence(std::move(meta))) break;
        if (!cache_manager_->reserve_tokens(next.root_sequence_id, next.prompt_tokens)) {
            // Head of line blocks: undo the empty sequence and retry next step.
            cache_manager_->release_sequence(next.root_sequence_id);
            break;
        }
        next.state = RequestState::Prefill;
        plan.prefill_requests.push_back(next.request_id);
        plan.scheduled_tokens += next.prompt_tokens;
        running_.push_back(next.request_id);
        waiting_.pop_front();
    }
    for (const RequestId id : running_) {
        if (requests_.at(id).request.state != RequestState::Decode) continue;
        plan.decode_requests.push_back(id);
        plan.scheduled_tokens += 1;
    }
    return plan;
}

void Scheduler::complete_step(RequestId request_id, std::uint32_t /*produced_tokens*/) {
    auto it = requests_.find(request_id);
    if (it != requests_.end() && it->second.request.state == RequestState::Prefill) {
        it->second.request.state = RequestState::Decode;
    }
}

void Scheduler::forget(RequestId id) {
    erase_id(waiting_, id);
    erase_id(running_, id);
    erase_id(parked_, id);
    requests_.erase(id);
}

void Scheduler::cancel(RequestId request_id) {
    auto it = requests_.find(request_id);
    if (it == requests_.end()) return;
    cache_manager_->release_sequence(it->second.request.root_sequence_id);
    forget(request_id);
}

bool Scheduler::preempt(RequestId request_id, std::string reason) {
    auto it = requests_.find(request_id);
    if (it == requests_.end()) return false;
    Tracked& t = it->second;
    const RequestState s = t.request.state;
    if (s != RequestState::Prefill && s != RequestState::Decode) return false;
    erase_id(running_, request_id);
    t.request.state = RequestState::Preempted;
    PreemptionInfo info;
    info.reason = std::move(reason);
    // Shared frames stay resident (the allocator refuses them); the count is
    // what actually left the pool.
    info.swapped_blocks = cache_manager_->swap_out_sequence(t.request.root_sequence_id);
    t.preemption = std::move(info);
    parked_.push_back(request_id);
    return true;
}

bool Scheduler::resume(RequestId request_id) {
    auto it = requests_.find(request_id);
    if (it == requests_.end() || it->second.request.state != RequestState::Preempted) return false;
    Tracked& t = it->second;
    if (!cache_manager_->swap_in_sequence(t.request.root_sequence_id)) return false;
    erase_id(parked_, request_id);
    t.request.state = RequestState::Decode;
    t.preemption.reset();
    running_.push_back(request_id);
    return true;
}

std::optional<PreemptionInfo> Scheduler::preemption_info(RequestId request_id) const {
    auto it = requests_.find(request_id);
    return it == requests_.end() ? std::nullopt : it->second.preemption;
}

std::optional<RequestState> Scheduler::state(RequestId request_id) const {
    auto it = requests_.find(request_id);
    if (it == requests_.end()) return std::nullopt;
    return it->second.request.state;
}

std::size_t Scheduler::active_size() const noexcept { return running_.size(); }

std::uint32_t Scheduler::frames_for(std::uint32_t tokens) const noexcept {
    const PhysicalBlock* first = allocator_->block(0);
    const std::uint32_t tpb = first == nullptr ? 0 : first->shape().tokens_per_block;
    return tpb == 0 ? 0 : (tokens + tpb - 1) / tpb;
}

void Scheduler::make_room(std::uint32_t prompt_tokens, std::size_t admitted_now) {
    const std::uint32_t reserve = config_.preemption_watermark_blocks;
    if (reserve == 0) return;
    const std::uint32_t pool = allocator_->stats().total_blocks;
    const std::uint32_t prompt_frames = frames_for(prompt_tokens);
    if (prompt_frames == 0 || prompt_frames > pool) return;  // can never be admitted
    // The reserve is capped at the pool, so a prompt of nearly the whole pool
    // is still admissible.
    const std::uint32_t target = std::min(prompt_frames + reserve, pool);
    // Victims: running requests admitted before this step, newest first.
    while (running_.size() > admitted_now) {
        const std::uint32_t free_before = allocator_->stats().free_blocks;
        if (free_before >= target) return;
        const RequestId victim = running_[running_.size() - admitted_now - 1];
        if (!preempt(victim, "cache pressure watermark")) return;
        // With nothing to swap into, preemption frees no frames; stop after
        // the first one that shows it.
        if (allocator_->stats().free_blocks <= free_before) return;
    }
}

}  // namespace qwenvl_paged

// scheduler.cpp -- admission and micro-batch decisions.
//
// Same decisions, order of checks and reason strings as
// src/runtime/scheduler.cpp:8-139 (capacity, transition, order, schedule,
// homogeneous profile) and src/runtime/scheduler.hpp:88-157 (regime key and
// admission classification); group_decode_launches restates the decode
// grouping of src/runtime/serving.cpp:1899-1936 for one shared plan.
#include "air/scheduler.hpp"

#include <algorithm>
#include <limits>

namespace air::runtime_detail {

CapacityDecision CapacityScheduler::evaluate(std::size_t active_requests, std::uint64_t active_reserved_bytes,
                                             const PreparedModel& backend, const ExecutionPlan& plan,
                                             std::uint64_t requested_tokens,
                                             std::uint64_t plan_preparation_bytes) const {
    if (active_requests >= max_active_requests_) return {false, 0U, "max-active-requests"};
    const auto reservation = backend.estimate_sequence_device_bytes(plan, requested_tokens);
    // A plan artifact needs memory that is free now; reusable KV pages do not count.
    if (plan_preparation_bytes != 0U) {
        const auto free = backend.free_device_bytes();
        if (free && plan_preparation_bytes > *free) return {false, reservation, "device-capacity-plan-artifact"};
    }
    if (const auto capacity = backend.sequence_capacity_bytes()) {
        if (plan_preparation_bytes > *capacity) return {false, reservation, "device-capacity-plan-artifact"};
        const auto usable = *capacity - plan_preparation_bytes;
        if (reservation > usable || active_reserved_bytes > usable - reservation) {
            return {false, reservation, "device-capacity"};
        }
    }
    return {true, reservation, "admitted"};
}

TransitionCapacityDecision CapacityScheduler::evaluate_transition(const PreparedModel& backend,
                                                                  const ExecutionPlan& target_plan,
                                                                  std::uint64_t temporary_device_bytes) const {
    const auto preparation = backend.estimate_plan_preparation_device_bytes(target_plan);
    if (preparation > std::numeric_limits<std::uint64_t>::max() - temporary_device_bytes) {
        return {false, preparation, temporary_device_bytes, "device-capacity-transition-overflow"};
    }
    const auto required = preparation + temporary_device_bytes;
    if (const auto free = backend.free_device_bytes(); free && required > *free) {
        return {false, preparation, temporary_device_bytes,
                preparation != 0U ? "device-capacity-transition-plan-artifact"
                                  : "device-capacity-transition-temporary"};
    }
    return {true, preparation, temporary_device_bytes, "admitted"};
}

std::vector<SchedulableSequence> MicrobatchScheduler::order(std::span<const SchedulableSequence> candidates) {
    std::vector<SchedulableSequence> decode;
    std::vector<SchedulableSequence> prefill;
    for (const auto& c : candidates) (c.phase == WorkPhase::decode ? decode : prefill).push_back(c);
    const auto rotate = [](std::vector<SchedulableSequence>& phase, std::size_t& cursor) {
        if (phase.empty()) {
            cursor = 0U;
            return;
        }
        cursor %= phase.size();
        std::rotate(phase.begin(), phase.begin() + static_cast<std::ptrdiff_t>(cursor), phase.end());
        cursor = (cursor + 1U) % phase.size();
    };
    rotate(decode, decode_cursor_);
    rotate(prefill, prefill_cursor_);
    decode.insert(decode.end(), prefill.begin(), prefill.end());
    return decode;
}

ScheduledBatch MicrobatchScheduler::schedule(std::span<const SchedulableSequence> candidates,
                                             std::uint32_t token_budget) {
    ScheduledBatch batch;
    if (token_budget == 0U || candidates.empty()) return batch;
    const auto ordered = order(candidates);
    auto remaining = token_budget;
    for (const auto& c : ordered) {
        if (remaining == 0U) break;
        if (c.max_tokens == 0U) continue;
        const auto tokens = c.phase == WorkPhase::decode ? 1U : std::min(c.max_tokens, remaining);
        if (tokens == 0U || tokens > remaining) continue;
        batch.slices.push_back({c.slot, c.phase, tokens});
        batch.token_count += tokens;
        remaining -= tokens;
        if (c.phase == WorkPhase::decode) {
            ++batch.decode_tokens;
        } else {
            batch.prefill_tokens += tokens;
            ++batch.prefill_sequences;
        }
    }
    return batch;
}

ExecutionRegimeKey execution_regime_key(const ExecutionPlan& plan) noexcept {
    return {plan.backend,           plan.linear.prefill_block, plan.linear.decode_block,
            plan.linear.decode_output, plan.attention.prefill, plan.attention.decode,
            plan.kv.page_tokens,    plan.scheduling.prefill_quantum_tokens};
}

RegimeAdmissionAction classify_regime_admission(const std::optional<ExecutionRegimeKey>& active,
                                                const ExecutionRegimeKey& requested, bool fallback_pinned) noexcept {
    if (fallback_pinned) return RegimeAdmissionAction::use_pinned_fallback;
    if (active && *active == requested) return RegimeAdmissionAction::compatible;
    return RegimeAdmissionAction::converge_to_fallback;
}

bool same_regime_request_shape(const RegimeRequestShape& a, const RegimeRequestShape& b) noexcept {
    return a.prompt_tokens == b.prompt_tokens && a.max_output_tokens == b.max_output_tokens;
}

bool homogeneous_regime_shape_accepts(std::span<const RegimeRequestShape> active,
                                      const RegimeRequestShape& incoming) noexcept {
    if (active.empty()) return false;
    return std::all_of(active.begin(), active.end(),
                       [&](const RegimeRequestShape& s) { return same_regime_request_shape(s, incoming); });
}

std::optional<RequestProfile> homogeneous_regime_profile(std::span<const RegimeRequestShape> requests) noexcept {
    if (requests.empty() || requests.size() > std::numeric_limits<std::uint32_t>::max()) return std::nullopt;
    const auto first = requests.front();
    for (const auto& r : requests.subspan(1U)) {
        if (!same_regime_request_shape(r, first)) return std::nullopt;
    }
    return RequestProfile{first.prompt_tokens, first.max_output_tokens, static_cast<std::uint32_t>(requests.size())};
}

std::vector<std::vector<std::size_t>> group_decode_launches(std::span<const ScheduledSlice> slices,
                                                            const ExecutionPlan& plan, std::uint32_t max_width) {
    const bool batching = max_width > 1U && (plan.linear.decode_block != QuantizedLinearExecutionKind::baseline ||
                                             plan.linear.decode_output != QuantizedLinearExecutionKind::baseline);
    std::vector<std::vector<std::size_t>> launches;
    std::size_t i = 0;
    while (i < slices.size()) {
        if (batching && slices[i].phase == WorkPhase::decode) {
            std::vector<std::size_t> rows;
            for (std::size_t j = i; j < slices.size() && rows.size() < max_width; ++j) {
                if (slices[j].phase != WorkPhase::decode) break;
                rows.push_back(j);
            }
            if (rows.size() >= 2U) {
                i += rows.size();
                launches.push_back(std::move(rows));
                continue;
            }
        }
        launches.push_back({i});
        ++i;
    }
    return launches;
}

} // namespace air::runtime_detail

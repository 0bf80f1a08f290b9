// scheduler.hpp -- admission and micro-batch scheduling.
//
// Restates AIR's runtime scheduler (src/runtime/scheduler.hpp:13-198,
// src/runtime/scheduler.cpp:8-139) with the same decisions and reason strings:
//   CapacityScheduler   admit <=> active < max, plan artifact <= free device
//                        bytes, reserved + need <= capacity - artifact
//   MicrobatchScheduler decode-first, phase-local round robin, one token per
//                        decode slice, prefill slices bounded by the budget
// On MI355X the capacity is the pool's reusable pages plus hipMemGetInfo's
// free bytes of the 288 GB HBM; the decisions are pure u64 arithmetic.
#pragma once

#include "air/backend.hpp"
#include "air/execution.hpp"

#include <cstddef>
#include <cstdint>
#include <optional>
#include <span>
#include <string>
#include <vector>

namespace air::runtime_detail {

struct CapacityDecision {
    bool admit{false};
    std::uint64_t reservation_bytes{0};
    std::string reason;
};

struct TransitionCapacityDecision {
    bool admit{false};
    std::uint64_t plan_preparation_bytes{0};
    std::uint64_t temporary_device_bytes{0};
    std::string reason;
};

class CapacityScheduler final {
public:
    explicit CapacityScheduler(std::uint32_t max_active_requests) : max_active_requests_(max_active_requests) {}

    [[nodiscard]] CapacityDecision evaluate(std::size_t active_requests, std::uint64_t active_reserved_bytes,
                                            const PreparedModel& backend, const ExecutionPlan& plan,
                                            std::uint64_t requested_tokens,
                                            std::uint64_t plan_preparation_bytes = 0U) const;

    // Admission of an in-place regime change: new plan artifacts plus the
    // temporary bytes of migrating live sequences must fit free memory.
    [[nodiscard]] TransitionCapacityDecision evaluate_transition(const PreparedModel& backend,
                                                                 const ExecutionPlan& target_plan,
                                                                 std::uint64_t temporary_device_bytes) const;

private:
    std::uint32_t max_active_requests_{1};
};

enum class WorkPhase {
    prefill = 0,
    decode,
};

struct SchedulableSequence {
    std::size_t slot{0};
    WorkPhase phase{WorkPhase::prefill};
    // Tokens this sequence may consume this cycle (decode: 1; 0: not runnable).
    std::uint32_t max_tokens{1};
};

struct ScheduledSlice {
    std::size_t slot{0};
    WorkPhase phase{WorkPhase::prefill};
    std::uint32_t token_count{0};
};

struct ScheduledBatch {
    std::vector<ScheduledSlice> slices;
    std::uint32_t token_count{0};
    std::uint32_t decode_tokens{0};
    std::uint32_t prefill_tokens{0};
    std::uint32_t prefill_sequences{0};
};

// Physical identity of an execution regime: the strategy label is left out,
// so plans that lower to the same device work batch together.
struct ExecutionRegimeKey {
    BackendKind backend{BackendKind::reference};
    QuantizedLinearExecutionKind prefill_block{QuantizedLinearExecutionKind::baseline};
    QuantizedLinearExecutionKind decode_block{QuantizedLinearExecutionKind::baseline};
    QuantizedLinearExecutionKind decode_output{QuantizedLinearExecutionKind::baseline};
    AttentionExecutionKind prefill_attention{AttentionExecutionKind::baseline};
    AttentionExecutionKind decode_attention{AttentionExecutionKind::baseline};
    std::optional<std::uint32_t> kv_page_tokens;
    std::uint32_t prefill_quantum_tokens{0};

    [[nodiscard]] friend bool operator==(const ExecutionRegimeKey&, const ExecutionRegimeKey&) = default;
};

[[nodiscard]] ExecutionRegimeKey execution_regime_key(const ExecutionPlan& plan) noexcept;

enum class RegimeAdmissionAction {
    compatible = 0,
    converge_to_fallback,
    use_pinned_fallback,
};

[[nodiscard]] RegimeAdmissionAction classify_regime_admission(const std::optional<ExecutionRegimeKey>& active,
                                                              const ExecutionRegimeKey& requested,
                                                              bool fallback_pinned) noexcept;

struct RegimeRequestShape {
    std::uint64_t prompt_tokens{0};
    std::uint64_t max_output_tokens{0};
};

[[nodiscard]] bool same_regime_request_shape(const RegimeRequestShape& a, const RegimeRequestShape& b) noexcept;
[[nodiscard]] bool homogeneous_regime_shape_accepts(std::span<const RegimeRequestShape> active,
                                                    const RegimeRequestShape& incoming) noexcept;
// Exact group profile only when every request has the same shape.
[[nodiscard]] std::optional<RequestProfile> homogeneous_regime_profile(
    std::span<const RegimeRequestShape> requests) noexcept;

class MicrobatchScheduler final {
public:
    // Decode candidates first, then prefill; each phase rotated by its own
    // cursor so a one-slot budget serves the slots in turn.
    [[nodiscard]] std::vector<SchedulableSequence> order(std::span<const SchedulableSequence> candidates);
    // Token slices of one worker cycle under token_budget.
    [[nodiscard]] ScheduledBatch schedule(std::span<const SchedulableSequence> candidates,
                                          std::uint32_t token_budget);

private:
    std::size_t decode_cursor_{0};
    std::size_t prefill_cursor_{0};
};

// Splits a scheduled batch into launches the way the serving loop does for
// greedy rows that share one plan (serving.cpp:1899-1936): runs of
// consecutive decode slices become one launch of at most max_width rows when
// the plan's decode tactics are not both baseline and the width exceeds 1; a
// run of one, and every prefill slice, stays a launch of its own.  Each
// launch lists indices into `slices`.
[[nodiscard]] std::vector<std::vector<std::size_t>> group_decode_launches(std::span<const ScheduledSlice> slices,
                                                                          const ExecutionPlan& plan,
                                                                          std::uint32_t max_width);

} // namespace air::runtime_detail

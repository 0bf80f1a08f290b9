// token_service.hpp -- the caller slice of InferenceService for token ids.
//
// TokenService drives a prepared model the way InferenceService's worker
// does (src/runtime/serving.cpp:1494-1990, generate_cohort at :2401-2481):
// a cohort of requests is validated before any member is queued, admitted
// through CapacityScheduler against the backend's device capacity, and run in
// worker cycles that MicrobatchScheduler fills decode-first under a token
// budget.  Consecutive prefill slices become one PreparedModel::prefill_batch
// call (prefill width 512 on the HIP backend); consecutive decode slices
// become decode_greedy_batch launches of up to the advertised decode width
// (64), grouped as group_decode_launches does.  Generation follows
// run_autoregressive (src/runtime/generation.cpp:26-85): the prompt's greedy
// token is the first output, each further token costs one decode step, and a
// request stops at max_new_tokens or at its stop token.
//
// The reference's service accepts only text (serving.hpp:69-73); requests
// here carry token ids, so no tokenizer runs.  Sampling is greedy only (the
// batched device paths of the reference are greedy-only as well,
// serving.cpp:1899-1905).  Planning modes, manifests, streaming callbacks,
// cancellation and decisions are not part of this slice.
#pragma once

#include "air/backend.hpp"
#include "air/scheduler.hpp"

#include <cstdint>
#include <memory>
#include <optional>
#include <span>
#include <vector>

namespace air {

struct TokenRequest {
    std::vector<TokenId> prompt;
    std::uint32_t max_new_tokens{16};
    std::optional<TokenId> stop_token;  // GenerationConfig::stop_on_eos with the model's eos id
};

// The timing and size fields of RequestMetrics (serving.hpp:77-105).
struct TokenMetrics {
    std::uint64_t request_id{0};
    std::uint64_t prompt_tokens{0};
    std::uint64_t generated_tokens{0};
    std::uint64_t kv_bytes{0};
    double queue_ms{0.0};
    double prefill_ms{0.0};
    double ttft_ms{0.0};
    double decode_ms{0.0};
    double total_ms{0.0};

    [[nodiscard]] double prefill_tokens_per_second() const noexcept;
    [[nodiscard]] double decode_tokens_per_second() const noexcept;
};

struct TokenResponse {
    std::vector<TokenId> tokens;
    bool hit_stop{false};
    TokenMetrics metrics;
};

struct TokenServiceConfig {
    ExecutionPlan plan{};                       // backend, tactics, KV page size, prefill quantum
    std::uint32_t max_active_requests{64};
    std::uint32_t max_queued_requests{256};
    std::uint32_t token_budget_per_cycle{512};
};

// Physical work of the service since creation.
struct TokenServiceStats {
    std::uint64_t cycles{0};
    std::uint64_t prefill_calls{0};
    std::uint64_t prefill_tokens{0};
    std::uint64_t decode_calls{0};
    std::uint64_t decode_rows{0};
    std::uint32_t max_decode_width{0};
    std::uint32_t max_prefill_sequences{0};
    double prefill_ms{0.0};   // wall time inside prefill_batch
    double decode_ms{0.0};    // wall time inside decode_greedy_batch
};

class TokenService {
public:
    [[nodiscard]] static Result<std::unique_ptr<TokenService>> create(
        std::shared_ptr<runtime_detail::PreparedModel> prepared, const TokenServiceConfig& config);

    // Runs every request to completion; responses in request order.  A
    // request the device cannot hold even alone fails the cohort before any
    // work starts; others wait for capacity.
    [[nodiscard]] Result<std::vector<TokenResponse>> generate_cohort(std::span<const TokenRequest> requests);

    [[nodiscard]] const TokenServiceStats& stats() const noexcept { return stats_; }
    [[nodiscard]] const TokenServiceConfig& config() const noexcept { return config_; }
    [[nodiscard]] runtime_detail::PreparedModel& prepared() noexcept { return *prepared_; }

private:
    TokenService(std::shared_ptr<runtime_detail::PreparedModel> prepared, const TokenServiceConfig& config)
        : prepared_(std::move(prepared)), config_(config), capacity_(config.max_active_requests) {}

    std::shared_ptr<runtime_detail::PreparedModel> prepared_;
    TokenServiceConfig config_;
    runtime_detail::CapacityScheduler capacity_;
    runtime_detail::MicrobatchScheduler microbatch_;
    TokenServiceStats stats_{};
    std::uint64_t next_request_{1};
};

} // namespace air

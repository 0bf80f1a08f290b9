// token_service.cpp -- TokenService: cohort admission and worker cycles.
#include "air/token_service.hpp"

#include <algorithm>
#include <chrono>
#include <deque>

namespace air {

namespace {

using Clock = std::chrono::steady_clock;

double milliseconds(Clock::duration d) { return std::chrono::duration<double, std::milli>(d).count(); }

struct Work {
    std::size_t index{0};  // request index
    const TokenRequest* request{nullptr};
    std::unique_ptr<runtime_detail::SequenceState> sequence;
    std::uint64_t reserved_bytes{0};
    std::size_t prompt_position{0};
    std::vector<TokenId> tokens;
    bool done{false};
    bool hit_stop{false};
    Clock::time_point submitted, admitted, first_token, finished;
    std::uint64_t kv_bytes{0};

    [[nodiscard]] bool prefilling() const noexcept { return prompt_position < request->prompt.size(); }
    // Records a generated token; true when the request is complete.
    bool accept(TokenId token, Clock::time_point now) {
        if (tokens.empty()) first_token = now;
        tokens.push_back(token);
        if (request->stop_token && token == *request->stop_token) hit_stop = true;
        done = hit_stop || tokens.size() >= request->max_new_tokens;
        return done;
    }
};

} // namespace

double TokenMetrics::prefill_tokens_per_second() const noexcept {
    return prefill_ms > 0.0 ? static_cast<double>(prompt_tokens) * 1000.0 / prefill_ms : 0.0;
}

double TokenMetrics::decode_tokens_per_second() const noexcept {
    if (generated_tokens <= 1U || decode_ms <= 0.0) return 0.0;
    return static_cast<double>(generated_tokens - 1U) * 1000.0 / decode_ms;
}

Result<std::unique_ptr<TokenService>> TokenService::create(std::shared_ptr<runtime_detail::PreparedModel> prepared,
                                                           const TokenServiceConfig& config) {
    if (!prepared) return Status::invalid_argument("token service requires a prepared model");
    if (config.max_active_requests == 0U) return Status::invalid_argument("max_active_requests must be non-zero");
    if (config.token_budget_per_cycle == 0U) return Status::invalid_argument("token budget must be non-zero");
    if (config.plan.scheduling.prefill_quantum_tokens == 0U) {
        return Status::invalid_argument("prefill quantum must be non-zero");
    }
    if (Status s = validate_execution_plan(config.plan, prepared->capabilities()); !s) return s;
    return std::unique_ptr<TokenService>(new TokenService(std::move(prepared), config));
}

Result<std::vector<TokenResponse>> TokenService::generate_cohort(std::span<const TokenRequest> requests) {
    // Validate every member before any is queued (serving.cpp:2413-2438).
    if (requests.empty()) return Status::invalid_argument("inference cohort must not be empty");
    if (config_.max_queued_requests != 0U && requests.size() > config_.max_queued_requests) {
        return Status::invalid_state("inference cohort exceeds submission queue capacity");
    }
    const auto& model_config = prepared_->model().config();
    for (const auto& r : requests) {
        if (r.prompt.empty()) return Status::invalid_argument("request prompt produces no tokens");
        if (r.prompt.size() + r.max_new_tokens > model_config.context_length) {
            return Status::invalid_argument("prompt plus requested output exceeds model context length");
        }
        for (const TokenId t : r.prompt) {
            if (t < 0 || static_cast<std::uint64_t>(t) >= model_config.vocabulary_size) {
                return Status::invalid_argument("input token is outside model vocabulary");
            }
        }
    }

    const auto submitted = Clock::now();
    std::vector<Work> work(requests.size());
    std::deque<Work*> queued;
    std::vector<TokenResponse> responses(requests.size());
    for (std::size_t i = 0; i < requests.size(); ++i) {
        work[i].index = i;
        work[i].request = &requests[i];
        work[i].submitted = submitted;
        responses[i].metrics.request_id = next_request_++;
        responses[i].metrics.prompt_tokens = requests[i].prompt.size();
        if (requests[i].max_new_tokens == 0U) {
            work[i].done = true;  // run_autoregressive returns before prefill
            work[i].admitted = work[i].first_token = work[i].finished = submitted;
        } else {
            queued.push_back(&work[i]);
        }
    }

    const auto& caps = prepared_->capabilities();
    const std::uint32_t prefill_width = std::max<std::uint32_t>(caps.max_prefill_batch_width, 1U);
    const std::uint32_t decode_width = std::max<std::uint32_t>(caps.max_decode_batch_width, 1U);
    std::vector<Work*> active;
    std::uint64_t reserved = 0;

    const auto finish = [&](Work& w) {
        w.finished = Clock::now();
        if (w.sequence) w.kv_bytes = w.sequence->resources().committed_kv_bytes;
        w.sequence.reset();  // returns its KV pages
        reserved -= w.reserved_bytes;
        w.reserved_bytes = 0;
    };

    while (!queued.empty() || !active.empty()) {
        // Admission, in arrival order, while capacity allows.
        while (!queued.empty()) {
            Work* w = queued.front();
            const std::uint64_t tokens = w->request->prompt.size() + w->request->max_new_tokens;
            const auto decision = capacity_.evaluate(active.size(), reserved, *prepared_, config_.plan, tokens);
            if (!decision.admit) {
                if (active.empty()) {
                    return Status::invalid_state("request cannot be admitted: " + decision.reason);
                }
                break;
            }
            auto sequence = prepared_->create_sequence(config_.plan);
            if (!sequence) return sequence.status();
            w->sequence = std::move(sequence).value();
            w->reserved_bytes = decision.reservation_bytes;
            w->admitted = Clock::now();
            reserved += decision.reservation_bytes;
            active.push_back(w);
            queued.pop_front();
        }

        // One worker cycle.
        std::vector<runtime_detail::SchedulableSequence> candidates;
        for (std::size_t slot = 0; slot < active.size(); ++slot) {
            const Work& w = *active[slot];
            std::uint32_t max_tokens = 1U;
            if (w.prefilling()) {
                const std::size_t remaining = w.request->prompt.size() - w.prompt_position;
                max_tokens = static_cast<std::uint32_t>(std::min<std::size_t>(
                    {remaining, config_.plan.scheduling.prefill_quantum_tokens, prefill_width}));
            }
            candidates.push_back({slot, w.prefilling() ? runtime_detail::WorkPhase::prefill
                                                       : runtime_detail::WorkPhase::decode,
                                  max_tokens});
        }
        const auto batch = microbatch_.schedule(candidates, config_.token_budget_per_cycle);
        ++stats_.cycles;

        for (std::size_t i = 0; i < batch.slices.size();) {
            const auto phase = batch.slices[i].phase;
            std::size_t end = i;
            while (end < batch.slices.size() && batch.slices[end].phase == phase) ++end;
            if (phase == runtime_detail::WorkPhase::prefill) {
                // Consecutive prefill slices: one physical multi-sequence call.
                std::vector<runtime_detail::PrefillBatchItem> items;
                std::vector<Work*> owners;
                for (std::size_t s = i; s < end; ++s) {
                    Work* w = active[batch.slices[s].slot];
                    const auto count = batch.slices[s].token_count;
                    const bool last = w->prompt_position + count == w->request->prompt.size();
                    items.push_back({w->sequence.get(),
                                     std::span<const TokenId>(w->request->prompt).subspan(w->prompt_position, count),
                                     last ? runtime_detail::PrefillBatchOutput::greedy
                                          : runtime_detail::PrefillBatchOutput::discard});
                    owners.push_back(w);
                }
                const auto started = Clock::now();
                auto result = prepared_->prefill_batch(items);
                if (!result) return result.status();
                const auto now = Clock::now();
                stats_.prefill_ms += milliseconds(now - started);
                ++stats_.prefill_calls;
                stats_.max_prefill_sequences = std::max<std::uint32_t>(stats_.max_prefill_sequences,
                                                                       static_cast<std::uint32_t>(items.size()));
                for (std::size_t j = 0; j < owners.size(); ++j) {
                    Work* w = owners[j];
                    w->prompt_position += items[j].tokens.size();
                    stats_.prefill_tokens += items[j].tokens.size();
                    if (!w->prefilling()) {
                        const auto& token = result.value().items[j].greedy_token;
                        if (!token) return Status::internal_error("prefill batch returned no greedy token");
                        if (w->accept(*token, now)) finish(*w);
                    }
                }
            } else {
                // Consecutive decode slices: launches of up to the decode width.
                for (std::size_t begin = i; begin < end; begin += decode_width) {
                    const std::size_t stop = std::min<std::size_t>(end, begin + decode_width);
                    std::vector<runtime_detail::GreedyDecodeBatchItem> items;
                    std::vector<Work*> owners;
                    for (std::size_t s = begin; s < stop; ++s) {
                        Work* w = active[batch.slices[s].slot];
                        items.push_back({w->sequence.get(), w->tokens.back()});
                        owners.push_back(w);
                    }
                    const auto started = Clock::now();
                    auto result = prepared_->decode_greedy_batch(items);
                    if (!result) return result.status();
                    const auto now = Clock::now();
                    stats_.decode_ms += milliseconds(now - started);
                    ++stats_.decode_calls;
                    stats_.decode_rows += items.size();
                    stats_.max_decode_width =
                        std::max<std::uint32_t>(stats_.max_decode_width, static_cast<std::uint32_t>(items.size()));
                    if (result.value().size() != items.size()) {
                        return Status::internal_error("decode batch returned the wrong token count");
                    }
                    for (std::size_t j = 0; j < owners.size(); ++j) {
                        if (owners[j]->accept(result.value()[j], now)) finish(*owners[j]);
                    }
                }
            }
            i = end;
        }
        active.erase(std::remove_if(active.begin(), active.end(), [](const Work* w) { return w->done; }),
                     active.end());
    }

    for (std::size_t i = 0; i < work.size(); ++i) {
        const Work& w = work[i];
        auto& r = responses[i];
        r.tokens = w.tokens;
        r.hit_stop = w.hit_stop;
        r.metrics.generated_tokens = w.tokens.size();
        r.metrics.kv_bytes = w.kv_bytes;
        if (w.tokens.empty()) continue;
        r.metrics.queue_ms = milliseconds(w.admitted - w.submitted);
        r.metrics.prefill_ms = milliseconds(w.first_token - w.admitted);
        r.metrics.ttft_ms = milliseconds(w.first_token - w.submitted);
        r.metrics.decode_ms = milliseconds(w.finished - w.first_token);
        r.metrics.total_ms = milliseconds(w.finished - w.submitted);
    }
    return responses;
}

} // namespace air

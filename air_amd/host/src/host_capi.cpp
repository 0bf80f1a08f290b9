// host_capi.cpp -- the C ABI of include/air_host.h over the C++ executor.
#include "air_host.h"

#include "air/gguf.hpp"
#include "air/hip_backend.hpp"
#include "air/synthetic.hpp"
#include "air/token_service.hpp"
#include "air_hip.h"

#include <chrono>
#include <exception>
#include <optional>
#include <string>

struct air_host_model {
    std::shared_ptr<const air::ModelDefinition> model;
    std::optional<air::TokenId> eos;
};

struct air_host_engine {
    std::shared_ptr<air::HipPreparedModel> prepared;
    std::unique_ptr<air::TokenService> service;
};

namespace {

thread_local std::string g_last_error;

int fail(const air::Status& s) {
    g_last_error = s.message();
    switch (s.code()) {
    case air::ErrorCode::ok: return AIR_HIP_OK;
    case air::ErrorCode::invalid_argument: return AIR_HIP_INVALID_ARGUMENT;
    case air::ErrorCode::invalid_state: return AIR_HIP_INVALID_STATE;
    case air::ErrorCode::io_error: return AIR_HIP_IO_ERROR;
    case air::ErrorCode::cancelled: return AIR_HIP_CANCELLED;
    case air::ErrorCode::data_error: return AIR_HIP_DATA_ERROR;
    case air::ErrorCode::unsupported: return AIR_HIP_UNSUPPORTED;
    default: return AIR_HIP_INTERNAL_ERROR;
    }
}

int fail_argument(const char* message) { return fail(air::Status::invalid_argument(message)); }

// Nothing throws across the boundary (allocation failure included).
template <typename F>
int guarded(F&& body) {
    try {
        return body();
    } catch (const std::exception& e) {
        g_last_error = std::string("host library exception: ") + e.what();
        return AIR_HIP_INTERNAL_ERROR;
    } catch (...) {
        g_last_error = "host library exception";
        return AIR_HIP_INTERNAL_ERROR;
    }
}

} // namespace

extern "C" {

int air_host_abi_version(void) { return AIR_HOST_ABI_VERSION; }

const char* air_host_last_error(void) { return g_last_error.c_str(); }

int air_host_synthetic_qwen2(const air_host_qwen2_spec* spec, air_host_model** out) {
    if (!spec || !out) return fail_argument("spec and out must not be null");
    *out = nullptr;
    return guarded([&] {
        air::SyntheticQwen2Spec s;
        s.config = air::qwen2_config(spec->layers, spec->embedding, spec->ffn, spec->heads, spec->kv_heads, spec->vocab,
                                     spec->context);
        s.weight_format = spec->weight_format;
        s.embedding_format = spec->embedding_format;
        s.seed = spec->seed;
        s.sigma = spec->sigma;
        s.qkv_bias = spec->qkv_bias != 0;
        s.output_bias = spec->output_bias != 0;
        s.tied_output = spec->tied_output != 0;
        auto model = air::make_synthetic_qwen2(s);
        if (!model) return fail(model.status());
        *out = new air_host_model{std::move(model).value(), std::nullopt};
        return static_cast<int>(AIR_HIP_OK);
    });
}

int air_host_model_describe(const air_host_model* model, uint64_t* storage_bytes, uint64_t* tensors) {
    if (!model || !model->model) return fail_argument("model must not be null");
    if (storage_bytes) *storage_bytes = model->model->storage() ? model->model->storage()->bytes().size() : 0U;
    if (tensors) *tensors = model->model->tensors().size();
    return AIR_HIP_OK;
}

int air_host_model_release(air_host_model* model) {
    delete model;
    return AIR_HIP_OK;
}

int air_host_load_gguf(const char* path, air_host_model** out) {
    if (!path || !out) return fail_argument("path and out must not be null");
    *out = nullptr;
    return guarded([&] {
        air::gguf::ModelInfo info;
        auto model = air::gguf::load_model(path, &info);
        if (!model) return fail(model.status());
        *out = new air_host_model{std::move(model).value(), info.eos};
        return static_cast<int>(AIR_HIP_OK);
    });
}

int air_host_write_gguf(const air_host_model* model, const char* path, int32_t eos) {
    if (!model || !model->model || !path) return fail_argument("model and path must not be null");
    return guarded([&] {
        air::gguf::WriteOptions options;
        if (eos >= 0) options.eos = eos;
        if (air::Status s = air::gguf::write_model(path, *model->model, options); !s) return fail(s);
        return static_cast<int>(AIR_HIP_OK);
    });
}

int air_host_model_get_config(const air_host_model* model, air_host_model_config* out) {
    if (!model || !model->model || !out) return fail_argument("model and out must not be null");
    const auto& c = model->model->config();
    *out = air_host_model_config{c.layer_count, c.embedding_size, c.feed_forward_size, c.attention_head_count,
                                 c.kv_head_count, c.rope_dimension_count, c.vocabulary_size, c.context_length,
                                 c.attention_sliding_window, c.rope_frequency_base, c.rms_norm_epsilon,
                                 model->eos ? *model->eos : -1,
                                 static_cast<uint32_t>(model->model->tensors().size())};
    return AIR_HIP_OK;
}

int air_host_model_tensor(const air_host_model* model, uint32_t index, air_host_tensor_info* out) {
    if (!model || !model->model || !out) return fail_argument("model and out must not be null");
    const auto& tensors = model->model->tensors();
    if (index >= tensors.size()) return fail_argument("tensor index is out of range");
    const auto& t = tensors[index];
    if (t.shape.dimensions.size() > 8U) return fail(air::Status::unsupported("tensor rank above 8"));
    *out = air_host_tensor_info{};
    out->name = t.name.c_str();
    out->type = t.format_type;
    out->rank = static_cast<uint32_t>(t.shape.dimensions.size());
    for (std::size_t d = 0; d < t.shape.dimensions.size(); ++d) out->dims[d] = t.shape.dimensions[d];
    out->offset = t.byte_offset;
    out->size = t.byte_size;
    return AIR_HIP_OK;
}

int air_host_engine_create(const air_host_model* model, const air_host_engine_config* config, air_host_engine** out) {
    if (!model || !model->model || !config || !out) return fail_argument("model, config and out must not be null");
    *out = nullptr;
    if (config->prefill_tactic != AIR_HIP_LINEAR_DECODE && config->prefill_tactic != AIR_HIP_LINEAR_PREFILL) {
        return fail_argument("prefill tactic must be AIR_HIP_LINEAR_DECODE or AIR_HIP_LINEAR_PREFILL");
    }
    if (config->attention_tactic != 0 && config->attention_tactic != 1) {
        return fail_argument("attention tactic must be 0 (baseline) or 1 (online softmax)");
    }
    return guarded([&] {
        air::HipPrepareOptions options;
        options.device = config->device;
        options.kv_pool_pages = config->kv_pool_pages;
        options.kv_chunk_pages = config->kv_chunk_pages;
        options.kv_page_tokens = config->page_tokens ? config->page_tokens : 16U;
        if (config->max_step_rows) options.max_step_rows = config->max_step_rows;
        options.decode_graphs = config->eager_decode == 0;
        auto prepared = air::HipPreparedModel::create(model->model, options);
        if (!prepared) return fail(prepared.status());
        std::shared_ptr<air::HipPreparedModel> shared(std::move(prepared).value());

        air::TokenServiceConfig sc;
        sc.plan.backend = air::BackendKind::hip;
        sc.plan.kv.page_tokens = config->page_tokens ? config->page_tokens : 16U;
        sc.plan.linear.prefill_block = config->prefill_tactic == AIR_HIP_LINEAR_PREFILL
                                           ? air::QuantizedLinearExecutionKind::hip_prefill
                                           : air::QuantizedLinearExecutionKind::hip_decode;
        sc.plan.linear.decode_block = air::QuantizedLinearExecutionKind::hip_decode;
        sc.plan.linear.decode_output = air::QuantizedLinearExecutionKind::hip_decode;
        const auto attention = config->attention_tactic == 1 ? air::AttentionExecutionKind::online_softmax
                                                             : air::AttentionExecutionKind::baseline;
        sc.plan.attention.prefill = attention;
        sc.plan.attention.decode = attention;
        if (config->prefill_quantum_tokens) sc.plan.scheduling.prefill_quantum_tokens = config->prefill_quantum_tokens;
        if (config->token_budget_per_cycle) sc.token_budget_per_cycle = config->token_budget_per_cycle;
        if (config->max_active_requests) sc.max_active_requests = config->max_active_requests;
        auto service = air::TokenService::create(shared, sc);
        if (!service) return fail(service.status());
        *out = new air_host_engine{std::move(shared), std::move(service).value()};
        return static_cast<int>(AIR_HIP_OK);
    });
}

int air_host_engine_release(air_host_engine* engine) {
    delete engine;
    return AIR_HIP_OK;
}

int air_host_engine_capacity(const air_host_engine* engine, air_host_capacity* out) {
    if (!engine || !out) return fail_argument("engine and out must not be null");
    return guarded([&] {
        const auto& prepared = *engine->prepared;
        const auto capacity = prepared.sequence_capacity_bytes();
        const auto free = prepared.free_device_bytes();
        if (!capacity || !free) return fail(air::Status::invalid_state("device memory information is unavailable"));
        *out = air_host_capacity{*capacity, *free, prepared.kv_pool_allocated_bytes(), prepared.kv_pool_free_bytes()};
        return static_cast<int>(AIR_HIP_OK);
    });
}

int air_host_engine_sequence_bytes(const air_host_engine* engine, uint64_t tokens, uint64_t* out) {
    if (!engine || !out) return fail_argument("engine and out must not be null");
    return guarded([&] {
        *out = engine->prepared->estimate_sequence_device_bytes(engine->service->config().plan, tokens);
        return static_cast<int>(AIR_HIP_OK);
    });
}

int air_host_generate_cohort(air_host_engine* engine, const int32_t* prompt_tokens, const uint32_t* prompt_lengths,
                             uint32_t requests, uint32_t max_new_tokens, int32_t stop_token, int32_t* out_tokens,
                             uint32_t* out_counts, air_host_cohort_stats* stats) {
    if (!engine || !prompt_tokens || !prompt_lengths || !out_counts || (max_new_tokens && !out_tokens)) {
        return fail_argument("engine, prompts, lengths and outputs must not be null");
    }
    return guarded([&] {
        std::vector<air::TokenRequest> batch(requests);
        std::size_t offset = 0;
        for (uint32_t i = 0; i < requests; ++i) {
            batch[i].prompt.assign(prompt_tokens + offset, prompt_tokens + offset + prompt_lengths[i]);
            offset += prompt_lengths[i];
            batch[i].max_new_tokens = max_new_tokens;
            if (stop_token >= 0) batch[i].stop_token = stop_token;
        }
        const air::TokenServiceStats before = engine->service->stats();
        const auto started = std::chrono::steady_clock::now();
        auto responses = engine->service->generate_cohort(batch);
        const auto finished = std::chrono::steady_clock::now();
        if (!responses) return fail(responses.status());
        double ttft = 0.0;
        std::uint64_t generated = 0;
        for (uint32_t i = 0; i < requests; ++i) {
            const auto& r = responses.value()[i];
            out_counts[i] = static_cast<uint32_t>(r.tokens.size());
            for (std::size_t t = 0; t < r.tokens.size(); ++t) {
                out_tokens[static_cast<std::size_t>(i) * max_new_tokens + t] = r.tokens[t];
            }
            ttft += r.metrics.ttft_ms;
            generated += r.tokens.size();
        }
        if (stats) {
            const auto& after = engine->service->stats();
            stats->wall_ms = std::chrono::duration<double, std::milli>(finished - started).count();
            stats->prefill_ms = after.prefill_ms - before.prefill_ms;
            stats->decode_ms = after.decode_ms - before.decode_ms;
            stats->cycles = after.cycles - before.cycles;
            stats->prefill_calls = after.prefill_calls - before.prefill_calls;
            stats->prefill_tokens = after.prefill_tokens - before.prefill_tokens;
            stats->decode_calls = after.decode_calls - before.decode_calls;
            stats->decode_rows = after.decode_rows - before.decode_rows;
            stats->max_decode_width = after.max_decode_width;
            stats->max_prefill_sequences = after.max_prefill_sequences;
            stats->generated_tokens = generated;
            stats->mean_ttft_ms = requests ? ttft / requests : 0.0;
        }
        return static_cast<int>(AIR_HIP_OK);
    });
}

} // extern "C"

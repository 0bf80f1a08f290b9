/*
 * air_host.h -- C ABI of the host executor library (libair_host.so).
 *
 * libair_host.so is the C++20 executor around the kernel library of
 * air_hip.h: model definitions, HipPreparedModel (resident weights, the
 * Qwen2 step engine, paged KV), CapacityScheduler / MicrobatchScheduler and
 * TokenService, the token-id caller slice of InferenceService
 * (src/runtime/serving.cpp:2401-2481).  This header exposes that caller
 * slice to non-C++ callers (Python ctypes in this repository): build or load
 * a model, prepare it on a device, run a cohort of greedy token requests.
 *
 * Conventions follow air_hip.h: plain C types, air_hip_status return codes,
 * air_host_last_error() for the calling thread's message, explicit release.
 */
#ifndef AIR_HOST_H
#define AIR_HOST_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AIR_HOST_ABI_VERSION 1

typedef struct air_host_model air_host_model;
typedef struct air_host_engine air_host_engine;

/* Version of this C ABI (no counterpart in the reference). */
int air_host_abi_version(void);
/* The calling thread's last failure message: the message of a failing
 * air::Status (include/air/status.hpp:19-40). */
const char* air_host_last_error(void);

/* Random-init Qwen2 model (weights N(0, sigma) quantized to weight_format,
 * norms 1, RoPE theta 1e6, RMSNorm eps 1e-6), generated on the host; the
 * same bytes for the same spec on every machine.  The in-memory form of the
 * synthetic GGUF models the reference's tests write (tests/core_tests.cpp:80,
 * tests/make_quantized_qwen2_gguf.py), as a ModelDefinition
 * (include/air/model.hpp:57). */
typedef struct air_host_qwen2_spec {
    uint32_t layers;
    uint32_t embedding;
    uint32_t ffn;
    uint32_t heads;
    uint32_t kv_heads;
    uint64_t vocab;
    uint64_t context;
    uint32_t weight_format;     /* GGML type id: 8 Q8_0, 2 Q4_0, 12 Q4_K */
    uint32_t embedding_format;
    uint64_t seed;
    float sigma;
    int32_t qkv_bias;
    int32_t output_bias;
    int32_t tied_output;
} air_host_qwen2_spec;

int air_host_synthetic_qwen2(const air_host_qwen2_spec* spec, air_host_model** out);
/* Model bytes and tensor count, for callers that size host memory
 * (ModelDefinition's storage and tensors(), include/air/model.hpp:57-72). */
int air_host_model_describe(const air_host_model* model, uint64_t* storage_bytes, uint64_t* tensors);
/* Frees the model (the ModelDefinition and its mapped storage). */
int air_host_model_release(air_host_model* model);

/* A GGUF v3 file (memory-mapped, read-only), loaded with the rules of AIR's
 * GgufFormat::load (src/formats/gguf/gguf_format.cpp:278-311, gguf_reader.cpp:
 * 346-472): the same limits, required keys, defaults and error classes
 * (io_error: unreadable; invalid_argument: not GGUF; unsupported: not V3 or
 * split; data_error: malformed). */
int air_host_load_gguf(const char* path, air_host_model** out);
/* Writes the model as a GGUF v3 file: Qwen2 metadata from its config, a
 * placeholder vocabulary of vocab tokens, eos_token_id when eos >= 0, and
 * every tensor at 32-byte aligned offsets -- the layout GgufFormat::load
 * reads (src/formats/gguf/gguf_format.cpp:283), as the reference's test
 * writers produce it (tests/core_tests.cpp:80-120). */
int air_host_write_gguf(const air_host_model* model, const char* path, int32_t eos);

typedef struct air_host_model_config {
    uint32_t layers;
    uint32_t embedding;
    uint32_t ffn;
    uint32_t heads;
    uint32_t kv_heads;
    uint32_t rope_dims;
    uint64_t vocab;
    uint64_t context;
    uint64_t sliding_window;
    double rope_base;
    double rms_eps;
    int32_t eos;                /* -1 when the file names none (or for synthetic models) */
    uint32_t tensors;
} air_host_model_config;
/* ModelDefinition::config() (include/air/model.hpp:17-55, 67). */
int air_host_model_get_config(const air_host_model* model, air_host_model_config* out);

/* Tensor `index` of the model's table (file order for GGUF). */
typedef struct air_host_tensor_info {
    const char* name;           /* valid while the model is alive */
    uint32_t type;              /* GGML type id */
    uint32_t rank;
    uint64_t dims[8];           /* GGML order: dims[0] is the contiguous direction */
    uint64_t offset;            /* byte offset in the model's storage (the file) */
    uint64_t size;              /* bytes */
} air_host_tensor_info;
/* Entry `index` of ModelDefinition::tensors() (include/air/model.hpp:70). */
int air_host_model_tensor(const air_host_model* model, uint32_t index, air_host_tensor_info* out);

typedef struct air_host_engine_config {
    int32_t device;
    uint32_t page_tokens;          /* KV page size in tokens (16 in the reference's CUDA plans) */
    uint32_t kv_pool_pages;        /* 0: the KV pool grows on demand (capacity = free + allocated); else a
                                      fixed pool of this many pages, allocated with the first sequence */
    uint32_t max_step_rows;        /* rows per device step (prefill width) */
    int32_t prefill_tactic;        /* AIR_HIP_LINEAR_DECODE or AIR_HIP_LINEAR_PREFILL for prompt blocks */
    uint32_t prefill_quantum_tokens;
    uint32_t token_budget_per_cycle;
    uint32_t max_active_requests;
    int32_t attention_tactic;      /* 0 baseline (the reference's double softmax), 1 online softmax (tiled f32) */
    int32_t eager_decode;          /* 1: launch decode steps kernel by kernel instead of replaying a captured
                                      graph per batch width (for kernel-level profiling) */
    uint32_t kv_chunk_pages;       /* pages per growth chunk of a growing pool (0: about 256 MiB of pages) */
} air_host_engine_config;

/* Prepares the model on `device` (weights resident, repacked) and creates
 * the token service.  The engine keeps the model alive.  A PreparedModel
 * (src/runtime/backend.hpp:97-145) under the token-id slice of
 * InferenceService (src/runtime/serving.cpp:203, 2034-2050). */
int air_host_engine_create(const air_host_model* model, const air_host_engine_config* config, air_host_engine** out);
/* Drains and frees the engine (InferenceService::shutdown,
 * src/runtime/serving.cpp:2037). */
int air_host_engine_release(air_host_engine* engine);

typedef struct air_host_capacity {
    uint64_t sequence_capacity_bytes;  /* what admission reserves against: free device memory plus the KV pool
                                          allocated (a growing pool), or the fixed pool */
    uint64_t free_device_bytes;        /* hipMemGetInfo free */
    uint64_t kv_pool_allocated_bytes;  /* KV pages allocated so far (0 before any step of a growing pool) */
    uint64_t kv_pool_free_bytes;       /* pool pages no sequence holds */
} air_host_capacity;

/* The engine's capacity answers (PreparedModel::sequence_capacity_bytes,
 * free_device_bytes, kv_pool_allocated_bytes, kv_pool_free_bytes,
 * src/runtime/backend.hpp:118-121). */
int air_host_engine_capacity(const air_host_engine* engine, air_host_capacity* out);
/* The device bytes admission reserves for a request of `tokens` prompt plus
 * generated tokens (PreparedModel::estimate_sequence_device_bytes with the
 * engine's plan, src/runtime/backend.hpp:134). */
int air_host_engine_sequence_bytes(const air_host_engine* engine, uint64_t tokens, uint64_t* out);

typedef struct air_host_cohort_stats {
    double wall_ms;                /* whole cohort, submission to last token */
    double prefill_ms;             /* inside prefill_batch calls */
    double decode_ms;              /* inside decode_greedy_batch calls */
    uint64_t cycles;
    uint64_t prefill_calls;
    uint64_t prefill_tokens;
    uint64_t decode_calls;
    uint64_t decode_rows;
    uint32_t max_decode_width;
    uint32_t max_prefill_sequences;
    uint64_t generated_tokens;
    double mean_ttft_ms;
} air_host_cohort_stats;

/* Runs `requests` greedy requests to completion, as InferenceService runs
 * token requests (src/runtime/serving.cpp:2401-2481).  Prompts are concatenated
 * in prompt_tokens with prompt_lengths[i] tokens each; out_tokens holds
 * requests x max_new_tokens ids (row i = request i), out_counts[i] the
 * number generated (fewer when stop_token >= 0 was produced).  stats may be
 * NULL; its counters cover this call only. */
int air_host_generate_cohort(air_host_engine* engine, const int32_t* prompt_tokens, const uint32_t* prompt_lengths,
                             uint32_t requests, uint32_t max_new_tokens, int32_t stop_token, int32_t* out_tokens,
                             uint32_t* out_counts, air_host_cohort_stats* stats);

#ifdef __cplusplus
}
#endif

#endif /* AIR_HOST_H */

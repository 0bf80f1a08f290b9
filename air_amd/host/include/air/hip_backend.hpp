// hip_backend.hpp -- the HIP prepared model: Qwen2 linears resident on one GPU.
//
// HipPreparedModel is the MI355X counterpart of CudaPreparedModel
// (src/runtime/backend.cpp:268-574): it owns the device residency of every
// quantized projection, advertises the HIP linear tactics per operation scope
// and answers the capacity queries CapacityScheduler asks.  Weights become
// resident once, repacked into the wavefront tile layout by
// air_hip_matrix_prepare; q|k|v and gate|up are concatenated along N (their
// GGUF rows are contiguous, so the fusion is a byte append) when the parts
// share a format, and their f32 biases are concatenated the same way.
//
// Sequences (paged KV, attention, device greedy selection) run on the
// HipStepEngine of hip_step.hpp, created with the first sequence from the
// plan's KV page size.  Checkpoints are not provided.
#pragma once

#include "air/backend.hpp"

#include <memory>

struct air_hip_context;
struct air_hip_matrix;
struct air_hip_kv_layout;

namespace air {

enum class LinearRole {
    attn_qkv = 0,   // fused q|k|v, N = q_width + 2 kv_width
    attn_q,
    attn_k,
    attn_v,
    attn_output,
    ffn_gate_up,    // fused gate|up, N = 2 ffn
    ffn_gate,
    ffn_up,
    ffn_down,
    output,         // lm_head (output.weight, or token_embd.weight when tied)
};

[[nodiscard]] const char* to_string(LinearRole role) noexcept;

struct HipLinearInfo {
    std::uint32_t format_type{0};
    std::uint64_t k{0};
    std::uint64_t n{0};
    bool has_bias{false};
    std::uint64_t resident_bytes{0};
};

struct HipPrepareOptions {
    int device{0};
    void* stream{nullptr};              // hipStream_t the engine launches on (null: a stream of its own)
    std::uint32_t max_decode_rows{64};  // workspace reserved for decode widths
    bool fuse{true};                    // concatenate q|k|v and gate|up when formats agree
    // 0 (default): the KV pool grows on demand, a chunk of kv_chunk_pages
    // pages at a time, and sequence_capacity_bytes answers the device memory
    // free plus the pool allocated, as the reference's growing pool does
    // (src/runtime/backend.cpp:541-560).  Otherwise a pool of exactly this
    // many pages, allocated with the first sequence, which admission is then
    // held to (a cap on KV memory).
    std::uint32_t kv_pool_pages{0};
    // Pages per chunk of a growing pool, rounded down to a power of two;
    // 0: about 256 MiB of pages.
    std::uint32_t kv_chunk_pages{0};
    // Page size of the plans this model will serve: a fixed pool is sized in
    // these pages, and a plan with another page size is refused.
    std::uint32_t kv_page_tokens{16};
    std::uint32_t max_step_rows{512};   // rows per device step (prefill chunk)
    // Decode steps (one row per sequence, greedy outputs) replay one captured
    // HIP graph per batch width instead of launching ~13 kernels per layer.
    bool decode_graphs{true};
};

class HipStepEngine;
struct StepResult;
enum class RowOutput : std::uint8_t;

class HipPreparedModel final : public runtime_detail::PreparedModel {
public:
    ~HipPreparedModel() override;
    HipPreparedModel(const HipPreparedModel&) = delete;
    HipPreparedModel& operator=(const HipPreparedModel&) = delete;

    [[nodiscard]] static Result<std::unique_ptr<HipPreparedModel>> create(std::shared_ptr<const ModelDefinition> model,
                                                                          const HipPrepareOptions& options);

    // PreparedModel
    [[nodiscard]] BackendKind backend() const noexcept override { return BackendKind::hip; }
    [[nodiscard]] const BackendCapabilities& capabilities() const noexcept override { return capabilities_; }
    [[nodiscard]] const ModelDefinition& model() const noexcept override { return *model_; }
    [[nodiscard]] Result<std::unique_ptr<runtime_detail::SequenceState>> create_sequence(
        const ExecutionPlan& plan) override;
    [[nodiscard]] Result<std::unique_ptr<runtime_detail::SequenceState>> restore_sequence(
        const ExecutionPlan& plan, const runtime_detail::SequenceCheckpoint& checkpoint) override;
    [[nodiscard]] std::uint64_t resident_device_bytes() const noexcept override;
    [[nodiscard]] std::uint64_t estimate_sequence_device_bytes(const ExecutionPlan& plan,
                                                               std::uint64_t max_tokens) const noexcept override;
    [[nodiscard]] std::optional<std::uint64_t> sequence_capacity_bytes() const override;
    [[nodiscard]] std::optional<std::uint64_t> free_device_bytes() const override;
    [[nodiscard]] std::uint64_t kv_pool_allocated_bytes() const noexcept override;
    [[nodiscard]] std::uint64_t kv_pool_free_bytes() const noexcept override;
    // Pages per growth chunk of the KV pool (0: a fixed pool, or no sequence yet).
    [[nodiscard]] std::uint32_t engine_chunk_pages() const noexcept;
    [[nodiscard]] Result<runtime_detail::PrefillBatchExecution> prefill_batch(
        std::span<const runtime_detail::PrefillBatchItem> items) override;
    [[nodiscard]] Result<std::vector<TokenId>> decode_greedy_batch(
        std::span<const runtime_detail::GreedyDecodeBatchItem> items) override;
    // The batched decode step of decode_greedy_batch returning every row's
    // vocabulary logits instead of its greedy token (one row per sequence, on
    // the same captured graph).  The reference's differential verifier
    // compares executors on logits step by step (src/verification/main.cpp:
    // 319-402); this is that comparison's batched entry point.  No
    // counterpart in PreparedModel.
    [[nodiscard]] Result<std::vector<std::vector<float>>> decode_batch_logits(
        std::span<const runtime_detail::GreedyDecodeBatchItem> items);

    // The lm_head matrix and whether it is token_embd (tied embeddings).
    [[nodiscard]] air_hip_matrix* output_matrix() const noexcept { return output_.matrix; }
    [[nodiscard]] const float* output_bias() const noexcept { return output_.bias; }
    [[nodiscard]] bool output_is_embedding() const noexcept { return output_is_embedding_; }
    [[nodiscard]] const HipPrepareOptions& options() const noexcept { return options_; }

    // Linear engine.  x: device f32 [rows x K], y: device f32 [rows x N], both
    // row-major; the role's bias (if any) is fused.  Asynchronous on the
    // engine's stream.  Tactics: hip-decode (exact codes, M <= 64 in
    // practice), hip-prefill (f16 MFMA GEMM, M up to 4096).
    [[nodiscard]] Status linear(std::uint32_t layer, LinearRole role, const float* x, float* y,
                                std::uint32_t rows, QuantizedLinearExecutionKind tactic) const;
    // One-row decode linear with the step's RMSNorm before it (norm_weight
    // non-null) and a residual add or SwiGLU after it (air_hip_decode_linear_fused).
    [[nodiscard]] Status decode_linear_fused(std::uint32_t layer, LinearRole role, const float* x, float* y,
                                             const float* norm_weight, double eps, int epilogue) const;
    // A linear and the element-wise step work on its output: residual add
    // (then, with norm_weight, the next RMSNorm into norm_out) or SwiGLU
    // (air_hip_linear_epilogue; carried by the split reduction at M 2..64).
    [[nodiscard]] Status linear_epilogue(std::uint32_t layer, LinearRole role, const float* x, std::uint32_t rows,
                                         float* out, int epilogue, const float* norm_weight, float* norm_out,
                                         double eps, QuantizedLinearExecutionKind tactic) const;
    // The q|k|v linear with RoPE and the KV append after it
    // (air_hip_linear_rope_kv; carried by the split reduction at M 2..64).
    [[nodiscard]] Status linear_rope_kv(std::uint32_t layer, LinearRole role, const float* x, std::uint32_t rows,
                                        float* qkv, const air_hip_kv_layout* kv, const std::int32_t* positions,
                                        const std::int32_t* page_tables, std::uint32_t q_heads,
                                        std::uint32_t kv_heads, std::uint32_t head_dim, std::uint32_t rope_dims,
                                        const float* rope_table, std::uint64_t table_positions,
                                        QuantizedLinearExecutionKind tactic) const;
    [[nodiscard]] Result<HipLinearInfo> linear_info(std::uint32_t layer, LinearRole role) const;
    [[nodiscard]] bool fused_qkv() const noexcept { return fused_qkv_; }
    [[nodiscard]] bool fused_gate_up() const noexcept { return fused_gate_up_; }
    // Every block linear is in a tile format (Q8_0, Q5_0, Q4_0, Q4_K), so the
    // fused M = 1 GEMV (air_hip_decode_linear_fused) takes all of them.
    [[nodiscard]] bool tile_formats() const noexcept { return tile_formats_; }
    [[nodiscard]] Status set_stream(void* stream);
    [[nodiscard]] Status synchronize() const;
    [[nodiscard]] air_hip_context* context() const noexcept { return ctx_; }
    [[nodiscard]] int device() const noexcept { return device_; }

private:
    struct Linear {
        air_hip_matrix* matrix{nullptr};
        float* bias{nullptr};  // device f32 [N] or null
        HipLinearInfo info{};
    };
    struct Layer {
        Linear qkv, q, k, v, o, gate_up, gate, up, down;
    };

    HipPreparedModel(std::shared_ptr<const ModelDefinition> model, int device);
    [[nodiscard]] const Linear* find(std::uint32_t layer, LinearRole role) const noexcept;
    [[nodiscard]] Status make_linear(std::span<const TensorDescriptor* const> parts,
                                     std::span<const TensorDescriptor* const> biases, Linear& out);
    void release(Linear& linear) noexcept;

    std::shared_ptr<const ModelDefinition> model_;
    int device_{0};
    air_hip_context* ctx_{nullptr};
    void* owned_stream_{nullptr};  // hipStream_t created when the options name none
    BackendCapabilities capabilities_{};
    std::vector<Layer> layers_;
    Linear output_{};
    bool fused_qkv_{false};
    bool fused_gate_up_{false};
    bool tile_formats_{true};
    bool output_is_embedding_{false};
    std::uint64_t bias_bytes_{0};
    HipPrepareOptions options_{};
    std::unique_ptr<HipStepEngine> engine_;
    [[nodiscard]] Result<HipStepEngine*> engine_for(const ExecutionPlan& plan);
    [[nodiscard]] Result<StepResult> decode_rows(std::span<const runtime_detail::GreedyDecodeBatchItem> items,
                                                 RowOutput output);
};

// Paged fp32 K and V of every layer for max_tokens plus the two page tables,
// saturating at UINT64_MAX (backend.cpp:511-538); 0 when either count is 0.
[[nodiscard]] std::uint64_t estimate_paged_fp32_sequence_bytes(const ModelConfig& config, std::uint32_t page_tokens,
                                                               std::uint64_t max_tokens) noexcept;

// The AIR factory spelling (backend.hpp:147-150).
[[nodiscard]] Result<std::unique_ptr<runtime_detail::PreparedModel>> prepare_hip_model(
    std::shared_ptr<const ModelDefinition> model, int device_ordinal);

// Maps an air_hip_status code and the thread's last ABI message to a Status.
[[nodiscard]] Status hip_status(int rc);

} // namespace air

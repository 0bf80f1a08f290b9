// hip_step.hpp -- Qwen2 sequences on the HIP executor.
//
// HipStepEngine runs the Qwen2 step of ReferenceExecutor::step_impl
// (src/reference/reference_executor.cpp:325-428) over a batch of rows, each
// row a (sequence, position, token): embedding rows, per layer RMSNorm ->
// fused q|k|v linear (+bias) -> RoPE -> paged KV append -> attention -> o
// linear -> residual -> RMSNorm -> fused gate|up linear -> SiLU * up -> down
// linear -> residual, then the final RMSNorm, the lm_head on the rows that
// need logits and the device greedy argmax.  Decode batches hold one row per
// sequence; a prefill holds a sequence's prompt as consecutive rows (causal
// attention over each row's own prefix), so one code path serves both, the
// way CudaExecutor's step and prefill paths share their kernels
// (src/cuda/cuda_backend.cu:2661-3619).
//
// KV: fp32 pages of `page_tokens` tokens of every layer (the reference CUDA
// executor's page pool, cuda_backend.cu:1186-1300) and a host free list; a
// sequence owns the pages of its committed tokens.  By default the pool grows
// on demand in chunks of 2^k pages, each its own allocation named in a device
// chunk table (pages never move, so captured decode graphs stay valid), and
// like the reference's it never shrinks; a pool of a fixed page count is one
// allocation made with the first sequence.
#pragma once

#include "air/backend.hpp"
#include "air/hip_backend.hpp"

#include <atomic>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

namespace air {

class HipStepEngine;

class HipSequence final : public runtime_detail::SequenceState {
public:
    HipSequence(HipStepEngine& engine, const LinearPolicy& linear, const AttentionPolicy& attention);
    ~HipSequence() override;

    [[nodiscard]] BackendKind backend() const noexcept override { return BackendKind::hip; }
    [[nodiscard]] Result<std::vector<float>> prefill(std::span<const TokenId> tokens) override;
    [[nodiscard]] Status prefill_discard(std::span<const TokenId> tokens) override;
    [[nodiscard]] Result<TokenId> prefill_greedy(std::span<const TokenId> tokens) override;
    [[nodiscard]] Result<std::vector<float>> decode(TokenId token) override;
    [[nodiscard]] Result<TokenId> decode_greedy(TokenId token) override;
    [[nodiscard]] runtime_detail::SequenceResources resources() const noexcept override;
    [[nodiscard]] Result<std::unique_ptr<runtime_detail::SequenceCheckpoint>> checkpoint() const override;

    [[nodiscard]] std::uint64_t tokens() const noexcept { return tokens_; }
    [[nodiscard]] QuantizedLinearExecutionKind prefill_block_tactic() const noexcept { return prefill_block_; }
    [[nodiscard]] QuantizedLinearExecutionKind decode_block_tactic() const noexcept { return decode_block_; }
    [[nodiscard]] QuantizedLinearExecutionKind decode_output_tactic() const noexcept { return decode_output_; }
    [[nodiscard]] AttentionExecutionKind prefill_attention() const noexcept { return prefill_attention_; }
    [[nodiscard]] AttentionExecutionKind decode_attention() const noexcept { return decode_attention_; }
    [[nodiscard]] const HipStepEngine& engine() const noexcept { return engine_; }

private:
    friend class HipStepEngine;
    HipStepEngine& engine_;
    QuantizedLinearExecutionKind prefill_block_, decode_block_, decode_output_;
    AttentionExecutionKind prefill_attention_, decode_attention_;
    std::vector<std::int32_t> pages_;
    std::uint64_t tokens_{0};
};

// What a row of a step asks for.
enum class RowOutput : std::uint8_t { none = 0, greedy, logits };

struct StepRow {
    HipSequence* sequence{nullptr};
    TokenId token{0};
    RowOutput output{RowOutput::none};
};

struct StepResult {
    std::vector<TokenId> greedy;              // one per row with RowOutput::greedy, in row order
    std::vector<std::vector<float>> logits;   // one per row with RowOutput::logits, in row order
};

class HipStepEngine {
public:
    // The model's linears are already resident in `prepared`; the engine adds
    // the embedding table, norm weights, the RoPE table, the KV pool and the
    // step buffers for up to max_rows rows per step.
    [[nodiscard]] static Result<std::unique_ptr<HipStepEngine>> create(const HipPreparedModel& prepared,
                                                                       std::uint32_t page_tokens,
                                                                       std::uint32_t pool_pages,
                                                                       std::uint32_t max_rows);
    ~HipStepEngine();

    // Bytes of one KV page (every layer's K and V for page_tokens tokens).
    [[nodiscard]] static std::uint64_t kv_page_bytes(const ModelConfig& c, std::uint32_t page_tokens) noexcept;
    // Pages of a fixed pool (HipPrepareOptions::kv_pool_pages), allocated
    // with the first sequence; 0 when the pool grows on demand.
    [[nodiscard]] static std::uint32_t planned_pool_pages(const HipPreparedModel& prepared, std::uint32_t page_tokens);
    // log2 of the pages per chunk of a growing pool: `requested` rounded down
    // to a power of two, or (0) about 256 MiB of pages; 1 to 65536 pages.
    [[nodiscard]] static std::uint32_t chunk_shift_for(std::uint64_t page_bytes, std::uint32_t requested) noexcept;
    // Chunk table entries: the most chunks a growing pool can hold.
    static constexpr std::uint32_t kMaxKvChunks = 4096U;

    // Rows of several sequences; the positions are each sequence's next
    // tokens in row order.  The batch commits to every sequence on success.
    [[nodiscard]] Result<StepResult> run(std::span<const StepRow> rows, QuantizedLinearExecutionKind block_tactic,
                                         QuantizedLinearExecutionKind output_tactic,
                                         AttentionExecutionKind attention);

    [[nodiscard]] std::uint32_t page_tokens() const noexcept { return page_tokens_; }
    [[nodiscard]] std::uint64_t page_bytes() const noexcept { return page_bytes_; }
    // Pages allocated so far (a fixed pool: all of them from the start).
    [[nodiscard]] std::uint64_t pool_bytes() const noexcept { return page_bytes_ * allocated_pages_.load(std::memory_order_relaxed); }
    [[nodiscard]] std::uint64_t free_pool_bytes() const noexcept;
    [[nodiscard]] bool pool_grows() const noexcept { return growable_; }
    [[nodiscard]] std::uint32_t chunk_pages() const noexcept { return growable_ ? 1U << chunk_shift_ : 0U; }
    [[nodiscard]] std::uint64_t resident_bytes() const noexcept {
        return resident_bytes_ + chunk_bytes_.load(std::memory_order_relaxed);
    }
    [[nodiscard]] std::uint32_t max_rows() const noexcept { return max_rows_; }

    void release_pages(std::vector<std::int32_t>& pages);

private:
    explicit HipStepEngine(const HipPreparedModel& prepared) : prepared_(prepared) {}
    [[nodiscard]] Status allocate(void** ptr, std::uint64_t bytes, const char* what);
    // Adds chunks to a growing pool until `missing` more pages are free
    // (pool_mutex_ held): each chunk zeroed and its base written to the
    // device table on the engine's stream, ahead of the step that uses it.
    [[nodiscard]] Status grow_pool(std::uint64_t missing);
    [[nodiscard]] air_hip_kv_layout kv_layout(std::uint32_t table_pages) const noexcept;
    [[nodiscard]] Status layers(std::uint32_t m, std::uint64_t max_tokens, std::uint32_t table_pages,
                                QuantizedLinearExecutionKind tactic, std::uint32_t tiles);
    [[nodiscard]] Status attention(std::uint32_t layer, std::uint32_t m, std::uint64_t max_tokens,
                                   std::uint32_t table_pages, std::uint32_t tiles, bool rope_done = false);
    [[nodiscard]] Status project(std::uint32_t layer, LinearRole fused, LinearRole first, LinearRole second,
                                 LinearRole third, const float* x, float* y, std::uint32_t m,
                                 QuantizedLinearExecutionKind tactic);
    // Device work of a decode-shaped step over rows 0..m-1: the layers, the
    // lm_head over every row and the argmax into argmax_dev_.
    [[nodiscard]] Status decode_device(std::uint32_t m, std::uint64_t max_tokens, std::uint32_t table_pages,
                                       QuantizedLinearExecutionKind block, QuantizedLinearExecutionKind output,
                                       std::uint32_t tiles);
    // decode_device through a graph captured per (width, tactics): replayed
    // when one exists for the context's current buffers, else run eagerly and
    // captured for the next step.
    [[nodiscard]] Status decode_graph(std::uint32_t m, std::uint64_t max_tokens, std::uint32_t table_pages,
                                      QuantizedLinearExecutionKind block, QuantizedLinearExecutionKind output,
                                      std::uint32_t tiles);
    [[nodiscard]] std::uint64_t context_generation() const noexcept;
    [[nodiscard]] void* stream() const noexcept { return prepared_.options().stream; }

    struct DecodeGraph {
        void* exec{nullptr};          // hipGraphExec_t; null when capture failed (eager from then on)
        std::uint64_t generation{0};  // context buffers the launches point into
    };
    std::map<std::uint64_t, DecodeGraph> graphs_;
    const char* layer_range_{"air.prefill.layer"};   // ROCTX range name of the current step's layers

    const HipPreparedModel& prepared_;
    std::uint32_t page_tokens_{0}, pool_pages_{0}, max_rows_{0}, max_pages_{0}, output_rows_{0};
    std::uint64_t page_bytes_{0}, resident_bytes_{0};
    std::uint32_t embed_{0}, q_width_{0}, kv_width_{0}, qkv_width_{0}, ffn_{0}, head_dim_{0};
    std::uint64_t vocab_{0};
    std::vector<std::int32_t> free_pages_;
    mutable std::mutex pool_mutex_;
    std::vector<void*> allocations_;  // device buffers, released by the destructor

    // KV pool: one allocation (fixed) or chunks named by a device table.
    bool growable_{false};
    std::uint32_t chunk_shift_{0};
    std::vector<void*> chunks_;              // chunk bases in page-id order, freed by the destructor
    float** chunk_table_{nullptr};           // device: kMaxKvChunks bases, null where not allocated
    float** chunk_host_{nullptr};            // pinned host copy each table entry is uploaded from
    std::atomic<std::uint64_t> allocated_pages_{0}, chunk_bytes_{0};

    // device memory
    float* pool_{nullptr};
    float* rope_table_{nullptr};      // float2 {cos, sin} [context][rope_dims / 2]
    std::vector<float*> attn_norm_, ffn_norm_;
    float* output_norm_{nullptr};
    air_hip_matrix* embedding_{nullptr};   // token_embd, or the output matrix when they are tied
    bool owns_embedding_{false};
    float *hidden_{nullptr}, *normed_{nullptr}, *qkv_{nullptr}, *att_{nullptr}, *proj_{nullptr};
    float *gate_up_{nullptr}, *act_{nullptr}, *part_{nullptr}, *final_{nullptr}, *logits_{nullptr};
    std::int32_t *tokens_dev_{nullptr}, *positions_dev_{nullptr}, *tables_dev_{nullptr}, *argmax_dev_{nullptr};
    std::int32_t* tiles_dev_{nullptr};  // attention tiles of the online tactic (4 x uint32 each)
    std::uint32_t tile_capacity_{0};
    std::int32_t* staging_{nullptr};    // pinned host: tokens | positions | page tables | tiles | argmax
};

} // namespace air

// execution.hpp -- execution plans and backend capabilities.
//
// The plan/capability contract of AIR (include/air/execution.hpp:13-133,
// src/runtime/execution.cpp:1-126), re-stated with the HIP backend added:
// BackendKind::hip and the two HIP linear tactics
//   hip_decode  "hip-decode"   exact-code MFMA decode linear, M = 1..64
//   hip_prefill "hip-prefill"  f16 MFMA linear for prefill-sized M
// A plan names a tactic per operation scope (prefill block linears, decode
// block linears, the terminal vocabulary projection) and is valid only if
// the prepared backend advertises that tactic for that scope; there is no
// name-based fallback.
#pragma once

#include "air/status.hpp"

#include <cstdint>
#include <optional>
#include <string>
#include <string_view>
#include <vector>

namespace air {

enum class BackendKind {
    reference = 0,
    cuda,
    hip,
};

[[nodiscard]] const char* to_string(BackendKind backend) noexcept;
[[nodiscard]] Result<BackendKind> backend_kind_from_string(std::string_view value);

enum class PrefillExecutionKind {
    serial = 0,
    native_batch,
};
[[nodiscard]] const char* to_string(PrefillExecutionKind kind) noexcept;

enum class KvStorageKind {
    contiguous = 0,
    paged,
};
[[nodiscard]] const char* to_string(KvStorageKind kind) noexcept;

enum class QuantizedLinearExecutionKind {
    baseline = 0,
    batch_reuse4,
    batch_reuse8,
    q5q8_dp4a_hybrid,
    dense_f32_cublas,
    hip_decode,
    hip_prefill,
};
[[nodiscard]] const char* to_string(QuantizedLinearExecutionKind kind) noexcept;
[[nodiscard]] Result<QuantizedLinearExecutionKind> quantized_linear_execution_kind_from_string(
    std::string_view value);

enum class AttentionExecutionKind {
    baseline = 0,
    online_softmax,
};
[[nodiscard]] const char* to_string(AttentionExecutionKind kind) noexcept;
[[nodiscard]] Result<AttentionExecutionKind> attention_execution_kind_from_string(std::string_view value);

struct BackendCapabilities {
    BackendKind backend{BackendKind::reference};
    PrefillExecutionKind prefill_execution{PrefillExecutionKind::serial};
    KvStorageKind kv_storage{KvStorageKind::contiguous};
    std::uint32_t max_prefill_batch_width{1};
    std::uint32_t max_decode_batch_width{1};
    bool sequence_checkpointing{false};
    bool exact_prefix_reuse{false};
    bool device_greedy_selection{false};
    std::vector<QuantizedLinearExecutionKind> prefill_block_quantized_linear{QuantizedLinearExecutionKind::baseline};
    std::vector<QuantizedLinearExecutionKind> decode_block_quantized_linear{QuantizedLinearExecutionKind::baseline};
    std::vector<QuantizedLinearExecutionKind> decode_output_quantized_linear{QuantizedLinearExecutionKind::baseline};
    std::vector<AttentionExecutionKind> prefill_attention{AttentionExecutionKind::baseline};
    std::vector<AttentionExecutionKind> decode_attention{AttentionExecutionKind::baseline};
};

struct RequestProfile {
    std::uint64_t prompt_tokens{0};
    std::uint64_t max_output_tokens{0};
    std::uint32_t active_sequences{1};
};

struct SchedulingPolicy {
    std::uint32_t prefill_quantum_tokens{32};
};

struct KvPolicy {
    std::optional<std::uint32_t> page_tokens;
};

struct LinearPolicy {
    QuantizedLinearExecutionKind prefill_block{QuantizedLinearExecutionKind::baseline};
    QuantizedLinearExecutionKind decode_block{QuantizedLinearExecutionKind::baseline};
    QuantizedLinearExecutionKind decode_output{QuantizedLinearExecutionKind::baseline};
};

struct AttentionPolicy {
    AttentionExecutionKind prefill{AttentionExecutionKind::baseline};
    AttentionExecutionKind decode{AttentionExecutionKind::baseline};
};

struct ExecutionPlan {
    BackendKind backend{BackendKind::reference};
    std::string strategy_id{"static"};
    SchedulingPolicy scheduling{};
    KvPolicy kv{};
    LinearPolicy linear{};
    AttentionPolicy attention{};
};

[[nodiscard]] Status validate_execution_plan(const ExecutionPlan& plan, const BackendCapabilities& capabilities);

} // namespace air

// model.hpp -- the canonical, immutable model the HIP executor prepares.
//
// A lean restatement of AIR's ModelConfig / TensorDescriptor / ModelDefinition
// (include/air/model.hpp, include/air/tensor.hpp, src/model/model.cpp:50-80)
// keeping what the Qwen2 linear path reads: the geometry, the per-tensor GGML
// format id and shape (GGML order: dimensions[0] is K, the contiguous
// direction), and a byte view into shared storage.  The tokenizer and the
// fingerprint are outside this library.
#pragma once

#include "air/status.hpp"

#include <cstddef>
#include <cstdint>
#include <memory>
#include <span>
#include <string>
#include <unordered_map>
#include <vector>

namespace air {

using TokenId = std::int32_t;

// GGML type ids of the formats this library reads (gguf_format.cpp:24-63).
enum class GgmlType : std::uint32_t {
    f32 = 0,
    f16 = 1,
    q4_0 = 2,
    q5_0 = 6,
    q8_0 = 8,
    q4_k = 12,
    q6_k = 14,
    bf16 = 30,
};

struct FormatGeometry {
    std::uint64_t block_elements{0};
    std::uint64_t block_bytes{0};
};

// Block geometry per GGML type id; block_elements == 0 for unknown ids.
[[nodiscard]] FormatGeometry format_geometry(std::uint32_t format_type) noexcept;
[[nodiscard]] const char* format_name(std::uint32_t format_type) noexcept;

// Exact byte size of a row-major GGML tensor, or an error when the contiguous
// dimension is not a whole number of blocks (gguf_format.cpp:215-267).
[[nodiscard]] Result<std::uint64_t> exact_tensor_bytes(std::uint32_t format_type,
                                                       std::span<const std::uint64_t> dimensions);

struct ModelConfig {
    std::string architecture;
    std::uint32_t layer_count{0};
    std::uint32_t embedding_size{0};
    std::uint32_t feed_forward_size{0};
    std::uint32_t attention_head_count{0};
    std::uint32_t kv_head_count{0};
    std::uint64_t attention_sliding_window{0};
    std::uint32_t rope_dimension_count{0};
    std::uint64_t context_length{0};
    std::uint64_t vocabulary_size{0};
    double rope_frequency_base{0.0};
    std::string rope_scaling_type{"none"};
    double rope_scaling_factor{1.0};
    double rope_scale_linear{1.0};
    double rms_norm_epsilon{0.0};
};

struct TensorShape {
    std::vector<std::uint64_t> dimensions;
    [[nodiscard]] std::uint64_t element_count() const noexcept;
};

struct TensorDescriptor {
    std::string name;
    std::uint32_t format_type{0};
    TensorShape shape;
    std::uint64_t byte_offset{0};
    std::uint64_t byte_size{0};
};

// Backing bytes of a model: a GGUF mapping or an in-memory image.
class ModelStorage {
public:
    virtual ~ModelStorage() = default;
    [[nodiscard]] virtual std::span<const std::byte> bytes() const noexcept = 0;
};

// In-memory storage (synthetic models, tests).
class BufferStorage final : public ModelStorage {
public:
    explicit BufferStorage(std::vector<std::byte> data) : data_(std::move(data)) {}
    [[nodiscard]] std::span<const std::byte> bytes() const noexcept override { return data_; }

private:
    std::vector<std::byte> data_;
};

class ModelDefinition {
public:
    ModelDefinition() = default;
    ModelDefinition(ModelConfig config, std::vector<TensorDescriptor> tensors,
                    std::shared_ptr<const ModelStorage> storage);

    [[nodiscard]] const ModelConfig& config() const noexcept { return config_; }
    [[nodiscard]] const std::vector<TensorDescriptor>& tensors() const noexcept { return tensors_; }
    [[nodiscard]] const std::shared_ptr<const ModelStorage>& storage() const noexcept { return storage_; }
    [[nodiscard]] const TensorDescriptor* find_tensor(const std::string& name) const noexcept;
    // Geometry, unique names, exact byte sizes and storage bounds.
    [[nodiscard]] Status validate() const;
    [[nodiscard]] Result<std::span<const std::byte>> tensor_bytes(const TensorDescriptor& tensor) const;

private:
    ModelConfig config_;
    std::vector<TensorDescriptor> tensors_;
    std::unordered_map<std::string, std::size_t> index_;
    std::shared_ptr<const ModelStorage> storage_;
};

// "blk.<layer>.<suffix>" (qwen2_contract.cpp:10-12).
[[nodiscard]] std::string block_tensor_name(std::uint32_t layer, const char* suffix);

// Qwen2 structural contract (qwen2_contract.cpp:33-117): geometry, RoPE and
// window restrictions, and the shape of every required/optional tensor.
[[nodiscard]] Status validate_qwen2_structure(const ModelDefinition& model);

} // namespace air

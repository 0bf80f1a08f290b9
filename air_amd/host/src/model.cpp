// model.cpp -- ModelDefinition checks and the Qwen2 structural contract.
//
// validate() keeps the tensor checks of src/model/model.cpp:90-166 (names,
// shapes, sizes, storage bounds) and the geometry checks; the exact byte size
// of a tensor follows gguf_format.cpp:245-256 (whole blocks of the element
// count).  validate_qwen2_structure restates qwen2_contract.cpp:33-117 with
// the same order of checks and the same messages.
#include "air/model.hpp"

#include <cmath>
#include <limits>
#include <unordered_set>

namespace air {

FormatGeometry format_geometry(std::uint32_t format_type) noexcept {
    switch (static_cast<GgmlType>(format_type)) {
    case GgmlType::f32: return {1, 4};
    case GgmlType::f16: return {1, 2};
    case GgmlType::bf16: return {1, 2};
    case GgmlType::q4_0: return {32, 18};
    case GgmlType::q5_0: return {32, 22};
    case GgmlType::q8_0: return {32, 34};
    case GgmlType::q4_k: return {256, 144};
    case GgmlType::q6_k: return {256, 210};
    }
    return {0, 0};
}

const char* format_name(std::uint32_t format_type) noexcept {
    switch (static_cast<GgmlType>(format_type)) {
    case GgmlType::f32: return "f32";
    case GgmlType::f16: return "f16";
    case GgmlType::bf16: return "bf16";
    case GgmlType::q4_0: return "q4_0";
    case GgmlType::q5_0: return "q5_0";
    case GgmlType::q8_0: return "q8_0";
    case GgmlType::q4_k: return "q4_K";
    case GgmlType::q6_k: return "q6_K";
    }
    return "unknown";
}

std::uint64_t TensorShape::element_count() const noexcept {
    if (dimensions.empty()) return 0;
    std::uint64_t count = 1;
    for (const auto d : dimensions) {
        if (d == 0 || count > std::numeric_limits<std::uint64_t>::max() / d) return 0;
        count *= d;
    }
    return count;
}

Result<std::uint64_t> exact_tensor_bytes(std::uint32_t format_type, std::span<const std::uint64_t> dimensions) {
    const auto geometry = format_geometry(format_type);
    if (geometry.block_elements == 0) {
        return Status::unsupported(std::string("unsupported tensor format id ") + std::to_string(format_type));
    }
    TensorShape shape{{dimensions.begin(), dimensions.end()}};
    const auto elements = shape.element_count();
    if (elements == 0) return Status::invalid_argument("tensor has invalid shape");
    if (dimensions[0] % geometry.block_elements != 0) {
        return Status::data_error("tensor contiguous dimension is not a whole number of blocks");
    }
    const auto blocks = elements / geometry.block_elements;
    if (blocks > std::numeric_limits<std::uint64_t>::max() / geometry.block_bytes) {
        return Status::data_error("tensor byte size overflows");
    }
    return blocks * geometry.block_bytes;
}

ModelDefinition::ModelDefinition(ModelConfig config, std::vector<TensorDescriptor> tensors,
                                 std::shared_ptr<const ModelStorage> storage)
    : config_(std::move(config)), tensors_(std::move(tensors)), storage_(std::move(storage)) {
    index_.reserve(tensors_.size());
    for (std::size_t i = 0; i < tensors_.size(); ++i) index_.emplace(tensors_[i].name, i);
}

const TensorDescriptor* ModelDefinition::find_tensor(const std::string& name) const noexcept {
    const auto it = index_.find(name);
    return it == index_.end() ? nullptr : &tensors_[it->second];
}

Status ModelDefinition::validate() const {
    if (config_.architecture.empty()) return Status::invalid_argument("model architecture is empty");
    if (config_.layer_count == 0) return Status::invalid_argument("layer count must be greater than zero");
    if (config_.embedding_size == 0) return Status::invalid_argument("embedding size must be greater than zero");
    if (config_.attention_head_count == 0) {
        return Status::invalid_argument("attention head count must be greater than zero");
    }
    if (config_.kv_head_count == 0 || config_.kv_head_count > config_.attention_head_count) {
        return Status::invalid_argument("KV head count must be in [1, attention_head_count]");
    }
    if (config_.context_length == 0) return Status::invalid_argument("context length must be greater than zero");
    if (config_.vocabulary_size == 0) return Status::invalid_argument("vocabulary size must be greater than zero");

    std::unordered_set<std::string> names;
    names.reserve(tensors_.size());
    const auto storage_bytes = storage_ ? storage_->bytes().size() : 0U;
    for (const auto& tensor : tensors_) {
        if (tensor.name.empty()) return Status::invalid_argument("tensor name is empty");
        if (!names.emplace(tensor.name).second) {
            return Status::invalid_argument("duplicate tensor name: " + tensor.name);
        }
        if (tensor.shape.element_count() == 0) {
            return Status::invalid_argument("tensor has invalid shape: " + tensor.name);
        }
        if (tensor.byte_size == 0) return Status::invalid_argument("tensor has zero storage size: " + tensor.name);
        const auto exact = exact_tensor_bytes(tensor.format_type, tensor.shape.dimensions);
        if (exact && exact.value() != tensor.byte_size) {
            return Status::data_error("tensor byte size does not match its format: " + tensor.name);
        }
        if (storage_ && (tensor.byte_offset > storage_bytes || tensor.byte_size > storage_bytes - tensor.byte_offset)) {
            return Status::data_error("tensor storage range is outside mapped model: " + tensor.name);
        }
    }
    return Status::ok();
}

Result<std::span<const std::byte>> ModelDefinition::tensor_bytes(const TensorDescriptor& tensor) const {
    if (!storage_) return Status::invalid_state("model has no backing storage");
    const auto bytes = storage_->bytes();
    if (tensor.byte_offset > bytes.size() || tensor.byte_size > bytes.size() - tensor.byte_offset) {
        return Status::data_error("tensor storage range is outside mapped model: " + tensor.name);
    }
    return bytes.subspan(tensor.byte_offset, tensor.byte_size);
}

std::string block_tensor_name(std::uint32_t layer, const char* suffix) {
    return "blk." + std::to_string(layer) + "." + suffix;
}

namespace {

Status require_shape(const ModelDefinition& model, const std::string& name,
                     std::initializer_list<std::uint64_t> dimensions, bool optional = false) {
    const auto* tensor = model.find_tensor(name);
    if (!tensor) return optional ? Status::ok() : Status::data_error("missing required Qwen2 tensor: " + name);
    if (tensor->shape.dimensions.size() != dimensions.size()) {
        return Status::data_error("rank mismatch for tensor: " + name);
    }
    std::size_t i = 0;
    for (const auto d : dimensions) {
        if (tensor->shape.dimensions[i++] != d) return Status::data_error("shape mismatch for tensor: " + name);
    }
    return Status::ok();
}

} // namespace

Status validate_qwen2_structure(const ModelDefinition& model) {
    const auto& c = model.config();
    if (c.architecture != "qwen2") return Status::unsupported("AIR Qwen2 execution supports only qwen2 architecture");
    if (c.layer_count == 0U || c.embedding_size == 0U || c.attention_head_count == 0U || c.kv_head_count == 0U ||
        c.context_length == 0U || c.vocabulary_size == 0U) {
        return Status::data_error("Qwen2 model geometry is incomplete");
    }
    if (c.embedding_size % c.attention_head_count != 0U) {
        return Status::data_error("Qwen2 embedding size is not divisible by attention head count");
    }
    if (c.attention_head_count % c.kv_head_count != 0U) {
        return Status::data_error("Qwen2 attention head count must be divisible by KV head count");
    }
    const std::uint64_t e = c.embedding_size;
    const std::uint64_t head = c.embedding_size / c.attention_head_count;
    const std::uint64_t qw = c.attention_head_count * head;
    const std::uint64_t kvw = c.kv_head_count * head;
    const std::uint64_t ffn = c.feed_forward_size;
    const std::uint64_t vocab = c.vocabulary_size;
    if (ffn == 0U) return Status::data_error("Qwen2 feed-forward size is missing");
    if (!(c.rms_norm_epsilon > 0.0)) return Status::data_error("Qwen2 RMS norm epsilon is missing or invalid");
    if (!(c.rope_frequency_base > 0.0)) return Status::data_error("Qwen2 RoPE base is missing or invalid");
    if (!c.rope_scaling_type.empty() && c.rope_scaling_type != "none") {
        return Status::unsupported("AIR Qwen2 execution does not implement RoPE scaling type: " + c.rope_scaling_type);
    }
    if (std::fabs(c.rope_scaling_factor - 1.0) > 1.0e-12 || std::fabs(c.rope_scale_linear - 1.0) > 1.0e-12) {
        return Status::unsupported("AIR Qwen2 execution does not implement scaled RoPE");
    }
    if (c.attention_sliding_window != 0U) {
        return Status::unsupported("AIR Qwen2 execution does not implement sliding-window attention");
    }
    if (c.rope_dimension_count != head || c.rope_dimension_count % 2U != 0U) {
        return Status::unsupported("AIR Qwen2 execution requires full, even head-dimension RoPE");
    }

    Status s = require_shape(model, "token_embd.weight", {e, vocab});
    if (!s) return s;
    if (!(s = require_shape(model, "output_norm.weight", {e}))) return s;
    if (model.find_tensor("output.weight") && !(s = require_shape(model, "output.weight", {e, vocab}))) return s;
    if (!(s = require_shape(model, "output.bias", {vocab}, true))) return s;
    for (std::uint32_t layer = 0; layer < c.layer_count; ++layer) {
        const auto n = [layer](const char* suffix) { return block_tensor_name(layer, suffix); };
        if (!(s = require_shape(model, n("attn_norm.weight"), {e}))) return s;
        if (!(s = require_shape(model, n("attn_q.weight"), {e, qw}))) return s;
        if (!(s = require_shape(model, n("attn_k.weight"), {e, kvw}))) return s;
        if (!(s = require_shape(model, n("attn_v.weight"), {e, kvw}))) return s;
        if (!(s = require_shape(model, n("attn_q.bias"), {qw}, true))) return s;
        if (!(s = require_shape(model, n("attn_k.bias"), {kvw}, true))) return s;
        if (!(s = require_shape(model, n("attn_v.bias"), {kvw}, true))) return s;
        if (!(s = require_shape(model, n("attn_output.weight"), {qw, e}))) return s;
        if (!(s = require_shape(model, n("ffn_norm.weight"), {e}))) return s;
        if (!(s = require_shape(model, n("ffn_gate.weight"), {e, ffn}))) return s;
        if (!(s = require_shape(model, n("ffn_up.weight"), {e, ffn}))) return s;
        if (!(s = require_shape(model, n("ffn_down.weight"), {ffn, e}))) return s;
    }
    return Status::ok();
}

} // namespace air

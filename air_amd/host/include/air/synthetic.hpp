// synthetic.hpp -- seeded random-init Qwen2 models in GGUF block formats.
//
// The benchmark configurations are random-init models (no checkpoints are
// available offline): weights ~N(0, sigma) quantized per GGUF block, q/k/v
// and output biases ~N(0, sigma) f32, norm weights 1.0 f32.  Each tensor has
// its own seed derived from (seed, tensor name), so a model is reproducible
// tensor by tensor.  Quantizers:
//   Q8_0  d = max|w| / 127 (f16), q = round-half-away(w / d)
//   Q4_0  d = (signed max-abs value) / -8 (f16), n = clamp(floor(w/d + 8.5), 0, 15)
//   Q4_K  8 sub-blocks of 32: step (max - min) / 15, 6-bit scales/mins
//         against f16 d = max step / 63 and dmin = max(-min) / 63
#pragma once

#include "air/model.hpp"

#include <cstdint>
#include <memory>
#include <span>
#include <vector>

namespace air {

// IEEE binary16 <-> binary32, round to nearest even (subnormals, inf, NaN kept).
[[nodiscard]] std::uint16_t f32_to_f16_bits(float value) noexcept;
[[nodiscard]] float f16_bits_to_f32(std::uint16_t bits) noexcept;

// Row-major f32 [n x k] -> GGUF bytes of `format_type` (k a multiple of the block).
[[nodiscard]] Result<std::vector<std::byte>> quantize_rows(std::uint32_t format_type, std::span<const float> w,
                                                           std::uint64_t k, std::uint64_t n);

// Deterministic N(0, sigma) values from a 64-bit seed: out[j] is value
// first + j of the seed's stream (first must be even), so chunks filled
// independently equal one sequential fill.
void normal_fill(std::span<float> out, std::uint64_t seed, float sigma, std::uint64_t first = 0);
[[nodiscard]] std::uint64_t tensor_seed(std::uint64_t seed, const std::string& name) noexcept;

struct SyntheticQwen2Spec {
    ModelConfig config{};
    std::uint32_t weight_format{static_cast<std::uint32_t>(GgmlType::q8_0)};
    std::uint32_t embedding_format{static_cast<std::uint32_t>(GgmlType::q8_0)};
    // attn_v / ffn_down and output.weight formats (kSameFormat: weight_format),
    // e.g. Q6_K beside Q4_K as in a Q4_K_M file.
    static constexpr std::uint32_t kSameFormat = 0xFFFFFFFFU;
    std::uint32_t v_down_format{kSameFormat};
    std::uint32_t output_format{kSameFormat};
    std::uint64_t seed{0xA17C0DEULL};
    float sigma{0.02f};
    bool qkv_bias{true};
    bool output_bias{false};
    bool tied_output{false};  // no output.weight: lm_head reads token_embd.weight
};

// Qwen2 configuration of the given geometry with the family's fixed values
// (RoPE theta 1e6, RMSNorm eps 1e-6, full-head RoPE, no window).
[[nodiscard]] ModelConfig qwen2_config(std::uint32_t layers, std::uint32_t embedding, std::uint32_t ffn,
                                       std::uint32_t heads, std::uint32_t kv_heads, std::uint64_t vocab,
                                       std::uint64_t context = 4096);

[[nodiscard]] Result<std::shared_ptr<const ModelDefinition>> make_synthetic_qwen2(const SyntheticQwen2Spec& spec);

} // namespace air

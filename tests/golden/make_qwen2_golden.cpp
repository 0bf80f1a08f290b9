// make_qwen2_golden.cpp -- golden greedy tokens and logits of AIR's own
// ReferenceExecutor on small synthetic Qwen2 models.
//
// Test-fixture generator: builds each model with air::make_synthetic_qwen2
// (deterministic, so the tests rebuild the identical bytes anywhere), runs it
// through the reference executor compiled from the reference sources
// (oracle/_ref/libairref.so: ReferenceExecutor::step, src/reference/
// reference_executor.cpp:325-428) one token at a time -- the prompt, then
// greedy continuation with Sampler's first-maximum rule
// (src/runtime/sampling.cpp:13-16) -- and writes every step's logits as f32
// bit patterns.  Run by tests/golden/Makefile; the output is committed.
#include "air/synthetic.hpp"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

extern "C" {
struct airref_qwen2_config {
    std::uint32_t layers, embedding, ffn, heads, kv_heads, rope_dims;
    std::uint64_t context, vocab;
    double rope_base, eps;
};
struct airref_qwen2;
int airref_qwen2_create(const airref_qwen2_config* cfg, std::uint32_t count, const char* const* names,
                        const int* types, const std::uint32_t* ranks, const std::uint64_t* dims,
                        const std::uint64_t* offsets, const std::uint64_t* sizes, const std::uint8_t* blob,
                        std::uint64_t blob_bytes, airref_qwen2** out);
int airref_qwen2_step(airref_qwen2* q, std::int32_t token, float* logits);
int airref_qwen2_reset(airref_qwen2* q);
void airref_qwen2_destroy(airref_qwen2* q);
}

namespace {

struct Case {
    const char* name;
    std::uint32_t weight_format, embedding_format;
    bool qkv_bias, output_bias, tied;
    std::uint64_t seed;
    std::vector<std::vector<std::int32_t>> prompts;
    std::uint32_t generate;
};

std::uint64_t greedy(const std::vector<float>& logits) {
    std::uint64_t best = 0;
    for (std::uint64_t i = 1; i < logits.size(); ++i)
        if (logits[best] < logits[i]) best = i;
    return best;
}

int run_case(const Case& c, std::FILE* out) {
    air::SyntheticQwen2Spec spec;
    spec.config = air::qwen2_config(2, 256, 512, 4, 2, 512, 64);
    spec.weight_format = c.weight_format;
    spec.embedding_format = c.embedding_format;
    spec.qkv_bias = c.qkv_bias;
    spec.output_bias = c.output_bias;
    spec.tied_output = c.tied;
    spec.seed = c.seed;
    auto built = air::make_synthetic_qwen2(spec);
    if (!built) {
        std::fprintf(stderr, "%s: %s\n", c.name, built.status().message().c_str());
        return 1;
    }
    const auto& model = *built.value();
    std::vector<const char*> names;
    std::vector<int> types;
    std::vector<std::uint32_t> ranks;
    std::vector<std::uint64_t> dims, offsets, sizes;
    for (const auto& t : model.tensors()) {
        names.push_back(t.name.c_str());
        types.push_back(static_cast<int>(t.format_type));
        ranks.push_back(static_cast<std::uint32_t>(t.shape.dimensions.size()));
        dims.push_back(t.shape.dimensions[0]);
        dims.push_back(t.shape.dimensions.size() > 1 ? t.shape.dimensions[1] : 0u);
        offsets.push_back(t.byte_offset);
        sizes.push_back(t.byte_size);
    }
    const auto& cfg = model.config();
    airref_qwen2_config rc{cfg.layer_count, cfg.embedding_size, cfg.feed_forward_size, cfg.attention_head_count,
                           cfg.kv_head_count, cfg.rope_dimension_count, cfg.context_length, cfg.vocabulary_size,
                           cfg.rope_frequency_base, cfg.rms_norm_epsilon};
    const auto blob = model.storage()->bytes();
    airref_qwen2* ref = nullptr;
    const int status = airref_qwen2_create(&rc, static_cast<std::uint32_t>(names.size()), names.data(), types.data(),
                                           ranks.data(), dims.data(), offsets.data(), sizes.data(),
                                           reinterpret_cast<const std::uint8_t*>(blob.data()), blob.size(), &ref);
    if (status != 0) {
        std::fprintf(stderr, "%s: reference refused the model (%d)\n", c.name, status);
        return 1;
    }
    std::fprintf(out, "case %s\n", c.name);
    std::fprintf(out, "config %u %u %u %u %u %llu %llu\n", cfg.layer_count, cfg.embedding_size, cfg.feed_forward_size,
                 cfg.attention_head_count, cfg.kv_head_count, static_cast<unsigned long long>(cfg.vocabulary_size),
                 static_cast<unsigned long long>(cfg.context_length));
    std::fprintf(out, "weights %u %u %llu %d %d %d\n", c.weight_format, c.embedding_format,
                 static_cast<unsigned long long>(c.seed), c.qkv_bias ? 1 : 0, c.output_bias ? 1 : 0, c.tied ? 1 : 0);
    std::vector<float> logits(cfg.vocabulary_size);
    for (const auto& prompt : c.prompts) {
        if (airref_qwen2_reset(ref) != 0) return 1;
        std::fprintf(out, "sequence %zu", prompt.size());
        for (const auto t : prompt) std::fprintf(out, " %d", t);
        std::fprintf(out, "\n");
        std::vector<std::int32_t> generated;
        std::vector<std::vector<float>> steps;
        for (const auto t : prompt) {
            if (airref_qwen2_step(ref, t, logits.data()) != 0) return 1;
            steps.push_back(logits);
        }
        for (std::uint32_t g = 0; g < c.generate; ++g) {
            const auto next = static_cast<std::int32_t>(greedy(steps.back()));
            generated.push_back(next);
            if (g + 1 == c.generate) break;
            if (airref_qwen2_step(ref, next, logits.data()) != 0) return 1;
            steps.push_back(logits);
        }
        std::fprintf(out, "generated %zu", generated.size());
        for (const auto t : generated) std::fprintf(out, " %d", t);
        std::fprintf(out, "\n");
        for (std::size_t s = 0; s < steps.size(); ++s) {
            std::fprintf(out, "logits %zu", s);
            for (const float v : steps[s]) {
                std::uint32_t bits;
                std::memcpy(&bits, &v, sizeof(bits));
                std::fprintf(out, " %08x", bits);
            }
            std::fprintf(out, "\n");
        }
    }
    std::fprintf(out, "end\n");
    airref_qwen2_destroy(ref);
    return 0;
}

} // namespace

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: make_qwen2_golden <out.txt>\n");
        return 2;
    }
    std::FILE* out = std::fopen(argv[1], "w");
    if (!out) return 2;
    std::fprintf(out, "# Qwen2 greedy goldens from AIR's ReferenceExecutor (make_qwen2_golden.cpp)\n");
    const std::vector<Case> cases = {
        {"q8_0", 8u, 8u, true, false, false, 0xA174D1FFULL, {{1, 17, 200, 3, 511}, {42, 42, 7}}, 6},
        {"q4_0_tied", 2u, 2u, true, true, true, 0xA174D200ULL, {{5, 300, 9, 77}, {0}}, 6},
        {"q4_k", 12u, 8u, false, false, false, 0xA174D201ULL, {{128, 64, 32, 16, 8, 4}}, 6},
    };
    for (const auto& c : cases) {
        if (run_case(c, out) != 0) return 1;
    }
    std::fclose(out);
    return 0;
}

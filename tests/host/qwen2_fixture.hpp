// qwen2_fixture.hpp -- reads tests/golden/qwen2_tiny.txt (written by
// tests/golden/make_qwen2_golden.cpp from AIR's ReferenceExecutor) and
// rebuilds each case's synthetic model.
#pragma once

#include "air/synthetic.hpp"
#include "air_oracle_qwen2.h"

#include <cstdint>
#include <cstring>
#include <fstream>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

namespace fixture {

struct Sequence {
    std::vector<std::int32_t> prompt;
    std::vector<std::int32_t> generated;
    std::vector<std::vector<float>> logits;  // one per step: prompt, then generated[0..n-2]
};

struct Case {
    std::string name;
    air::SyntheticQwen2Spec spec;
    std::vector<Sequence> sequences;
};

inline std::vector<Case> load(const std::string& path) {
    std::vector<Case> cases;
    std::ifstream in(path);
    std::string line;
    while (std::getline(in, line)) {
        if (line.empty() || line[0] == '#') continue;
        std::istringstream ss(line);
        std::string tag;
        ss >> tag;
        if (tag == "case") {
            cases.emplace_back();
            ss >> cases.back().name;
        } else if (tag == "config") {
            std::uint32_t layers, e, ffn, heads, kv;
            std::uint64_t vocab, ctx;
            ss >> layers >> e >> ffn >> heads >> kv >> vocab >> ctx;
            cases.back().spec.config = air::qwen2_config(layers, e, ffn, heads, kv, vocab, ctx);
        } else if (tag == "weights") {
            std::uint64_t seed;
            int qkv_bias, out_bias, tied;
            auto& s = cases.back().spec;
            ss >> s.weight_format >> s.embedding_format >> seed >> qkv_bias >> out_bias >> tied;
            s.seed = seed;
            s.qkv_bias = qkv_bias != 0;
            s.output_bias = out_bias != 0;
            s.tied_output = tied != 0;
        } else if (tag == "sequence") {
            std::size_t n;
            ss >> n;
            Sequence seq;
            seq.prompt.resize(n);
            for (auto& t : seq.prompt) ss >> t;
            cases.back().sequences.push_back(std::move(seq));
        } else if (tag == "generated") {
            std::size_t n;
            ss >> n;
            auto& g = cases.back().sequences.back().generated;
            g.resize(n);
            for (auto& t : g) ss >> t;
        } else if (tag == "logits") {
            std::size_t step;
            ss >> step;
            std::vector<float> v;
            std::string hex;
            while (ss >> hex) {
                const std::uint32_t bits = static_cast<std::uint32_t>(std::stoul(hex, nullptr, 16));
                float f;
                std::memcpy(&f, &bits, sizeof(f));
                v.push_back(f);
            }
            cases.back().sequences.back().logits.push_back(std::move(v));
        }
    }
    return cases;
}

// Oracle view of a built model (pointers into the model's storage).
struct OracleModel {
    std::vector<oracle_qwen2_layer> layers;
    oracle_qwen2_model model{};
};

inline oracle_tensor tensor_of(const air::ModelDefinition& m, const std::string& name) {
    oracle_tensor t{};
    const auto* d = m.find_tensor(name);
    if (!d) return t;
    const auto bytes = m.tensor_bytes(*d).value();
    t.type = static_cast<int>(d->format_type);
    t.bytes = reinterpret_cast<const std::uint8_t*>(bytes.data());
    t.nbytes = bytes.size();
    t.rank = static_cast<std::uint32_t>(d->shape.dimensions.size());
    t.dims[0] = d->shape.dimensions[0];
    t.dims[1] = t.rank > 1 ? d->shape.dimensions[1] : 1u;
    return t;
}

inline std::unique_ptr<OracleModel> oracle_view(const air::ModelDefinition& m) {
    auto o = std::make_unique<OracleModel>();
    const auto& c = m.config();
    for (std::uint32_t l = 0; l < c.layer_count; ++l) {
        const auto n = [l](const char* s) { return air::block_tensor_name(l, s); };
        oracle_qwen2_layer L{};
        L.attn_norm = tensor_of(m, n("attn_norm.weight"));
        L.q = tensor_of(m, n("attn_q.weight"));
        L.k = tensor_of(m, n("attn_k.weight"));
        L.v = tensor_of(m, n("attn_v.weight"));
        L.q_bias = tensor_of(m, n("attn_q.bias"));
        L.k_bias = tensor_of(m, n("attn_k.bias"));
        L.v_bias = tensor_of(m, n("attn_v.bias"));
        L.o = tensor_of(m, n("attn_output.weight"));
        L.ffn_norm = tensor_of(m, n("ffn_norm.weight"));
        L.gate = tensor_of(m, n("ffn_gate.weight"));
        L.up = tensor_of(m, n("ffn_up.weight"));
        L.down = tensor_of(m, n("ffn_down.weight"));
        o->layers.push_back(L);
    }
    auto& om = o->model;
    om.layers = c.layer_count;
    om.embedding = c.embedding_size;
    om.ffn = c.feed_forward_size;
    om.heads = c.attention_head_count;
    om.kv_heads = c.kv_head_count;
    om.rope_dims = c.rope_dimension_count;
    om.context = c.context_length;
    om.vocab = c.vocabulary_size;
    om.rope_base = c.rope_frequency_base;
    om.eps = c.rms_norm_epsilon;
    om.token_embd = tensor_of(m, "token_embd.weight");
    om.output_norm = tensor_of(m, "output_norm.weight");
    om.output = tensor_of(m, "output.weight");
    om.output_bias = tensor_of(m, "output.bias");
    om.layer = o->layers.data();
    return o;
}

}  // namespace fixture

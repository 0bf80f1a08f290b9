// ref_shim.cpp -- C entry points over AIR's own reference CPU executor.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's unmodified sources where they lie under /root/reference
// (tensor_reader.cpp, model.cpp, storage.cpp, ...) into oracle/_ref/.  It lets
// the tests check the plain-C oracle against the real reference on the same
// bytes, and lets bench.py time the real reference matvec as the CPU baseline.
// Nothing in the product links it.
//
// The model is assembled the way the reference's own tests do it
// (tests/reference_tests.cpp:34-86): raw tensor bytes go to a temporary file,
// ModelStorage::map_read_only maps it, and ModelDefinition wraps the
// descriptors.

#include "air/format.hpp"
#include "air/model.hpp"
#include "air/reference.hpp"
#include "air/storage.hpp"

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <memory>
#include <string>
#include <unistd.h>
#include <vector>

namespace {

bool data_type_for(int ggml, air::DataType& out) {
    switch (ggml) {
    case 0: out = air::DataType::f32; return true;
    case 1: out = air::DataType::f16; return true;
    case 2: out = air::DataType::q4_0; return true;
    case 6: out = air::DataType::q5_0; return true;
    case 8: out = air::DataType::q8_0; return true;
    case 12: out = air::DataType::q4_k; return true;
    case 14: out = air::DataType::q6_k; return true;
    case 30: out = air::DataType::bf16; return true;
    default: return false;
    }
}

int code_of(const air::Status& s) { return static_cast<int>(s.code()); }

// Builds a one-tensor ModelDefinition over a temporary mapped file.
std::shared_ptr<const air::ModelDefinition> one_tensor_model(
    const char* name, air::DataType type, int ggml, std::vector<std::uint64_t> dims,
    const std::uint8_t* bytes, std::uint64_t nbytes, int& rc) {
    char path[] = "/tmp/airref-XXXXXX";
    const int fd = mkstemp(path);
    if (fd < 0) { rc = 3; return {}; }
    std::uint64_t written = 0;
    while (written < nbytes) {
        const auto n = ::write(fd, bytes + written, nbytes - written);
        if (n <= 0) { ::close(fd); std::filesystem::remove(path); rc = 3; return {}; }
        written += static_cast<std::uint64_t>(n);
    }
    ::close(fd);
    auto storage = air::ModelStorage::map_read_only(path);
    std::filesystem::remove(path);
    if (!storage) { rc = code_of(storage.status()); return {}; }

    air::TensorDescriptor t;
    t.name = name;
    t.type = type;
    t.format_type = static_cast<std::uint32_t>(ggml);
    t.shape.dimensions = std::move(dims);
    t.byte_offset = 0;
    t.byte_size = nbytes;
    t.byte_size_exact = true;
    air::ModelConfig config;
    config.architecture = "oracle-fixture";
    air::TokenizerDefinition tokenizer;
    std::vector<air::TensorDescriptor> tensors;
    tensors.push_back(std::move(t));
    rc = 0;
    return std::make_shared<air::ModelDefinition>(
        air::ModelFingerprint{"test", config.architecture, "oracle"}, std::move(config),
        std::move(tokenizer), std::move(tensors), std::move(storage).value());
}

} // namespace

extern "C" {

// ReferenceTensorReader::vector over a rank-1 tensor of `elements` values.
int airref_decode(int ggml_type, const std::uint8_t* bytes, std::uint64_t nbytes,
                  std::uint64_t elements, float* out) {
    air::DataType type{};
    if (!data_type_for(ggml_type, type)) return 6;
    int rc = 0;
    auto model = one_tensor_model("t", type, ggml_type, {elements}, bytes, nbytes, rc);
    if (!model) return rc;
    air::ReferenceTensorReader reader(model);
    auto decoded = reader.vector("t");
    if (!decoded) return code_of(decoded.status());
    if (decoded.value().size() != elements) return 5;
    std::memcpy(out, decoded.value().data(), elements * sizeof(float));
    return 0;
}

// ReferenceTensorReader::matvec over a GGML matrix with dims {K, N}, applied to
// each of M input rows.
int airref_matvec(int ggml_type, const std::uint8_t* bytes, std::uint64_t nbytes,
                  std::uint64_t K, std::uint64_t N, std::uint32_t M,
                  const float* x, float* y) {
    air::DataType type{};
    if (!data_type_for(ggml_type, type)) return 6;
    int rc = 0;
    auto model = one_tensor_model("w", type, ggml_type, {K, N}, bytes, nbytes, rc);
    if (!model) return rc;
    air::ReferenceTensorReader reader(model);
    for (std::uint32_t m = 0; m < M; ++m) {
        auto out = reader.matvec("w", std::span<const float>(x + static_cast<std::uint64_t>(m) * K, K));
        if (!out) return code_of(out.status());
        std::memcpy(y + static_cast<std::uint64_t>(m) * N, out.value().data(), N * sizeof(float));
    }
    return 0;
}

// A persistent one-matrix model, so that timing loops measure only
// ReferenceTensorReader::matvec and not the model assembly.
struct airref_model {
    std::shared_ptr<const air::ModelDefinition> model;
    std::uint64_t k{0}, n{0};
};

int airref_model_create(int ggml_type, const std::uint8_t* bytes, std::uint64_t nbytes,
                        std::uint64_t K, std::uint64_t N, airref_model** out) {
    air::DataType type{};
    if (!out) return 1;
    *out = nullptr;
    if (!data_type_for(ggml_type, type)) return 6;
    int rc = 0;
    auto model = one_tensor_model("w", type, ggml_type, {K, N}, bytes, nbytes, rc);
    if (!model) return rc;
    *out = new airref_model{std::move(model), K, N};
    return 0;
}

int airref_model_matvec(const airref_model* m, const float* x, float* y) {
    if (!m) return 1;
    air::ReferenceTensorReader reader(m->model);
    auto out = reader.matvec("w", std::span<const float>(x, m->k));
    if (!out) return code_of(out.status());
    std::memcpy(y, out.value().data(), m->n * sizeof(float));
    return 0;
}

void airref_model_destroy(airref_model* m) { delete m; }

// ---- a whole Qwen2 model through ReferenceExecutor -----------------------

struct airref_qwen2_config {
    std::uint32_t layers, embedding, ffn, heads, kv_heads, rope_dims;
    std::uint64_t context, vocab;
    double rope_base, eps;
};

struct airref_qwen2 {
    std::unique_ptr<air::ReferenceExecutor> executor;
    std::unique_ptr<air::ReferenceKvCache> cache;
    airref_qwen2_config config{};
};

// Tensors are `count` entries of one blob (offsets/sizes in bytes, dims
// [count][2] in GGML order, rank 1 or 2).  The blob goes to a temporary
// mapped file, as the reference's tests assemble models.
int airref_qwen2_create(const airref_qwen2_config* cfg, std::uint32_t count, const char* const* names,
                        const int* types, const std::uint32_t* ranks, const std::uint64_t* dims,
                        const std::uint64_t* offsets, const std::uint64_t* sizes, const std::uint8_t* blob,
                        std::uint64_t blob_bytes, airref_qwen2** out) {
    if (!cfg || !out) return 1;
    *out = nullptr;
    char path[] = "/tmp/airref-qwen2-XXXXXX";
    const int fd = mkstemp(path);
    if (fd < 0) return 3;
    std::uint64_t written = 0;
    while (written < blob_bytes) {
        const auto n = ::write(fd, blob + written, blob_bytes - written);
        if (n <= 0) { ::close(fd); std::filesystem::remove(path); return 3; }
        written += static_cast<std::uint64_t>(n);
    }
    ::close(fd);
    auto storage = air::ModelStorage::map_read_only(path);
    std::filesystem::remove(path);
    if (!storage) return code_of(storage.status());

    std::vector<air::TensorDescriptor> tensors;
    for (std::uint32_t i = 0; i < count; ++i) {
        air::TensorDescriptor t;
        t.name = names[i];
        if (!data_type_for(types[i], t.type)) return 6;
        t.format_type = static_cast<std::uint32_t>(types[i]);
        t.shape.dimensions.assign(dims + 2u * i, dims + 2u * i + ranks[i]);
        t.byte_offset = offsets[i];
        t.byte_size = sizes[i];
        t.byte_size_exact = true;
        tensors.push_back(std::move(t));
    }
    air::ModelConfig config;
    config.architecture = "qwen2";
    config.layer_count = cfg->layers;
    config.embedding_size = cfg->embedding;
    config.feed_forward_size = cfg->ffn;
    config.attention_head_count = cfg->heads;
    config.kv_head_count = cfg->kv_heads;
    config.rope_dimension_count = cfg->rope_dims;
    config.context_length = cfg->context;
    config.vocabulary_size = cfg->vocab;
    config.rope_frequency_base = cfg->rope_base;
    config.rms_norm_epsilon = cfg->eps;
    air::TokenizerDefinition tokenizer;
    for (std::uint64_t i = 0; i < cfg->vocab; ++i) tokenizer.vocabulary.push_back("t" + std::to_string(i));
    auto model = std::make_shared<air::ModelDefinition>(
        air::ModelFingerprint{"test", "qwen2", "oracle"}, std::move(config), std::move(tokenizer),
        std::move(tensors), std::move(storage).value());
    auto executor = air::ReferenceExecutor::create(model);
    if (!executor) return code_of(executor.status());
    auto* q = new airref_qwen2();
    q->executor = std::move(executor).value();
    q->config = *cfg;
    q->cache = std::make_unique<air::ReferenceKvCache>(cfg->layers, cfg->kv_heads, cfg->embedding / cfg->heads,
                                                       cfg->context);
    *out = q;
    return 0;
}

// ReferenceExecutor::step: appends `token` and writes the vocabulary logits.
int airref_qwen2_step(airref_qwen2* q, std::int32_t token, float* logits) {
    if (!q) return 1;
    auto out = q->executor->step(token, *q->cache);
    if (!out) return code_of(out.status());
    std::memcpy(logits, out.value().data(), out.value().size() * sizeof(float));
    return 0;
}

// Drops the sequence (a fresh cache).
int airref_qwen2_reset(airref_qwen2* q) {
    if (!q) return 1;
    const auto& c = q->config;
    q->cache = std::make_unique<air::ReferenceKvCache>(c.layers, c.kv_heads, c.embedding / c.heads, c.context);
    return 0;
}

void airref_qwen2_destroy(airref_qwen2* q) { delete q; }

// GgufFormat::load of AIR itself on a file: the status code, and on success
// the config and tensor table.  Lets the tests check that this repository's
// GGUF reader and writer agree with AIR's reader on the same files.
struct airref_gguf_config {
    std::uint32_t layers, embedding, ffn, heads, kv_heads, rope_dims;
    std::uint64_t vocab, context, sliding_window;
    double rope_base, rms_eps;
    std::int32_t eos;
    std::uint32_t tensors;
};

int airref_gguf_load(const char* path, airref_gguf_config* out, std::uint64_t* offsets, std::uint64_t* sizes,
                     std::uint32_t* types, std::uint32_t capacity) {
    air::GgufFormat format;
    auto model = format.load(path);
    if (!model) return code_of(model.status());
    const auto& c = model.value().config();
    const auto& tok = model.value().tokenizer();
    *out = airref_gguf_config{c.layer_count, c.embedding_size, c.feed_forward_size, c.attention_head_count,
                              c.kv_head_count, c.rope_dimension_count, c.vocabulary_size, c.context_length,
                              c.attention_sliding_window, c.rope_frequency_base, c.rms_norm_epsilon,
                              tok.special_ids.eos ? *tok.special_ids.eos : -1,
                              static_cast<std::uint32_t>(model.value().tensors().size())};
    const auto& tensors = model.value().tensors();
    for (std::uint32_t i = 0; i < capacity && i < tensors.size(); ++i) {
        offsets[i] = tensors[i].byte_offset;
        sizes[i] = tensors[i].byte_size;
        types[i] = tensors[i].format_type;
    }
    return 0;
}

} // extern "C"

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

} // extern "C"

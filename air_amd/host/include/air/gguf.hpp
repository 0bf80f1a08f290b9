// gguf.hpp -- GGUF v3 model files: reader, ModelDefinition loader, writer.
//
// The on-disk format (little-endian): "GGUF", u32 version, u64 tensor count,
// u64 metadata count, the metadata entries (string key, u32 value type,
// value; arrays carry an element type and a u64 count), the tensor infos
// (string name, u32 rank, u64 dims in GGML order, u32 GGML type, u64 offset
// relative to the data section), padding to `general.alignment` (32 by
// default), then the tensor data.  The loader follows AIR's GgufFormat
// (src/formats/gguf/gguf_reader.cpp:346-472, gguf_format.cpp:89-311): the same
// limits, required keys, defaults and error classes, so a file AIR accepts
// loads here with the same ModelConfig and tensor byte ranges.
//
// The file is memory-mapped read-only once; parsing walks the mapping with a
// bounds-checked cursor and the model's tensor bytes are views into the same
// mapping (no copy until the weights are made resident on the GPU).
#pragma once

#include "air/model.hpp"

#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <vector>

namespace air::gguf {

// GGUF metadata value types (gguf_reader.hpp:14-28).
enum class ValueType : std::uint32_t {
    u8 = 0, i8 = 1, u16 = 2, i16 = 3, u32 = 4, i32 = 5, f32 = 6, boolean = 7,
    string = 8, array = 9, u64 = 10, i64 = 11, f64 = 12,
};

// One metadata value: a scalar is an array of one element.  Numbers keep
// their bit pattern widened to 64 bits (signed values sign-extended, f32
// widened to f64); strings are kept as strings.
struct Value {
    ValueType element{ValueType::u8};
    bool is_array{false};
    std::vector<std::uint64_t> numbers;
    std::vector<std::string> strings;

    [[nodiscard]] std::size_t size() const noexcept;
    [[nodiscard]] bool is_integer() const noexcept;
    [[nodiscard]] bool is_signed() const noexcept;
    [[nodiscard]] bool is_float() const noexcept;
    // Scalar accessors (nullopt for arrays and for other types).
    [[nodiscard]] std::optional<std::uint64_t> as_u64() const noexcept;   // unsigned, or non-negative signed
    [[nodiscard]] std::optional<double> as_number() const noexcept;       // any integer or float
    [[nodiscard]] std::optional<bool> as_bool() const noexcept;
    [[nodiscard]] const std::string* as_string() const noexcept;
};

struct TensorInfo {
    std::string name;
    std::vector<std::uint64_t> dimensions;
    std::uint32_t type{0};
    std::uint64_t offset{0};   // relative to the data section
};

// A read-only memory mapping of a whole file.
class MappedFile final : public ModelStorage {
public:
    [[nodiscard]] static Result<std::shared_ptr<MappedFile>> open(const std::string& path);
    ~MappedFile() override;
    MappedFile(const MappedFile&) = delete;
    MappedFile& operator=(const MappedFile&) = delete;
    [[nodiscard]] std::span<const std::byte> bytes() const noexcept override {
        return {static_cast<const std::byte*>(data_), size_};
    }

private:
    MappedFile() = default;
    void* data_{nullptr};
    std::size_t size_{0};
};

struct Document {
    std::uint32_t version{0};
    std::uint32_t alignment{32};
    std::uint64_t data_offset{0};
    std::uint64_t file_size{0};
    std::map<std::string, Value> metadata;
    std::vector<TensorInfo> tensors;

    [[nodiscard]] const Value* find(const std::string& key) const noexcept;
};

// Parses the header of a mapped GGUF file.
[[nodiscard]] Result<Document> parse(std::span<const std::byte> file, const std::string& path);

// Block geometry of every GGML type id GGUF files carry (gguf_format.cpp:24-63);
// block_elements == 0 for ids without a fixed block (and unknown ids).
[[nodiscard]] FormatGeometry ggml_geometry(std::uint32_t type) noexcept;

// What the loader read besides the ModelDefinition (AIR keeps these in its
// ModelFingerprint and TokenizerDefinition).
struct ModelInfo {
    std::string format;          // "gguf-v3"
    std::string architecture;
    std::string name;            // general.name, else the file name
    std::string tokenizer_model; // tokenizer.ggml.model
    std::optional<TokenId> bos, eos;
};

// GgufFormat::load: header, tokenizer vocabulary size and special ids,
// ModelConfig, tensor descriptors over the mapping, model validation.
[[nodiscard]] Result<std::shared_ptr<const ModelDefinition>> load_model(const std::string& path,
                                                                        ModelInfo* info = nullptr);

// Writes `model` as a GGUF v3 file a loader (this one, AIR's, llama.cpp's)
// reads back: the Qwen2 metadata of its config, a placeholder vocabulary of
// config.vocabulary_size tokens ("<t0>", ...) with eos_token_id = `eos`,
// and every tensor in model order at `alignment`-aligned offsets.
struct WriteOptions {
    std::string name{"AIR-on-MI355X synthetic model"};
    std::uint32_t alignment{32};
    std::optional<TokenId> eos;
};
[[nodiscard]] Status write_model(const std::string& path, const ModelDefinition& model,
                                 const WriteOptions& options = {});

} // namespace air::gguf

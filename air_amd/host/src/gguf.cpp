// gguf.cpp -- GGUF v3 reader, ModelDefinition loader and writer.
#include "air/gguf.hpp"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <bit>
#include <cstring>
#include <fstream>
#include <limits>
#include <set>

namespace air::gguf {

namespace {

// Safety limits of AIR's reader (gguf_reader.cpp:16-20).
constexpr std::uint64_t kMaxStringBytes = 256ULL << 20;
constexpr std::uint64_t kMaxArrayElements = 16ULL << 20;
constexpr std::uint64_t kMaxMetadataEntries = 1ULL << 20;
constexpr std::uint64_t kMaxTensors = 4ULL << 20;
constexpr std::uint32_t kMaxRank = 8;

unsigned width_of(ValueType t) noexcept {
    switch (t) {
    case ValueType::u8: case ValueType::i8: case ValueType::boolean: return 1;
    case ValueType::u16: case ValueType::i16: return 2;
    case ValueType::u32: case ValueType::i32: case ValueType::f32: return 4;
    case ValueType::u64: case ValueType::i64: case ValueType::f64: return 8;
    case ValueType::string: case ValueType::array: return 0;
    }
    return 0;
}

// Bounds-checked little-endian reads over the mapping.
class Cursor {
public:
    explicit Cursor(std::span<const std::byte> bytes) : bytes_(bytes) {}
    [[nodiscard]] std::uint64_t position() const noexcept { return pos_; }

    Result<std::uint64_t> uint(unsigned width) {
        if (Status s = need(width); !s) return s;
        std::uint64_t v = 0;
        for (unsigned i = 0; i < width; ++i) v |= static_cast<std::uint64_t>(bytes_[pos_ + i]) << (8U * i);
        pos_ += width;
        return v;
    }
    Result<std::string> string() {
        auto length = uint(8);
        if (!length) return length.status();
        if (length.value() > kMaxStringBytes) return Status::data_error("GGUF string exceeds AIR safety limit");
        if (Status s = need(length.value()); !s) return s;
        std::string out(reinterpret_cast<const char*>(bytes_.data() + pos_), static_cast<std::size_t>(length.value()));
        pos_ += length.value();
        return out;
    }

private:
    Status need(std::uint64_t n) const {
        if (n > bytes_.size() - pos_) {
            return Status::data_error("GGUF ends unexpectedly at byte " + std::to_string(pos_));
        }
        return Status::ok();
    }
    std::span<const std::byte> bytes_;
    std::uint64_t pos_{0};
};

Result<ValueType> read_type(Cursor& c) {
    auto raw = c.uint(4);
    if (!raw) return raw.status();
    if (raw.value() > static_cast<std::uint32_t>(ValueType::f64)) {
        return Status::data_error("unknown GGUF metadata value type: " + std::to_string(raw.value()));
    }
    return static_cast<ValueType>(raw.value());
}

// One element of type t appended to v (numbers widened, see Value).
Status read_element(Cursor& c, ValueType t, Value& v) {
    if (t == ValueType::string) {
        auto s = c.string();
        if (!s) return s.status();
        v.strings.push_back(std::move(s).value());
        return Status::ok();
    }
    auto raw = c.uint(width_of(t));
    if (!raw) return raw.status();
    std::uint64_t bits = raw.value();
    switch (t) {
    case ValueType::i8: bits = static_cast<std::uint64_t>(static_cast<std::int64_t>(static_cast<std::int8_t>(bits))); break;
    case ValueType::i16: bits = static_cast<std::uint64_t>(static_cast<std::int64_t>(static_cast<std::int16_t>(bits))); break;
    case ValueType::i32: bits = static_cast<std::uint64_t>(static_cast<std::int64_t>(static_cast<std::int32_t>(bits))); break;
    case ValueType::f32:
        bits = std::bit_cast<std::uint64_t>(static_cast<double>(std::bit_cast<float>(static_cast<std::uint32_t>(bits))));
        break;
    case ValueType::boolean: bits = bits != 0 ? 1U : 0U; break;
    default: break;
    }
    v.numbers.push_back(bits);
    return Status::ok();
}

Result<Value> read_value(Cursor& c) {
    auto type = read_type(c);
    if (!type) return type.status();
    Value v;
    if (type.value() != ValueType::array) {
        v.element = type.value();
        if (Status s = read_element(c, v.element, v); !s) return s;
        return v;
    }
    auto element = read_type(c);
    if (!element) return element.status();
    auto count = c.uint(8);
    if (!count) return count.status();
    if (count.value() > kMaxArrayElements) return Status::data_error("GGUF array exceeds AIR safety limit");
    if (element.value() == ValueType::array) return Status::data_error("nested GGUF arrays are invalid");
    v.element = element.value();
    v.is_array = true;
    for (std::uint64_t i = 0; i < count.value(); ++i) {
        if (Status s = read_element(c, v.element, v); !s) return s;
    }
    return v;
}

std::uint64_t align_up(std::uint64_t v, std::uint64_t a) { return (v + a - 1U) / a * a; }

Result<std::uint32_t> narrow(std::uint64_t v, const std::string& key) {
    if (v > std::numeric_limits<std::uint32_t>::max()) {
        return Status::data_error("GGUF metadata exceeds AIR integer range: " + key);
    }
    return static_cast<std::uint32_t>(v);
}

Result<std::string> require_string(const Document& d, const std::string& key) {
    const Value* v = d.find(key);
    if (!v) return Status::data_error("missing GGUF metadata: " + key);
    const std::string* s = v->as_string();
    if (!s) return Status::data_error("GGUF metadata has wrong type: " + key);
    return *s;
}

Result<std::uint64_t> require_u64(const Document& d, const std::string& key) {
    const Value* v = d.find(key);
    const auto u = v ? v->as_u64() : std::nullopt;
    if (!u) return Status::data_error("missing or non-integer GGUF metadata: " + key);
    return *u;
}

std::optional<std::uint64_t> optional_u64(const Document& d, const std::string& key) {
    const Value* v = d.find(key);
    return v ? v->as_u64() : std::nullopt;
}

std::optional<double> optional_number(const Document& d, const std::string& key) {
    const Value* v = d.find(key);
    return v ? v->as_number() : std::nullopt;
}

// A special-token id: absent, or an integer inside the vocabulary
// (gguf_format.cpp:72-87).
Result<std::optional<TokenId>> special_id(const Document& d, const std::string& key, std::uint64_t vocab) {
    const Value* v = d.find(key);
    if (!v) return std::optional<TokenId>{};
    const auto id = v->as_u64();
    if (!id) return Status::data_error("GGUF special-token id has wrong type: " + key);
    if (*id >= vocab || *id > static_cast<std::uint64_t>(std::numeric_limits<TokenId>::max())) {
        return Status::data_error("GGUF special-token id is outside vocabulary: " + key);
    }
    return std::optional<TokenId>{static_cast<TokenId>(*id)};
}

// ModelConfig from the architecture's keys, AIR's defaults (gguf_format.cpp:89-152).
Result<ModelConfig> build_config(const Document& d, const std::string& arch, std::uint64_t vocab) {
    const auto key = [&arch](const char* suffix) { return arch + "." + suffix; };
    ModelConfig c;
    c.architecture = arch;
    auto layers = require_u64(d, key("block_count"));
    auto embedding = require_u64(d, key("embedding_length"));
    auto heads = require_u64(d, key("attention.head_count"));
    auto context = require_u64(d, key("context_length"));
    if (!layers) return layers.status();
    if (!embedding) return embedding.status();
    if (!heads) return heads.status();
    if (!context) return context.status();
    auto l32 = narrow(layers.value(), key("block_count"));
    auto e32 = narrow(embedding.value(), key("embedding_length"));
    auto h32 = narrow(heads.value(), key("attention.head_count"));
    if (!l32) return l32.status();
    if (!e32) return e32.status();
    if (!h32) return h32.status();
    c.layer_count = l32.value();
    c.embedding_size = e32.value();
    c.attention_head_count = h32.value();
    c.context_length = context.value();
    c.vocabulary_size = vocab;
    auto kv = narrow(optional_u64(d, key("attention.head_count_kv")).value_or(heads.value()),
                     key("attention.head_count_kv"));
    if (!kv) return kv.status();
    c.kv_head_count = kv.value();
    c.attention_sliding_window = optional_u64(d, key("attention.sliding_window")).value_or(0U);
    if (const auto ff = optional_u64(d, key("feed_forward_length"))) {
        auto f32v = narrow(*ff, key("feed_forward_length"));
        if (!f32v) return f32v.status();
        c.feed_forward_size = f32v.value();
    }
    const std::uint64_t default_rope = c.attention_head_count ? c.embedding_size / c.attention_head_count : 0U;
    auto rope = narrow(optional_u64(d, key("rope.dimension_count")).value_or(default_rope), key("rope.dimension_count"));
    if (!rope) return rope.status();
    c.rope_dimension_count = rope.value();
    c.rope_frequency_base = optional_number(d, key("rope.freq_base")).value_or(0.0);
    if (const Value* v = d.find(key("rope.scaling.type")); v && v->as_string()) c.rope_scaling_type = *v->as_string();
    c.rope_scaling_factor = optional_number(d, key("rope.scaling.factor")).value_or(1.0);
    c.rope_scale_linear = optional_number(d, key("rope.scale_linear")).value_or(1.0);
    c.rms_norm_epsilon = optional_number(d, key("attention.layer_norm_rms_epsilon")).value_or(0.0);
    if (const auto declared = optional_u64(d, key("vocab_size")); declared && *declared != vocab) {
        return Status::data_error("GGUF architecture vocab_size disagrees with tokenizer token count");
    }
    return c;
}

// Tensor descriptors over the mapping: exact sizes where the type has a
// fixed block, else the span up to the next tensor (gguf_format.cpp:215-267).
Result<std::vector<TensorDescriptor>> build_tensors(const Document& d) {
    std::vector<std::size_t> order(d.tensors.size());
    for (std::size_t i = 0; i < order.size(); ++i) order[i] = i;
    std::sort(order.begin(), order.end(),
              [&d](std::size_t a, std::size_t b) { return d.tensors[a].offset < d.tensors[b].offset; });
    std::vector<std::uint64_t> span(d.tensors.size(), 0);
    for (std::size_t k = 0; k < order.size(); ++k) {
        const std::uint64_t begin = d.tensors[order[k]].offset;
        const std::uint64_t end =
            k + 1 < order.size() ? d.tensors[order[k + 1]].offset : d.file_size - d.data_offset;
        if (end < begin) return Status::data_error("GGUF tensor offsets are not monotonic");
        span[order[k]] = end - begin;
    }
    std::vector<TensorDescriptor> out;
    out.reserve(d.tensors.size());
    for (std::size_t i = 0; i < d.tensors.size(); ++i) {
        const TensorInfo& t = d.tensors[i];
        TensorDescriptor desc;
        desc.name = t.name;
        desc.format_type = t.type;
        desc.shape.dimensions = t.dimensions;
        desc.byte_offset = d.data_offset + t.offset;
        const FormatGeometry g = ggml_geometry(t.type);
        const std::uint64_t elements = desc.shape.element_count();
        if (g.block_elements != 0 && elements != 0 && elements % g.block_elements == 0) {
            const std::uint64_t blocks = elements / g.block_elements;
            if (blocks > std::numeric_limits<std::uint64_t>::max() / g.block_bytes) {
                return Status::data_error("GGUF tensor byte size overflows: " + desc.name);
            }
            desc.byte_size = blocks * g.block_bytes;
            if (desc.byte_size > span[i]) {
                return Status::data_error("GGUF tensor overlaps following tensor or file end: " + desc.name);
            }
        } else {
            desc.byte_size = span[i];
        }
        if (desc.byte_size == 0) return Status::data_error("GGUF tensor occupies zero bytes: " + desc.name);
        out.push_back(std::move(desc));
    }
    return out;
}

} // namespace

// ---- Value -----------------------------------------------------------------

std::size_t Value::size() const noexcept { return element == ValueType::string ? strings.size() : numbers.size(); }

bool Value::is_integer() const noexcept {
    switch (element) {
    case ValueType::u8: case ValueType::i8: case ValueType::u16: case ValueType::i16: case ValueType::u32:
    case ValueType::i32: case ValueType::u64: case ValueType::i64: return true;
    default: return false;
    }
}

bool Value::is_signed() const noexcept {
    return element == ValueType::i8 || element == ValueType::i16 || element == ValueType::i32 ||
           element == ValueType::i64;
}

bool Value::is_float() const noexcept { return element == ValueType::f32 || element == ValueType::f64; }

std::optional<std::uint64_t> Value::as_u64() const noexcept {
    if (is_array || !is_integer() || numbers.size() != 1) return std::nullopt;
    if (is_signed() && static_cast<std::int64_t>(numbers[0]) < 0) return std::nullopt;
    return numbers[0];
}

std::optional<double> Value::as_number() const noexcept {
    if (is_array || numbers.size() != 1) return std::nullopt;
    if (is_float()) return std::bit_cast<double>(numbers[0]);
    if (is_signed()) return static_cast<double>(static_cast<std::int64_t>(numbers[0]));
    if (is_integer()) return static_cast<double>(numbers[0]);
    return std::nullopt;
}

std::optional<bool> Value::as_bool() const noexcept {
    if (is_array || element != ValueType::boolean || numbers.size() != 1) return std::nullopt;
    return numbers[0] != 0;
}

const std::string* Value::as_string() const noexcept {
    if (is_array || element != ValueType::string || strings.size() != 1) return nullptr;
    return &strings[0];
}

const Value* Document::find(const std::string& key) const noexcept {
    const auto it = metadata.find(key);
    return it == metadata.end() ? nullptr : &it->second;
}

// ---- MappedFile ------------------------------------------------------------

Result<std::shared_ptr<MappedFile>> MappedFile::open(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) return Status::io_error("unable to open or read GGUF file: " + path);
    struct stat st {};
    if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        return Status::io_error("unable to open or read GGUF file: " + path);
    }
    void* data = ::mmap(nullptr, static_cast<std::size_t>(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (data == MAP_FAILED) return Status::io_error("unable to map GGUF file: " + path);
    std::shared_ptr<MappedFile> file(new MappedFile());
    file->data_ = data;
    file->size_ = static_cast<std::size_t>(st.st_size);
    return file;
}

MappedFile::~MappedFile() {
    if (data_) ::munmap(data_, size_);
}

// ---- reader ----------------------------------------------------------------

FormatGeometry ggml_geometry(std::uint32_t type) noexcept {
    switch (type) {
    case 0: return {1, 4};       // f32
    case 1: return {1, 2};       // f16
    case 2: return {32, 18};     // q4_0
    case 3: return {32, 20};     // q4_1
    case 6: return {32, 22};     // q5_0
    case 7: return {32, 24};     // q5_1
    case 8: return {32, 34};     // q8_0
    case 9: return {32, 40};     // q8_1
    case 10: return {256, 84};   // q2_K
    case 11: return {256, 110};  // q3_K
    case 12: return {256, 144};  // q4_K
    case 13: return {256, 176};  // q5_K
    case 14: return {256, 210};  // q6_K
    case 15: return {256, 292};  // q8_K
    case 16: return {256, 66};   // iq2_xxs
    case 17: return {256, 74};   // iq2_xs
    case 18: return {256, 98};   // iq3_xxs
    case 19: return {256, 50};   // iq1_s
    case 20: return {32, 18};    // iq4_nl
    case 21: return {256, 110};  // iq3_s
    case 22: return {256, 82};   // iq2_s
    case 23: return {256, 136};  // iq4_xs
    case 24: return {1, 1};      // i8
    case 25: return {1, 2};      // i16
    case 26: return {1, 4};      // i32
    case 27: return {1, 8};      // i64
    case 28: return {1, 8};      // f64
    case 29: return {256, 56};   // iq1_m
    case 30: return {1, 2};      // bf16
    case 34: return {256, 54};   // tq1_0
    case 35: return {256, 66};   // tq2_0
    default: return {0, 0};
    }
}

Result<Document> parse(std::span<const std::byte> file, const std::string& path) {
    Cursor c(file);
    if (file.size() < 4 || std::memcmp(file.data(), "GGUF", 4) != 0) {
        return Status::invalid_argument("file is not GGUF: " + path);
    }
    (void)c.uint(4);
    auto version = c.uint(4);
    auto tensor_count = c.uint(8);
    auto metadata_count = c.uint(8);
    if (!version) return version.status();
    if (!tensor_count) return tensor_count.status();
    if (!metadata_count) return metadata_count.status();
    if (version.value() != 3) {
        return Status::unsupported("AIR currently supports GGUF V3; file uses V" + std::to_string(version.value()));
    }
    if (tensor_count.value() > kMaxTensors || metadata_count.value() > kMaxMetadataEntries) {
        return Status::data_error("GGUF header counts exceed AIR safety limits");
    }
    Document d;
    d.version = static_cast<std::uint32_t>(version.value());
    d.file_size = file.size();
    for (std::uint64_t i = 0; i < metadata_count.value(); ++i) {
        auto key = c.string();
        if (!key) return key.status();
        if (key.value().empty()) return Status::data_error("GGUF metadata key is empty");
        if (d.metadata.count(key.value())) return Status::data_error("duplicate GGUF metadata key: " + key.value());
        auto value = read_value(c);
        if (!value) return value.status();
        d.metadata.emplace(std::move(key).value(), std::move(value).value());
    }
    if (const auto a = optional_u64(d, "general.alignment")) {
        if (*a == 0 || (*a & (*a - 1)) != 0 || *a > 4096) {
            return Status::data_error("general.alignment must be a power of two in [1, 4096]");
        }
        d.alignment = static_cast<std::uint32_t>(*a);
    }
    if (const auto splits = optional_u64(d, "split.count"); splits && *splits > 1) {
        return Status::unsupported("multi-file GGUF model sets are deferred until model execution requires them");
    }
    std::set<std::string> names;
    for (std::uint64_t i = 0; i < tensor_count.value(); ++i) {
        TensorInfo t;
        auto name = c.string();
        auto rank = c.uint(4);
        if (!name) return name.status();
        if (!rank) return rank.status();
        if (name.value().empty()) return Status::data_error("GGUF tensor name is empty");
        if (!names.insert(name.value()).second) return Status::data_error("duplicate GGUF tensor name: " + name.value());
        if (rank.value() == 0 || rank.value() > kMaxRank) {
            return Status::data_error("GGUF tensor has invalid dimension count: " + name.value());
        }
        t.name = std::move(name).value();
        for (std::uint64_t k = 0; k < rank.value(); ++k) {
            auto dim = c.uint(8);
            if (!dim) return dim.status();
            if (dim.value() == 0) return Status::data_error("GGUF tensor has zero dimension: " + t.name);
            t.dimensions.push_back(dim.value());
        }
        auto type = c.uint(4);
        auto offset = c.uint(8);
        if (!type) return type.status();
        if (!offset) return offset.status();
        t.type = static_cast<std::uint32_t>(type.value());
        t.offset = offset.value();
        d.tensors.push_back(std::move(t));
    }
    d.data_offset = align_up(c.position(), d.alignment);
    if (d.data_offset > d.file_size) return Status::data_error("GGUF tensor-data offset exceeds file size");
    for (const auto& t : d.tensors) {
        if (t.offset > d.file_size - d.data_offset) {
            return Status::data_error("GGUF tensor offset exceeds tensor-data blob: " + t.name);
        }
    }
    return d;
}

Result<std::shared_ptr<const ModelDefinition>> load_model(const std::string& path, ModelInfo* info) {
    auto file = MappedFile::open(path);
    if (!file) return file.status();
    auto document = parse(file.value()->bytes(), path);
    if (!document) return document.status();
    const Document& d = document.value();

    auto arch = require_string(d, "general.architecture");
    if (!arch) return arch.status();
    auto tokenizer = require_string(d, "tokenizer.ggml.model");
    if (!tokenizer) return tokenizer.status();
    const Value* tokens = d.find("tokenizer.ggml.tokens");
    if (!tokens || !tokens->is_array || tokens->element != ValueType::string || tokens->strings.empty()) {
        return Status::data_error("missing or empty tokenizer.ggml.tokens");
    }
    const std::uint64_t vocab = tokens->strings.size();
    if (vocab > static_cast<std::uint64_t>(std::numeric_limits<TokenId>::max())) {
        return Status::unsupported("tokenizer vocabulary exceeds AIR TokenId range");
    }
    ModelInfo out_info;
    for (const char* key : {"tokenizer.ggml.bos_token_id", "tokenizer.ggml.eos_token_id",
                            "tokenizer.ggml.unknown_token_id", "tokenizer.ggml.padding_token_id",
                            "tokenizer.ggml.eot_token_id", "tokenizer.ggml.eom_token_id"}) {
        auto id = special_id(d, key, vocab);
        if (!id) return id.status();
        if (std::strcmp(key, "tokenizer.ggml.bos_token_id") == 0) out_info.bos = id.value();
        if (std::strcmp(key, "tokenizer.ggml.eos_token_id") == 0) out_info.eos = id.value();
    }
    auto config = build_config(d, arch.value(), vocab);
    if (!config) return config.status();
    auto tensors = build_tensors(d);
    if (!tensors) return tensors.status();

    auto model = std::make_shared<const ModelDefinition>(std::move(config).value(), std::move(tensors).value(),
                                                         std::shared_ptr<const ModelStorage>(file.value()));
    if (Status s = model->validate(); !s) return s;
    if (info) {
        out_info.format = "gguf-v" + std::to_string(d.version);
        out_info.architecture = arch.value();
        const Value* name = d.find("general.name");
        out_info.name = name && name->as_string() ? *name->as_string() : path.substr(path.find_last_of('/') + 1);
        out_info.tokenizer_model = tokenizer.value();
        *info = std::move(out_info);
    }
    return std::shared_ptr<const ModelDefinition>(model);
}

// ---- writer ----------------------------------------------------------------

namespace {

class Writer {
public:
    void u32(std::uint32_t v) { put(v, 4); }
    void u64(std::uint64_t v) { put(v, 8); }
    void str(const std::string& s) {
        u64(s.size());
        bytes_.insert(bytes_.end(), reinterpret_cast<const std::byte*>(s.data()),
                      reinterpret_cast<const std::byte*>(s.data()) + s.size());
    }
    void key_string(const std::string& k, const std::string& v) { str(k); u32(8); str(v); }
    void key_u32(const std::string& k, std::uint32_t v) { str(k); u32(4); u32(v); }
    void key_u64(const std::string& k, std::uint64_t v) { str(k); u32(10); u64(v); }
    void key_f64(const std::string& k, double v) { str(k); u32(12); u64(std::bit_cast<std::uint64_t>(v)); }
    void key_strings(const std::string& k, const std::vector<std::string>& v) {
        str(k); u32(9); u32(8); u64(v.size());
        for (const auto& s : v) str(s);
    }
    void pad(std::uint64_t alignment) { bytes_.resize(align_up(bytes_.size(), alignment), std::byte{0}); }
    [[nodiscard]] const std::vector<std::byte>& bytes() const noexcept { return bytes_; }

private:
    void put(std::uint64_t v, unsigned width) {
        for (unsigned i = 0; i < width; ++i) bytes_.push_back(static_cast<std::byte>((v >> (8U * i)) & 0xFFU));
    }
    std::vector<std::byte> bytes_;
};

} // namespace

Status write_model(const std::string& path, const ModelDefinition& model, const WriteOptions& options) {
    const auto& c = model.config();
    if (options.alignment == 0 || (options.alignment & (options.alignment - 1U)) != 0 || options.alignment > 4096) {
        return Status::invalid_argument("alignment must be a power of two in [1, 4096]");
    }
    if (c.vocabulary_size == 0 || c.vocabulary_size > static_cast<std::uint64_t>(std::numeric_limits<TokenId>::max())) {
        return Status::invalid_argument("vocabulary size must be in [1, 2^31)");
    }
    const std::string arch = c.architecture.empty() ? "qwen2" : c.architecture;
    const auto key = [&arch](const char* suffix) { return arch + "." + suffix; };
    Writer h;
    std::uint64_t metadata = 0;
    Writer kv;
    const auto count = [&metadata]() { ++metadata; };
    kv.key_string("general.architecture", arch); count();
    kv.key_string("general.name", options.name); count();
    kv.key_u32("general.alignment", options.alignment); count();
    kv.key_u32(key("block_count"), c.layer_count); count();
    kv.key_u64(key("context_length"), c.context_length); count();
    kv.key_u32(key("embedding_length"), c.embedding_size); count();
    kv.key_u32(key("feed_forward_length"), c.feed_forward_size); count();
    kv.key_u32(key("attention.head_count"), c.attention_head_count); count();
    kv.key_u32(key("attention.head_count_kv"), c.kv_head_count); count();
    kv.key_u32(key("rope.dimension_count"), c.rope_dimension_count); count();
    // f64 keeps the double values of the config exact through a round trip.
    kv.key_f64(key("rope.freq_base"), c.rope_frequency_base); count();
    kv.key_f64(key("attention.layer_norm_rms_epsilon"), c.rms_norm_epsilon); count();
    if (c.attention_sliding_window != 0) {
        kv.key_u64(key("attention.sliding_window"), c.attention_sliding_window);
        count();
    }
    if (c.rope_scaling_type != "none") {
        kv.key_string(key("rope.scaling.type"), c.rope_scaling_type);
        kv.key_f64(key("rope.scaling.factor"), c.rope_scaling_factor);
        metadata += 2;
    }
    kv.key_string("tokenizer.ggml.model", "gpt2"); count();
    std::vector<std::string> vocab(static_cast<std::size_t>(c.vocabulary_size));
    for (std::size_t i = 0; i < vocab.size(); ++i) vocab[i] = "<t" + std::to_string(i) + ">";
    kv.key_strings("tokenizer.ggml.tokens", vocab); count();
    if (options.eos) {
        if (*options.eos < 0 || static_cast<std::uint64_t>(*options.eos) >= c.vocabulary_size) {
            return Status::invalid_argument("eos token is outside the vocabulary");
        }
        kv.key_u32("tokenizer.ggml.eos_token_id", static_cast<std::uint32_t>(*options.eos));
        count();
    }

    // Tensor infos with aligned offsets in model order.
    Writer infos;
    std::vector<std::uint64_t> offsets;
    std::uint64_t offset = 0;
    for (const auto& t : model.tensors()) {
        infos.str(t.name);
        infos.u32(static_cast<std::uint32_t>(t.shape.dimensions.size()));
        for (const auto d : t.shape.dimensions) infos.u64(d);
        infos.u32(t.format_type);
        offset = align_up(offset, options.alignment);
        infos.u64(offset);
        offsets.push_back(offset);
        offset += t.byte_size;
    }

    h.u32(0x46554747U);  // "GGUF"
    h.u32(3);
    h.u64(model.tensors().size());
    h.u64(metadata);
    std::ofstream out(path, std::ios::binary | std::ios::trunc);
    if (!out) return Status::io_error("unable to create GGUF file: " + path);
    const auto write = [&out](std::span<const std::byte> b) {
        out.write(reinterpret_cast<const char*>(b.data()), static_cast<std::streamsize>(b.size()));
    };
    write(h.bytes());
    write(kv.bytes());
    write(infos.bytes());
    std::uint64_t position = h.bytes().size() + kv.bytes().size() + infos.bytes().size();
    const std::vector<std::byte> zeros(options.alignment, std::byte{0});
    const auto pad_to = [&](std::uint64_t target) {
        while (position < target) {
            const auto n = std::min<std::uint64_t>(target - position, zeros.size());
            write({zeros.data(), static_cast<std::size_t>(n)});
            position += n;
        }
    };
    const std::uint64_t data_offset = align_up(position, options.alignment);
    pad_to(data_offset);
    for (std::size_t i = 0; i < model.tensors().size(); ++i) {
        auto bytes = model.tensor_bytes(model.tensors()[i]);
        if (!bytes) return bytes.status();
        pad_to(data_offset + offsets[i]);
        write(bytes.value());
        position += bytes.value().size();
    }
    out.flush();
    if (!out) return Status::io_error("failed while writing GGUF file: " + path);
    return Status::ok();
}

} // namespace air::gguf

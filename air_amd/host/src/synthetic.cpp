// synthetic.cpp -- seeded random-init Qwen2 models and GGUF block quantizers.
//
// The block layouts written here are the ones the reference decodes
// (src/reference/tensor_reader.cpp:85-196): Q8_0 [d:f16][q:int8 x32],
// Q4_0 [d:f16][16 bytes: element i low nibble, element i+16 high nibble],
// Q4_K [d:f16][dmin:f16][12 bytes of 6-bit scales/mins][128 bytes: group g
// byte i = sub-block 2g element i low, sub-block 2g+1 element i high].
#include "air/synthetic.hpp"

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstring>
#include <thread>

namespace air {

std::uint16_t f32_to_f16_bits(float value) noexcept {
    std::uint32_t x;
    std::memcpy(&x, &value, sizeof(x));
    const std::uint32_t sign = (x >> 16) & 0x8000U;
    const std::uint32_t exp = (x >> 23) & 0xFFU;
    std::uint32_t man = x & 0x7FFFFFU;
    if (exp == 0xFFU) return static_cast<std::uint16_t>(sign | 0x7C00U | (man ? (0x200U | (man >> 13)) : 0U));
    const int e = static_cast<int>(exp) - 127 + 15;
    if (e >= 31) return static_cast<std::uint16_t>(sign | 0x7C00U);
    if (e <= 0) {
        if (e < -10) return static_cast<std::uint16_t>(sign);
        man |= 0x800000U;
        const int shift = 14 - e;  // value / 2^-24 = man24 >> shift
        std::uint32_t half = man >> shift;
        const std::uint32_t rem = man & ((1U << shift) - 1U);
        const std::uint32_t mid = 1U << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1U))) ++half;
        return static_cast<std::uint16_t>(sign | half);
    }
    std::uint32_t half = sign | (static_cast<std::uint32_t>(e) << 10) | (man >> 13);
    const std::uint32_t rem = man & 0x1FFFU;
    if (rem > 0x1000U || (rem == 0x1000U && (half & 1U))) ++half;  // a carry rounds into the exponent
    return static_cast<std::uint16_t>(half);
}

float f16_bits_to_f32(std::uint16_t bits) noexcept {
    const std::uint32_t sign = static_cast<std::uint32_t>(bits & 0x8000U) << 16;
    const std::uint32_t exp = (bits >> 10) & 0x1FU;
    std::uint32_t man = bits & 0x3FFU;
    std::uint32_t out;
    if (exp == 0U) {
        if (man == 0U) {
            out = sign;
        } else {
            int e = -1;
            do {
                ++e;
                man <<= 1;
            } while ((man & 0x400U) == 0U);
            out = sign | (static_cast<std::uint32_t>(127 - 15 - e) << 23) | ((man & 0x3FFU) << 13);
        }
    } else if (exp == 0x1FU) {
        out = sign | 0x7F800000U | (man << 13);
    } else {
        out = sign | ((exp + 127U - 15U) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &out, sizeof(f));
    return f;
}

namespace {

std::uint64_t splitmix64(std::uint64_t& state) noexcept {
    std::uint64_t z = (state += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

float round_half_away(float v) noexcept { return v >= 0.0f ? std::floor(v + 0.5f) : -std::floor(-v + 0.5f); }

void put_f16(std::byte* dst, float v) noexcept {
    const auto bits = f32_to_f16_bits(v);
    std::memcpy(dst, &bits, 2);
}

void quantize_q8_0_block(const float* b, std::byte* out) noexcept {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(b[i]));
    const float d = amax / 127.0f;
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    put_f16(out, d);
    for (int i = 0; i < 32; ++i) {
        const float q = std::clamp(round_half_away(b[i] * inv), -127.0f, 127.0f);
        out[2 + i] = static_cast<std::byte>(static_cast<std::int8_t>(q));
    }
}

void quantize_q4_0_block(const float* b, std::byte* out) noexcept {
    float vmax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        if (std::fabs(b[i]) > std::fabs(vmax)) vmax = b[i];
    }
    const float d = vmax / -8.0f;
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    put_f16(out, d);
    std::uint8_t q[32];
    for (int i = 0; i < 32; ++i) q[i] = static_cast<std::uint8_t>(std::clamp(std::floor(b[i] * inv + 8.5f), 0.0f, 15.0f));
    for (int i = 0; i < 16; ++i) out[2 + i] = static_cast<std::byte>(q[i] | (q[i + 16] << 4));
}

// Q5_0: d = -vmax / 16 (vmax the value of largest magnitude), code
// q = clamp(floor(x / d + 16.5), 0, 31); low nibbles in qs (elements i and
// i + 16 share byte i), fifth bits in the 32-bit qh (bit j for element j).
void quantize_q5_0_block(const float* b, std::byte* out) noexcept {
    float vmax = 0.0f;
    for (int i = 0; i < 32; ++i) {
        if (std::fabs(b[i]) > std::fabs(vmax)) vmax = b[i];
    }
    const float d = vmax / -16.0f;
    const float inv = d != 0.0f ? 1.0f / d : 0.0f;
    put_f16(out, d);
    std::uint32_t qh = 0;
    std::uint8_t q[32];
    for (int i = 0; i < 32; ++i) {
        q[i] = static_cast<std::uint8_t>(std::clamp(std::floor(b[i] * inv + 16.5f), 0.0f, 31.0f));
        qh |= static_cast<std::uint32_t>(q[i] >> 4) << i;
    }
    std::memcpy(out + 2, &qh, 4);
    for (int i = 0; i < 16; ++i) out[6 + i] = static_cast<std::byte>((q[i] & 0x0f) | ((q[i + 16] & 0x0f) << 4));
}

// Q6_K: sixteen sub-blocks of 16 with an int8 scale each under one f16 d;
// codes q in [0, 63] stand for q - 32.  Sub-block s covers elements 16 s ..
// 16 s + 15.  In each half of 128, element i + 32 j (i < 32, j < 4) keeps
// its low four bits in nibble j >> 1 of ql[i + 32 (j & 1)] and its high two
// bits at bits 2j, 2j + 1 of qh[i].
void quantize_q6_k_block(const float* b, std::byte* out) noexcept {
    float step[16];
    float max_step = 0.0f;
    for (int s = 0; s < 16; ++s) {
        float vmax = 0.0f;
        for (int i = 0; i < 16; ++i) {
            if (std::fabs(b[16 * s + i]) > std::fabs(vmax)) vmax = b[16 * s + i];
        }
        step[s] = vmax / -32.0f;
        if (std::fabs(step[s]) > std::fabs(max_step)) max_step = step[s];
    }
    const float d = max_step / -128.0f;
    const float dq = f16_bits_to_f32(f32_to_f16_bits(d));
    std::int8_t sc[16];
    for (int s = 0; s < 16; ++s) {
        sc[s] = static_cast<std::int8_t>(dq != 0.0f ? std::clamp(round_half_away(step[s] / dq), -128.0f, 127.0f) : 0.0f);
    }
    std::uint8_t q[256];
    for (int s = 0; s < 16; ++s) {
        const float unit = dq * static_cast<float>(sc[s]);
        const float inv = unit != 0.0f ? 1.0f / unit : 0.0f;
        for (int i = 0; i < 16; ++i) {
            q[16 * s + i] = static_cast<std::uint8_t>(std::clamp(round_half_away(b[16 * s + i] * inv) + 32.0f, 0.0f, 63.0f));
        }
    }
    std::memset(out, 0, 210);
    for (int half = 0; half < 2; ++half) {
        const std::uint8_t* h = q + 128 * half;
        for (int i = 0; i < 32; ++i) {
            for (int j = 0; j < 4; ++j) {
                const std::uint8_t v = h[i + 32 * j];
                auto& lo = out[64 * half + i + 32 * (j & 1)];
                lo = static_cast<std::byte>(std::to_integer<std::uint8_t>(lo) | ((v & 0x0f) << (4 * (j >> 1))));
                auto& hi = out[128 + 32 * half + i];
                hi = static_cast<std::byte>(std::to_integer<std::uint8_t>(hi) | ((v >> 4) << (2 * j)));
            }
        }
    }
    std::memcpy(out + 192, sc, 16);
    put_f16(out + 208, d);
}

// BF16: the high half of the f32 bits, rounded to nearest even.
void put_bf16(std::byte* dst, float v) noexcept {
    std::uint32_t bits = 0;
    std::memcpy(&bits, &v, 4);
    bits += 0x7fffu + ((bits >> 16) & 1u);
    const auto h = static_cast<std::uint16_t>(bits >> 16);
    std::memcpy(dst, &h, 2);
}

void quantize_q4_k_block(const float* b, std::byte* out) noexcept {
    float lo[8], step[8];
    float max_step = 0.0f, max_neg = 0.0f;
    for (int j = 0; j < 8; ++j) {
        float mn = 0.0f, mx = b[j * 32];
        for (int i = 0; i < 32; ++i) {
            mn = std::min(mn, b[j * 32 + i]);
            mx = std::max(mx, b[j * 32 + i]);
        }
        lo[j] = mn;
        step[j] = (mx - mn) / 15.0f;
        max_step = std::max(max_step, step[j]);
        max_neg = std::max(max_neg, -mn);
    }
    const auto d_bits = f32_to_f16_bits(max_step / 63.0f);
    const auto dmin_bits = f32_to_f16_bits(max_neg / 63.0f);
    const float d = f16_bits_to_f32(d_bits);
    const float dmin = f16_bits_to_f32(dmin_bits);
    std::uint8_t sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        sc[j] = static_cast<std::uint8_t>(d > 0.0f ? std::clamp(round_half_away(step[j] / d), 0.0f, 63.0f) : 0.0f);
        mn[j] = static_cast<std::uint8_t>(dmin > 0.0f ? std::clamp(round_half_away(-lo[j] / dmin), 0.0f, 63.0f) : 0.0f);
    }
    std::memcpy(out, &d_bits, 2);
    std::memcpy(out + 2, &dmin_bits, 2);
    auto* s = reinterpret_cast<std::uint8_t*>(out + 4);
    for (int j = 0; j < 4; ++j) {
        s[j] = static_cast<std::uint8_t>((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = static_cast<std::uint8_t>((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = static_cast<std::uint8_t>((sc[j + 4] & 0x0F) | ((mn[j + 4] & 0x0F) << 4));
    }
    std::uint8_t q[8][32];
    for (int j = 0; j < 8; ++j) {
        const float st = d * static_cast<float>(sc[j]);
        const float off = dmin * static_cast<float>(mn[j]);
        for (int i = 0; i < 32; ++i) {
            const float v = st > 0.0f ? (b[j * 32 + i] + off) / st : 0.0f;
            q[j][i] = static_cast<std::uint8_t>(std::clamp(round_half_away(v), 0.0f, 15.0f));
        }
    }
    auto* qs = reinterpret_cast<std::uint8_t*>(out + 16);
    for (int g = 0; g < 4; ++g) {
        for (int i = 0; i < 32; ++i) qs[g * 32 + i] = static_cast<std::uint8_t>(q[2 * g][i] | (q[2 * g + 1][i] << 4));
    }
}

// `blocks` consecutive blocks of `format_type` from w into out.
void quantize_blocks(std::uint32_t format_type, const float* w, std::uint64_t blocks, std::byte* out) noexcept {
    const auto g = format_geometry(format_type);
    for (std::uint64_t i = 0; i < blocks; ++i) {
        const float* src = w + i * g.block_elements;
        std::byte* dst = out + i * g.block_bytes;
        switch (static_cast<GgmlType>(format_type)) {
        case GgmlType::f32: std::memcpy(dst, src, 4); break;
        case GgmlType::f16: put_f16(dst, *src); break;
        case GgmlType::bf16: put_bf16(dst, *src); break;
        case GgmlType::q8_0: quantize_q8_0_block(src, dst); break;
        case GgmlType::q4_0: quantize_q4_0_block(src, dst); break;
        case GgmlType::q5_0: quantize_q5_0_block(src, dst); break;
        case GgmlType::q4_k: quantize_q4_k_block(src, dst); break;
        case GgmlType::q6_k: quantize_q6_k_block(src, dst); break;
        }
    }
}

} // namespace

Result<std::vector<std::byte>> quantize_rows(std::uint32_t format_type, std::span<const float> w, std::uint64_t k,
                                             std::uint64_t n) {
    const std::uint64_t dims[] = {k, n};
    auto bytes = exact_tensor_bytes(format_type, dims);
    if (!bytes) return bytes.status();
    if (w.size() != k * n) return Status::invalid_argument("quantize_rows: value count does not match k x n");
    std::vector<std::byte> out(bytes.value());
    quantize_blocks(format_type, w.data(), k * n / format_geometry(format_type).block_elements, out.data());
    return out;
}

// Value i of the stream is the (i mod 2) half of Box-Muller pair i / 2, made
// from splitmix64 draws i and i + 1; a chunk starting at an even `first`
// therefore starts from state seed + first * gamma.
void normal_fill(std::span<float> out, std::uint64_t seed, float sigma, std::uint64_t first) {
    std::uint64_t state = seed + first * 0x9E3779B97F4A7C15ULL;
    constexpr double kTwoPi = 6.283185307179586476925286766559;
    for (std::size_t i = 0; i < out.size(); i += 2) {
        // Box-Muller over two 53-bit uniforms, u1 in (0, 1].
        const double u1 = (static_cast<double>(splitmix64(state) >> 11) + 1.0) * 0x1.0p-53;
        const double u2 = static_cast<double>(splitmix64(state) >> 11) * 0x1.0p-53;
        const double r = std::sqrt(-2.0 * std::log(u1));
        out[i] = static_cast<float>(sigma * r * std::cos(kTwoPi * u2));
        if (i + 1 < out.size()) out[i + 1] = static_cast<float>(sigma * r * std::sin(kTwoPi * u2));
    }
}

std::uint64_t tensor_seed(std::uint64_t seed, const std::string& name) noexcept {
    std::uint64_t h = 0xCBF29CE484222325ULL;  // FNV-1a over the name
    for (const char c : name) h = (h ^ static_cast<unsigned char>(c)) * 0x100000001B3ULL;
    std::uint64_t state = seed ^ h;
    return splitmix64(state);
}

ModelConfig qwen2_config(std::uint32_t layers, std::uint32_t embedding, std::uint32_t ffn, std::uint32_t heads,
                         std::uint32_t kv_heads, std::uint64_t vocab, std::uint64_t context) {
    ModelConfig c;
    c.architecture = "qwen2";
    c.layer_count = layers;
    c.embedding_size = embedding;
    c.feed_forward_size = ffn;
    c.attention_head_count = heads;
    c.kv_head_count = kv_heads;
    c.rope_dimension_count = heads ? embedding / heads : 0U;
    c.context_length = context;
    c.vocabulary_size = vocab;
    c.rope_frequency_base = 1.0e6;
    c.rms_norm_epsilon = 1.0e-6;
    return c;
}

Result<std::shared_ptr<const ModelDefinition>> make_synthetic_qwen2(const SyntheticQwen2Spec& spec) {
    const auto& c = spec.config;
    if (c.attention_head_count == 0U || c.kv_head_count == 0U) {
        return Status::invalid_argument("synthetic Qwen2 needs head counts");
    }
    const std::uint64_t e = c.embedding_size;
    const std::uint64_t head = e / c.attention_head_count;
    const std::uint64_t qw = c.attention_head_count * head;
    const std::uint64_t kvw = c.kv_head_count * head;
    const std::uint64_t ffn = c.feed_forward_size;
    const std::uint64_t vocab = c.vocabulary_size;
    const auto f32 = static_cast<std::uint32_t>(GgmlType::f32);

    struct Pending {
        std::string name;
        std::uint32_t format;
        std::uint64_t k, n;  // GGML {k, n}; vectors have n = 1
        enum { normal, ones } fill;
        bool vector;
    };
    std::vector<Pending> pending;
    pending.push_back({"token_embd.weight", spec.embedding_format, e, vocab, Pending::normal, false});
    pending.push_back({"output_norm.weight", f32, e, 1, Pending::ones, true});
    const auto pick = [&](std::uint32_t f) { return f == SyntheticQwen2Spec::kSameFormat ? spec.weight_format : f; };
    const std::uint32_t v_down = pick(spec.v_down_format);
    if (!spec.tied_output) pending.push_back({"output.weight", pick(spec.output_format), e, vocab, Pending::normal, false});
    if (spec.output_bias) pending.push_back({"output.bias", f32, vocab, 1, Pending::normal, true});
    for (std::uint32_t l = 0; l < c.layer_count; ++l) {
        const auto n = [l](const char* s) { return block_tensor_name(l, s); };
        pending.push_back({n("attn_norm.weight"), f32, e, 1, Pending::ones, true});
        pending.push_back({n("attn_q.weight"), spec.weight_format, e, qw, Pending::normal, false});
        pending.push_back({n("attn_k.weight"), spec.weight_format, e, kvw, Pending::normal, false});
        pending.push_back({n("attn_v.weight"), v_down, e, kvw, Pending::normal, false});
        if (spec.qkv_bias) {
            pending.push_back({n("attn_q.bias"), f32, qw, 1, Pending::normal, true});
            pending.push_back({n("attn_k.bias"), f32, kvw, 1, Pending::normal, true});
            pending.push_back({n("attn_v.bias"), f32, kvw, 1, Pending::normal, true});
        }
        pending.push_back({n("attn_output.weight"), spec.weight_format, qw, e, Pending::normal, false});
        pending.push_back({n("ffn_norm.weight"), f32, e, 1, Pending::ones, true});
        pending.push_back({n("ffn_gate.weight"), spec.weight_format, e, ffn, Pending::normal, false});
        pending.push_back({n("ffn_up.weight"), spec.weight_format, e, ffn, Pending::normal, false});
        pending.push_back({n("ffn_down.weight"), v_down, ffn, e, Pending::normal, false});
    }

    std::vector<TensorDescriptor> tensors;
    std::uint64_t offset = 0;
    for (const auto& p : pending) {
        TensorDescriptor t;
        t.name = p.name;
        t.format_type = p.format;
        t.shape.dimensions = p.vector ? std::vector<std::uint64_t>{p.k} : std::vector<std::uint64_t>{p.k, p.n};
        auto bytes = exact_tensor_bytes(p.format, t.shape.dimensions);
        if (!bytes) return Status::invalid_argument("synthetic tensor " + p.name + ": " + bytes.status().message());
        t.byte_offset = offset;
        t.byte_size = bytes.value();
        offset += (t.byte_size + 31U) & ~std::uint64_t{31U};
        tensors.push_back(std::move(t));
    }

    // Chunks of 2^20 values (whole blocks, even offsets) filled and quantized
    // on up to 16 threads; the bytes equal a sequential fill.
    std::vector<std::byte> storage(offset);
    struct Job {
        std::size_t tensor;
        std::uint64_t first, count;
    };
    constexpr std::uint64_t kChunk = 1ULL << 20;
    std::vector<Job> jobs;
    for (std::size_t i = 0; i < pending.size(); ++i) {
        const std::uint64_t total = pending[i].k * pending[i].n;
        for (std::uint64_t first = 0; first < total; first += kChunk) {
            jobs.push_back({i, first, std::min(kChunk, total - first)});
        }
    }
    std::atomic<std::size_t> next{0};
    const auto worker = [&]() {
        std::vector<float> values;
        for (std::size_t j = next.fetch_add(1); j < jobs.size(); j = next.fetch_add(1)) {
            const auto& job = jobs[j];
            const auto& p = pending[job.tensor];
            values.assign(job.count, 1.0f);
            if (p.fill == Pending::normal) {
                normal_fill(values, tensor_seed(spec.seed, p.name), spec.sigma, job.first);
            }
            const auto g = format_geometry(p.format);
            quantize_blocks(p.format, values.data(), job.count / g.block_elements,
                            storage.data() + tensors[job.tensor].byte_offset +
                                job.first / g.block_elements * g.block_bytes);
        }
    };
    const unsigned threads = std::clamp(std::thread::hardware_concurrency(), 1U, 16U);
    std::vector<std::thread> pool;
    for (unsigned t = 1; t < threads && jobs.size() > 1U; ++t) pool.emplace_back(worker);
    worker();
    for (auto& t : pool) t.join();
    auto model = std::make_shared<const ModelDefinition>(
        c, std::move(tensors), std::make_shared<const BufferStorage>(std::move(storage)));
    if (Status s = model->validate(); !s) return s;
    if (Status s = validate_qwen2_structure(*model); !s) return s;
    return std::shared_ptr<const ModelDefinition>(model);
}

} // namespace air

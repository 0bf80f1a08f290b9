// make_reference_blocks.cpp -- writes tests/golden/reference_blocks.json.
//
// Regenerates the block fixtures of AIR's own unit tests so the CPU oracle can
// be checked against them:
//   * the known-answer blocks of tests/reference_tests.cpp:158-190
//     (Q4_0 0x98 -> 16 x 0 then 16 x 1; Q5_0 -> 0 / 1; Q8_0 bytes 0..31;
//     Q4_K scales 0x01, quants 0x21 -> 1 / 2; Q6_K -> 1);
//   * the randomized blocks of tests/reference_tests.cpp:244-370: 32 blocks per
//     format drawn from std::mt19937(0xA17C0DE) with
//     std::uniform_int_distribution<int>(0, 255) (and (-8, 8) for Q6_K
//     scales) in the same draw order, and the expected values computed with
//     the test's independent per-format formulas.
// It must be built with g++/libstdc++ (the distribution's algorithm is the
// standard library's).  Build and run:
//   g++ -std=c++20 -O2 -o /tmp/mrb tests/golden/make_reference_blocks.cpp
//   /tmp/mrb > tests/golden/reference_blocks.json
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

namespace {

std::string hex(const std::vector<std::uint8_t>& b) {
    static const char* d = "0123456789abcdef";
    std::string s;
    for (auto v : b) { s += d[v >> 4]; s += d[v & 15]; }
    return s;
}

std::string floats(const std::vector<float>& v) {
    std::string s = "[";
    char buf[32];
    for (std::size_t i = 0; i < v.size(); ++i) {
        // keep the sign of negative zero ("-0" would read back as integer 0)
        if (v[i] == 0.0F && std::signbit(v[i])) std::snprintf(buf, sizeof buf, "%s-0.0", i ? "," : "");
        else std::snprintf(buf, sizeof buf, "%s%.9g", i ? "," : "", static_cast<double>(v[i]));
        s += buf;
    }
    return s + "]";
}

void entry(const char* name, int ggml, std::size_t elements, const std::vector<std::uint8_t>& bytes,
           const std::vector<float>& expected, bool last) {
    std::printf("  \"%s\": {\"type\": %d, \"elements\": %zu, \"bytes\": \"%s\", \"expected\": %s}%s\n", name, ggml,
                elements, hex(bytes).c_str(), floats(expected).c_str(), last ? "" : ",");
}

void scale_min(std::uint32_t index, const std::uint8_t* packed, std::uint8_t& scale, std::uint8_t& minimum) {
    if (index < 4U) {
        scale = packed[index] & 63U;
        minimum = packed[index + 4U] & 63U;
    } else {
        scale = static_cast<std::uint8_t>((packed[index + 4U] & 0x0fU) | ((packed[index - 4U] >> 6U) << 4U));
        minimum = static_cast<std::uint8_t>((packed[index + 4U] >> 4U) | ((packed[index] >> 6U) << 4U));
    }
}

} // namespace

int main() {
    std::printf("{\n");
    std::printf("  \"_source\": \"AIR tests/reference_tests.cpp:158-190 (known answers) and :244-370 (mt19937 0xA17C0DE)\",\n");

    // ---- known-answer blocks ----
    {
        std::vector<std::uint8_t> q4(18, 0x98);
        q4[0] = 0x00; q4[1] = 0x3c;
        std::vector<float> e(32);
        for (int i = 0; i < 32; ++i) e[i] = i < 16 ? 0.0F : 1.0F;
        entry("kat_q4_0", 2, 32, q4, e, false);
    }
    {
        std::vector<std::uint8_t> q5(22, 0x10);
        q5[0] = 0x00; q5[1] = 0x3c;
        for (int i = 2; i < 6; ++i) q5[i] = 0xff;
        std::vector<float> e(32);
        for (int i = 0; i < 32; ++i) e[i] = i < 16 ? 0.0F : 1.0F;
        entry("kat_q5_0", 6, 32, q5, e, false);
    }
    {
        std::vector<std::uint8_t> q8(34, 0);
        q8[0] = 0x00; q8[1] = 0x3c;
        std::vector<float> e(32);
        for (int i = 0; i < 32; ++i) { q8[2 + i] = static_cast<std::uint8_t>(i); e[i] = static_cast<float>(i); }
        entry("kat_q8_0", 8, 32, q8, e, false);
    }
    {
        std::vector<std::uint8_t> q4k(144, 0x21);
        q4k[0] = 0x00; q4k[1] = 0x3c; q4k[2] = 0x00; q4k[3] = 0x00;
        for (int i = 4; i < 16; ++i) q4k[i] = 0x01;
        std::vector<float> e(256);
        for (int g = 0; g < 4; ++g)
            for (int i = 0; i < 32; ++i) { e[g * 64 + i] = 1.0F; e[g * 64 + 32 + i] = 2.0F; }
        entry("kat_q4_k", 12, 256, q4k, e, false);
    }
    {
        std::vector<std::uint8_t> q6k(210, 0);
        for (int i = 0; i < 128; ++i) q6k[i] = 0x11;
        for (int i = 128; i < 192; ++i) q6k[i] = 0xaa;
        for (int i = 192; i < 208; ++i) q6k[i] = 0x01;
        q6k[208] = 0x00; q6k[209] = 0x3c;
        entry("kat_q6_k", 14, 256, q6k, std::vector<float>(256, 1.0F), false);
    }

    // ---- randomized blocks, same draw order as the reference test ----
    constexpr std::size_t cases = 32U;
    std::mt19937 rng(0xA17C0DEU);
    std::uniform_int_distribution<int> byte_dist(0, 255);
    std::uniform_int_distribution<int> scale_dist(-8, 8);

    std::vector<std::uint8_t> q4(cases * 18U);
    std::vector<float> q4e(cases * 32U);
    for (std::size_t b = 0; b < cases; ++b) {
        auto* raw = q4.data() + b * 18U;
        raw[0] = 0x00; raw[1] = 0x3c;
        for (std::size_t i = 0; i < 16U; ++i) {
            const auto packed = static_cast<std::uint8_t>(byte_dist(rng));
            raw[2 + i] = packed;
            q4e[b * 32U + i] = static_cast<float>(static_cast<int>(packed & 0x0fU) - 8);
            q4e[b * 32U + 16U + i] = static_cast<float>(static_cast<int>(packed >> 4U) - 8);
        }
    }
    std::vector<std::uint8_t> q5(cases * 22U);
    std::vector<float> q5e(cases * 32U);
    for (std::size_t b = 0; b < cases; ++b) {
        auto* raw = q5.data() + b * 22U;
        raw[0] = 0x00; raw[1] = 0x3c;
        for (std::size_t i = 0; i < 4U; ++i) raw[2 + i] = static_cast<std::uint8_t>(byte_dist(rng));
        for (std::size_t i = 0; i < 16U; ++i) raw[6 + i] = static_cast<std::uint8_t>(byte_dist(rng));
        for (std::uint32_t i = 0; i < 32U; ++i) {
            const std::uint8_t packed = raw[6 + (i % 16U)];
            const std::uint8_t low = i < 16U ? (packed & 0x0fU) : (packed >> 4U);
            const std::uint8_t high = static_cast<std::uint8_t>(((raw[2 + i / 8U] >> (i % 8U)) & 1U) << 4U);
            q5e[b * 32U + i] = static_cast<float>(static_cast<int>(low | high) - 16);
        }
    }
    std::vector<std::uint8_t> q8(cases * 34U);
    std::vector<float> q8e(cases * 32U);
    for (std::size_t b = 0; b < cases; ++b) {
        auto* raw = q8.data() + b * 34U;
        raw[0] = 0x00; raw[1] = 0x3c;
        for (std::size_t i = 0; i < 32U; ++i) {
            const auto v = static_cast<std::uint8_t>(byte_dist(rng));
            raw[2 + i] = v;
            q8e[b * 32U + i] = static_cast<float>(static_cast<std::int8_t>(v));
        }
    }
    std::vector<std::uint8_t> q4k(cases * 144U);
    std::vector<float> q4ke(cases * 256U);
    for (std::size_t b = 0; b < cases; ++b) {
        auto* raw = q4k.data() + b * 144U;
        raw[0] = 0x00; raw[1] = 0x3c;  // d = 1
        raw[2] = 0x00; raw[3] = 0x38;  // dmin = 0.5
        for (std::size_t i = 0; i < 12U; ++i) raw[4 + i] = static_cast<std::uint8_t>(byte_dist(rng));
        for (std::size_t i = 0; i < 128U; ++i) raw[16 + i] = static_cast<std::uint8_t>(byte_dist(rng));
        std::uint32_t si = 0U;
        for (std::uint32_t g = 0; g < 4U; ++g) {
            std::uint8_t s0 = 0, m0 = 0, s1 = 0, m1 = 0;
            scale_min(si, raw + 4, s0, m0);
            scale_min(si + 1U, raw + 4, s1, m1);
            for (std::uint32_t i = 0; i < 32U; ++i) {
                const std::uint8_t packed = raw[16 + g * 32U + i];
                q4ke[b * 256U + g * 64U + i] = static_cast<float>(s0) * static_cast<float>(packed & 0x0fU) - 0.5F * static_cast<float>(m0);
                q4ke[b * 256U + g * 64U + 32U + i] = static_cast<float>(s1) * static_cast<float>(packed >> 4U) - 0.5F * static_cast<float>(m1);
            }
            si += 2U;
        }
    }
    std::vector<std::uint8_t> q6k(cases * 210U);
    std::vector<float> q6ke(cases * 256U);
    for (std::size_t b = 0; b < cases; ++b) {
        auto* raw = q6k.data() + b * 210U;
        for (std::size_t i = 0; i < 192U; ++i) raw[i] = static_cast<std::uint8_t>(byte_dist(rng));
        for (std::size_t i = 0; i < 16U; ++i) raw[192 + i] = static_cast<std::uint8_t>(static_cast<std::int8_t>(scale_dist(rng)));
        raw[208] = 0x00; raw[209] = 0x38;  // d = 0.5
        for (std::uint32_t half = 0; half < 2U; ++half) {
            const auto* low = raw + half * 64U;
            const auto* high = raw + 128U + half * 32U;
            const auto* scales = raw + 192U + half * 8U;
            for (std::uint32_t i = 0; i < 32U; ++i) {
                const std::uint8_t lo0 = low[i], lo1 = low[i + 32U], hi = high[i];
                const std::uint32_t pair = i / 16U;
                auto dec = [](std::uint8_t l, std::uint8_t h) { return static_cast<std::int32_t>(l | static_cast<std::uint8_t>(h << 4U)) - 32; };
                const std::int32_t values[4] = {dec(lo0 & 0x0fU, (hi >> 0U) & 3U), dec(lo1 & 0x0fU, (hi >> 2U) & 3U),
                                                dec(lo0 >> 4U, (hi >> 4U) & 3U), dec(lo1 >> 4U, (hi >> 6U) & 3U)};
                const std::uint32_t offsets[4] = {0U, 32U, 64U, 96U};
                const std::uint32_t scale_offsets[4] = {0U, 2U, 4U, 6U};
                for (std::uint32_t lane = 0; lane < 4U; ++lane) {
                    const auto sc = static_cast<std::int8_t>(scales[pair + scale_offsets[lane]]);
                    q6ke[b * 256U + half * 128U + offsets[lane] + i] = 0.5F * static_cast<float>(sc) * static_cast<float>(values[lane]);
                }
            }
        }
    }
    entry("random_q4_0", 2, cases * 32U, q4, q4e, false);
    entry("random_q5_0", 6, cases * 32U, q5, q5e, false);
    entry("random_q8_0", 8, cases * 32U, q8, q8e, false);
    entry("random_q4_k", 12, cases * 256U, q4k, q4ke, false);
    entry("random_q6_k", 14, cases * 256U, q6k, q6ke, true);
    std::printf("}\n");
    return 0;
}

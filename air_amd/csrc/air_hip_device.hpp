// air_hip_device.hpp -- device helpers shared by the HIP kernels.
#pragma once

#include "air_hip_layout.hpp"

#include <hip/hip_runtime.h>
#include <cstdint>

namespace air_hip {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half8v __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
// Native 128/64-bit integer vectors for staging registers: HIP's uint4 is a
// struct whose copies become memcpys, which can pin an array of them in
// scratch memory; these stay in VGPRs.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Exact IEEE half -> single from the bit pattern, integer-only so NaN
// payloads and subnormals decode exactly as src/reference/tensor_reader.cpp:11-36.
__device__ __forceinline__ float f16_bits_to_f32(std::uint32_t h) {
    const std::uint32_t sign = (h & 0x8000u) << 16;
    const std::uint32_t exponent = (h >> 10) & 0x1fu;
    std::uint32_t mantissa = h & 0x03ffu;
    std::uint32_t bits;
    if (exponent == 0u) {
        if (mantissa == 0u) {
            bits = sign;
        } else {
            // value = mantissa * 2^-24: normalise with one count-leading-zeros
            const std::uint32_t shift = __clz(mantissa) - 21u; // bit 10 reached
            mantissa = (mantissa << shift) & 0x03ffu;
            bits = sign | ((113u - shift) << 23) | (mantissa << 13);
        }
    } else if (exponent == 0x1fu) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    }
    return __uint_as_float(bits);
}

__device__ __forceinline__ half2v bits_as_half2(std::uint32_t v) {
    return __builtin_bit_cast(half2v, v);
}

// Four biased Q8_0 codes u = q + 128 (one dword) -> four exact f16 values q.
// v_perm_b32 places each byte under the exponent byte 0x64: f16 0x64uu = 1024+u.
__device__ __forceinline__ void q8_dword_to_half(std::uint32_t u, half2v& lo, half2v& hi) {
    const half2v bias = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = bits_as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
    hi = bits_as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
}

// One nibble dword (placement kNibblePos) -> eight exact f16 values n - offset.
// Each half is the nibble under an exponent (f16 0x64nn = 1024 + n, 0x54n0 =
// 64 + n) minus that bias.  The two exponent patterns are passed through an
// empty asm so they live in VGPRs: VOP3 takes no literal on this chip, and
// with the mask in an SGPR and the pattern in a VGPR the mask-and-insert is
// one v_and_or_b32 instead of an AND and an OR (the asm is not volatile, so
// its copies are shared and hoisted).
template <int Offset>
__device__ __forceinline__ half8v nibble_dword_to_half8(std::uint32_t w) {
    const half2v b_hi = {(_Float16)(1024.0f + Offset), (_Float16)(1024.0f + Offset)};
    const half2v b_lo = {(_Float16)(64.0f + Offset), (_Float16)(64.0f + Offset)};
    std::uint32_t e_hi = 0x64006400u, e_lo = 0x54005400u;
    asm("" : "+v"(e_hi));
    asm("" : "+v"(e_lo));
    const std::uint32_t w8 = w >> 8;
    const half2v p0 = bits_as_half2((w & 0x000f000fu) | e_hi) - b_hi;
    const half2v p1 = bits_as_half2((w & 0x00f000f0u) | e_lo) - b_lo;
    const half2v p2 = bits_as_half2((w8 & 0x000f000fu) | e_hi) - b_hi;
    const half2v p3 = bits_as_half2((w8 & 0x00f000f0u) | e_lo) - b_lo;
    half8v out;
    out[0] = p0[0]; out[1] = p0[1]; out[2] = p1[0]; out[3] = p1[1];
    out[4] = p2[0]; out[5] = p2[1]; out[6] = p3[0]; out[7] = p3[1];
    return out;
}

// Q4_K 6-bit scale/min of sub-block j from the 12 packed bytes
// (src/reference/tensor_reader.cpp:153-165).  `s` holds the three dwords of
// the packed bytes (little-endian).
__device__ __forceinline__ std::uint32_t byte_of(const std::uint32_t s[3], std::uint32_t i) {
    return (s[i >> 2] >> ((i & 3u) * 8u)) & 0xffu;
}
__device__ __forceinline__ void q4k_scale_min(const std::uint32_t s[3], std::uint32_t j,
                                              std::uint32_t& sc, std::uint32_t& mn) {
    if (j < 4u) {
        sc = byte_of(s, j) & 63u;
        mn = byte_of(s, j + 4u) & 63u;
    } else {
        sc = (byte_of(s, j + 4u) & 0x0fu) | ((byte_of(s, j - 4u) >> 6) << 4);
        mn = (byte_of(s, j + 4u) >> 4) | ((byte_of(s, j) >> 6) << 4);
    }
}

// The 6-bit scales and mins of Q4_K sub-blocks 4u .. 4u + 3 (u = upper),
// one per byte, from the same packed dwords: sub-blocks 0-3 have scale =
// byte j & 63 and min = byte j + 4 & 63; 4-7 the low / high nibble of byte
// j + 4 with bits 6-7 of byte j - 4 (scale) / byte j (min) above it --
// q4k_scale_min for four sub-blocks at once.
__device__ __forceinline__ void q4k_scale_min_x4(const std::uint32_t s[3], bool upper, std::uint32_t& scales,
                                                 std::uint32_t& mins) {
    scales = upper ? ((s[2] & 0x0f0f0f0fu) | ((s[0] >> 2) & 0x30303030u)) : (s[0] & 0x3f3f3f3fu);
    mins = upper ? (((s[2] >> 4) & 0x0f0f0f0fu) | ((s[1] >> 2) & 0x30303030u)) : (s[1] & 0x3f3f3f3fu);
}

// Q6_K super-block record (linear_dense.hip): byte b (0..47) of lane group
// g's codes lies at 48 g + b, so a lane group reads its whole super-block in
// three 16-byte loads.  Group g's bytes: 4-byte runs 12 (2 h + s) + {0, 4:
// low nibbles of quadrants with j % 2 = 0, 1; 8: high pairs} for half h,
// half-quadrant s, elements 4 g..+3.
__host__ __device__ constexpr std::uint32_t q6k_code_offset(std::uint32_t g, std::uint32_t b) { return 48u * g + b; }

__device__ __forceinline__ float lane_value(float v, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

template <int kCtrl>
__device__ __forceinline__ float dpp_float(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}

// Maximum over the 64 lanes: within each 16-lane row by DPP (quad swaps,
// half-row and row mirrors), then across the four rows by readlane.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_float<0xb1>(v));    // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, dpp_float<0x4e>(v));    // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, dpp_float<0x141>(v));   // row_half_mirror
    v = fmaxf(v, dpp_float<0x140>(v));   // row_mirror
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

__device__ __forceinline__ float4v mfma16x16x32(const half8v& a, const half8v& b, const float4v& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Power-of-two scale of one (row, 32-element block) of activations: with
// amax = max|x| over the block, amax*s lies in [2^14, 2^15), so the f16 hi
// part cannot overflow and the lo part keeps the residual.  Zero and
// non-finite blocks are left unscaled (NaN/inf then propagate as in f32).
__device__ __forceinline__ void block_scale(float amax, float& s, float& inv) {
    const std::uint32_t e = (__float_as_uint(amax) >> 23) & 0xffu;
    if (!(amax > 0.0f) || e == 0xffu) {
        s = 1.0f;
        inv = 1.0f;
        return;
    }
    int se = 268 - static_cast<int>(e);  // s = 2^(141 - e)
    se = se > 253 ? 253 : se;
    s = __uint_as_float(static_cast<std::uint32_t>(se) << 23);
    inv = __uint_as_float(static_cast<std::uint32_t>(254 - se) << 23);
}

// Splits eight scaled activations v*s into f16 hi + lo with hi + lo = v*s to
// ~21 significant bits: cvt_pkrtz rounds toward zero, so hi is v*s truncated
// to 11 bits, the residual v*s - hi is exact in f32, and lo is that residual
// truncated to 11 bits as well (the error is below one ulp of lo).
__device__ __forceinline__ void split8(const float (&v)[8], float s, half8v& hi, half8v& lo) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float a = v[2 * e] * s;
        const float b = v[2 * e + 1] * s;
        const auto h = __builtin_amdgcn_cvt_pkrtz(a, b);
        const auto l = __builtin_amdgcn_cvt_pkrtz(a - static_cast<float>(h[0]), b - static_cast<float>(h[1]));
        hi[2 * e] = static_cast<_Float16>(h[0]);
        hi[2 * e + 1] = static_cast<_Float16>(h[1]);
        lo[2 * e] = static_cast<_Float16>(l[0]);
        lo[2 * e + 1] = static_cast<_Float16>(l[1]);
    }
}

// Stores run r (eight consecutive activations v of row m; run r = 4 * block
// + g) of a row-scaled activation split: hi and lo f16 records of the
// skinny kernel's tile layout (xs[block][mp / 16][hi, lo][64 lanes]), and
// for g == 0 the block's scaled sum (block_sums[block][mp]).  The four runs
// of a block must sit in four adjacent active lanes (their sums are combined
// across lanes).
__device__ __forceinline__ void emit_split_run(std::uint64_t r, const float (&v)[8], float s, std::uint32_t m,
                                               std::uint32_t mp, uint4* __restrict__ xs,
                                               float* __restrict__ block_sums) {
    const std::uint32_t mtiles = mp / 16u;
    const std::uint64_t b = r >> 2;
    const std::uint32_t g = static_cast<std::uint32_t>(r & 3u);
    half8v hi, lo;
    split8(v, s, hi, lo);
    float sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += v[e] * s;
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    const std::uint32_t lane = (m & 15u) + 16u * g;
    xs[((b * mtiles + (m >> 4)) * 2u + 0u) * 64u + lane] = __builtin_bit_cast(uint4, hi);
    xs[((b * mtiles + (m >> 4)) * 2u + 1u) * 64u + lane] = __builtin_bit_cast(uint4, lo);
    if (g == 0u) block_sums[b * mp + m] = sum;
}

// K-split partials combined without a reduction launch.  Element e of split
// `split` joins the left-deep chain ((0 + p0) + p1) + ... + p(splits-1) --
// the split-order sum a reduction launch computes -- through the 64-bit
// words slots[i * elems + e], i = 0 .. splits - 2, which are zero between
// launches.  Slot i joins the chain of splits 0..i with p(i+1): each side
// exchanges (float bits << 32 | 1) into it; the one that finds the other's
// word adds the two (IEEE addition is commutative, so the bits do not depend
// on the order of arrival), clears the slot and carries the sum on to slot
// i + 1.  The value and its flag travel in one atomic word, so no fence is
// needed.  Returns true for the caller left holding the whole chain in v.
__device__ __forceinline__ bool chain_combine(std::uint64_t* slots, std::uint64_t elems, std::uint64_t e,
                                              std::uint32_t split, std::uint32_t splits, float& v) {
    if (split == 0u) v = 0.0f + v;
    for (std::uint32_t i = split == 0u ? 0u : split - 1u; i + 1u < splits; ++i) {
        std::uint64_t* slot = slots + static_cast<std::uint64_t>(i) * elems + e;
        const std::uint64_t mine = (static_cast<std::uint64_t>(__float_as_uint(v)) << 32) | 1u;
        const std::uint64_t other = __hip_atomic_exchange(slot, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (other == 0u) return false;
        __hip_atomic_store(slot, std::uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        v = v + __uint_as_float(static_cast<std::uint32_t>(other >> 32));
    }
    return true;
}

} // namespace air_hip

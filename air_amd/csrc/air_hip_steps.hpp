// air_hip_steps.hpp -- per-lane weight codes of one 64-k step (internal).
//
// The GEMM-shaped kernels (prefill, skinny decode) walk K in steps of 64
// (two 32-element blocks) whatever the format's resident tile width: a Q8_0
// tile is one step, a Q4_0 tile two, a Q4_K super-block four.  A lane's
// share of one step of one 16-row tile is its code words plus the scales of
// its row; padded row tiles (rt >= nt) read as codes that decode to zero.
#pragma once

#include "air_hip_device.hpp"

namespace air_hip {

constexpr unsigned kStepK = 64;

template <int FMT>
struct StepCodes;

template <>
struct StepCodes<kQ8_0> {
    u32x4 c;               // bytes of blocks 2kt, 2kt+1
    std::uint32_t d;       // two f16 scales
};
template <>
struct StepCodes<kQ4_0> {
    u32x2 c;               // dwords of blocks 2hs, 2hs+1 of the 128-k tile
    std::uint32_t d;       // their two f16 scales
};
template <>
struct StepCodes<kQ4_K> {
    u32x2 c;               // dwords of sub-blocks 2sub, 2sub+1
    u32x4 h;               // the 16-byte super-block header of the lane's row
};

// Dense storage (F16 / BF16 rows, Q6_K super-block records): a lane's share of
// one 64-k step of one 16-row tile as the prefill GEMM's A fragment (row
// l % 16, elements 8 (l / 16)..+7 of both 32-element blocks).
template <>
struct StepCodes<kF16> {
    u32x4 v[2];            // f16 bits of blocks 0 and 1
};
template <>
struct StepCodes<kBF16> {
    u32x4 v[2];            // bf16 bits of blocks 0 and 1
};
template <>
struct StepCodes<kQ6_K> {
    u32x2 ql[2];           // [block]: the eight low-nibble bytes
    u32x2 qh;              // the eight high-bit-pair bytes (both blocks)
    std::uint32_t sc;      // the step's four int8 sub-block scales
    std::uint32_t d;       // f16 bits of the super-block's d
};

constexpr bool dense_storage(int fmt) { return fmt == kF16 || fmt == kBF16 || fmt == kQ6_K; }

// Rows of a dense matrix of n rows and k columns; rows past n read as zero
// weights.  Q6_K: step s is quadrant pair q = s % 4 of super-block s / 4 --
// half h = q / 2, quadrants j = 2 (q % 2) + b for its blocks b; element
// 8 g + e of a quadrant (half-quadrant g / 2, element i = 8 (g % 2) + e of
// it) has its low nibble (nibble q % 2) and its high pair (bits 2 j) in the
// record's runs for lane group i / 4 and half-quadrant pair 2 h + g / 2
// (linear_dense.hip), its scale in scales byte 8 h + 2 j + g / 2
// (src/reference/tensor_reader.cpp:197-242).
template <int FMT>
__device__ __forceinline__ void load_dense_step(const void* w, std::uint64_t n, std::uint64_t k, std::uint32_t rt,
                                                std::uint32_t s, std::uint32_t lane, StepCodes<FMT>& out) {
    const std::uint64_t row = static_cast<std::uint64_t>(rt) * 16u + (lane & 15u);
    const std::uint32_t g = lane >> 4;
    if constexpr (FMT == kQ6_K) {
        if (row >= n) {
            out.ql[0] = out.ql[1] = out.qh = u32x2{0u, 0u};
            out.sc = 0u;
            out.d = 0u;
            return;
        }
        const std::uint64_t sbs = k / 256u;
        const std::uint64_t blk = row * sbs + s / 4u;
        const unsigned char* rec = static_cast<const unsigned char*>(w) + blk * 208u;
        const std::uint32_t q = s & 3u, h = q >> 1;
        // Runs of lane groups 2 (g % 2) and 2 (g % 2) + 1 (q6k_code_offset).
        const std::uint32_t b = 12u * (2u * h + (g >> 1));
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const std::uint32_t gg = 2u * (g & 1u) + static_cast<std::uint32_t>(r);
            out.ql[0][r] = *reinterpret_cast<const std::uint32_t*>(rec + q6k_code_offset(gg, b));
            out.ql[1][r] = *reinterpret_cast<const std::uint32_t*>(rec + q6k_code_offset(gg, b + 4u));
            out.qh[r] = *reinterpret_cast<const std::uint32_t*>(rec + q6k_code_offset(gg, b + 8u));
        }
        out.sc = *reinterpret_cast<const std::uint32_t*>(rec + 192u + 8u * h + 4u * (q & 1u));
        out.d = reinterpret_cast<const std::uint16_t*>(static_cast<const unsigned char*>(w) + n * sbs * 208u)[blk];
    } else {
        const std::uint64_t k0 = static_cast<std::uint64_t>(s) * kStepK + 8u * g;
        out.v[0] = u32x4{0u, 0u, 0u, 0u};
        out.v[1] = u32x4{0u, 0u, 0u, 0u};
        if (row < n) {
            const std::uint16_t* base = static_cast<const std::uint16_t*>(w) + row * k;
            if (k0 < k) out.v[0] = *reinterpret_cast<const u32x4*>(base + k0);
            if (k0 + 32u < k) out.v[1] = *reinterpret_cast<const u32x4*>(base + k0 + 32u);
        }
    }
}

// Streaming (read-once) code loads use non-temporal hints so they do not
// displace reused data in the caches; NT = false for kernels whose
// workgroups share weight tiles through L2.  Only Q8_0 takes the hint: a
// Q4_0 / Q4_K step reads half of each lane's 16-byte record and the next
// step the other half, which a streaming hint would evict in between.
template <typename T, bool NT>
__device__ __forceinline__ T load_code(const T* p) {
    if constexpr (NT) {
        return __builtin_nontemporal_load(p);
    } else {
        return *p;
    }
}

template <int FMT, bool NT = false>
__device__ __forceinline__ void load_step(const void* codes, const void* scales, std::uint32_t rt, std::uint32_t kt_count,
                                          std::uint32_t s, std::uint32_t lane, bool live, StepCodes<FMT>& out) {
    if constexpr (FMT == kQ8_0) {
        if (!live) { out.c = u32x4{0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u}; out.d = 0u; return; }
        const std::uint64_t tile = static_cast<std::uint64_t>(rt) * kt_count + s;
        out.c = load_code<u32x4, NT>(static_cast<const u32x4*>(codes) + tile * 64u + lane);
        out.d = static_cast<const std::uint32_t*>(scales)[tile * 16u + (lane & 15u)];
    } else if constexpr (FMT == kQ4_0) {
        if (!live) { out.c = u32x2{0x88888888u, 0x88888888u}; out.d = 0u; return; }
        const std::uint64_t tile = static_cast<std::uint64_t>(rt) * kt_count + (s >> 1);
        const u32x2* rec = static_cast<const u32x2*>(codes) + (tile * 64u + lane) * 2u + (s & 1u);
        out.c = *rec;
        out.d = static_cast<const std::uint32_t*>(scales)[(tile * 16u + (lane & 15u)) * 2u + (s & 1u)];
    } else {
        if (!live) { out.c = u32x2{0u, 0u}; out.h = u32x4{0u, 0u, 0u, 0u}; return; }
        const std::uint64_t tile = static_cast<std::uint64_t>(rt) * kt_count + (s >> 2);
        const std::uint32_t sub = s & 3u;
        const u32x2* rec = static_cast<const u32x2*>(codes) + ((tile * 2u + (sub >> 1)) * 64u + lane) * 2u + (sub & 1u);
        out.c = *rec;
        out.h = static_cast<const u32x4*>(scales)[tile * 16u + (lane & 15u)];
    }
}

// Exact codes of block b (0, 1) of the step as f16 operand fragments
// (lane: row l%16, k 8(l/16)+e): Q8_0 q, Q4_0 n-8, Q4_K n.
template <int FMT>
__device__ __forceinline__ half8v step_codes(const StepCodes<FMT>& in, int b) {
    if constexpr (FMT == kQ8_0) {
        half2v p0, p1, p2, p3;
        q8_dword_to_half(b == 0 ? in.c.x : in.c.z, p0, p1);
        q8_dword_to_half(b == 0 ? in.c.y : in.c.w, p2, p3);
        half8v w;
        w[0] = p0[0]; w[1] = p0[1]; w[2] = p1[0]; w[3] = p1[1];
        w[4] = p2[0]; w[5] = p2[1]; w[6] = p3[0]; w[7] = p3[1];
        return w;
    } else if constexpr (FMT == kQ4_0) {
        return nibble_dword_to_half8<8>(b == 0 ? in.c.x : in.c.y);
    } else {
        return nibble_dword_to_half8<0>(b == 0 ? in.c.x : in.c.y);
    }
}

__device__ __forceinline__ float f16_bits_value(std::uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(bits16)));
}

// f32 factors of block b of step s for the lane's row: w = scale * code - offset
// (offset is zero except for Q4_K, where scale = d*sc_j and offset = dmin*m_j).
template <int FMT>
__device__ __forceinline__ void step_scale(const StepCodes<FMT>& in, std::uint32_t s, int b, float& scale,
                                           float& offset) {
    if constexpr (FMT == kQ4_K) {
        // Sub-block j = 2(s mod 4) + b: the four-byte word of its half of the
        // super-block (the same for both blocks of the step), then its byte.
        const std::uint32_t packed[3] = {in.h.y, in.h.z, in.h.w};
        const std::uint32_t j = 2u * (s & 3u) + static_cast<std::uint32_t>(b);
        std::uint32_t scales = 0, mins = 0;
        q4k_scale_min_x4(packed, j >= 4u, scales, mins);
        const std::uint32_t shift = 8u * (j & 3u);
        scale = f16_bits_value(in.h.x & 0xffffu) * static_cast<float>((scales >> shift) & 0xffu);
        offset = f16_bits_value(in.h.x >> 16) * static_cast<float>((mins >> shift) & 0xffu);
    } else {
        scale = f16_bits_value((in.d >> (16 * b)) & 0xffffu);
        offset = 0.0f;
    }
}

} // namespace air_hip

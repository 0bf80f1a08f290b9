// air_hip_layout.hpp -- GGUF block formats and the resident tile layouts.
//
// Canonical GGUF blocks (the bytes a GGUF file holds, decoded by
// src/reference/tensor_reader.cpp:85-196 and src/cuda/cuda_backend.cu:249-307):
//   Q8_0  32 elements / 34 B : [d f16][32 x int8 q]              w = d*q
//   Q4_0  32 elements / 18 B : [d f16][16 B nibbles]             w = d*(n-8)
//         byte i holds element i (low nibble) and i+16 (high nibble)
//   Q4_K 256 elements / 144 B: [d f16][dmin f16][12 B 6-bit scales/mins][128 B nibbles]
//         sub-block j (32 elements): w = (d*sc_j)*n - dmin*m_j
//
// Resident ("wavefront tile") layout.  A matrix with GGML dims {K, N} (N rows
// of K) is cut into row tiles of 16 rows and k tiles; every k tile of every
// row tile is one contiguous record that a 64-lane wavefront fetches with one
// 16-byte load per lane (Q4_K: two).  Lane l serves row (l % 16) of the tile
// and the eight consecutive k positions 8*(l/16)..+7 of each 32-element
// block, which is exactly the B-operand fragment of the CDNA4 MFMA
// v_mfma_f32_16x16x32_f16 (B[k][n], k = 8*(l/16)+e, n = l%16).  Rows and k
// are zero-padded to whole tiles (padded codes decode to 0 with scale 0).
//
//   Q8_0 tile = 16 rows x 64 k (2 blocks)
//     codes  [NT][KT][64 lanes][16 B]   bytes 0-7: block 2kt, k = 8g+e
//                                       bytes 8-15: block 2kt+1, k = 32+8g+e
//            each byte is u = q ^ 0x80 (= q + 128), so f16(0x6400|u) = 1024+u
//     scales [NT][KT][16 rows][2] f16   (d of the two blocks)
//   Q4_0 tile = 16 rows x 128 k (4 blocks)
//     codes  [NT][KT][64 lanes][4 dwords]  dword j: block 4kt+j, 8 nibbles
//            n(e) at bit NIBBLE_POS[e] = {0,16,4,20,8,24,12,28} for e = 0..7
//     scales [NT][KT][16 rows][4] f16
//   Q4_K tile = 16 rows x 256 k (1 super-block)
//     codes  [NT][KT][2 halves][64 lanes][4 dwords]  dword j of half h:
//            sub-block 4h+j, nibble placement as Q4_0
//     scales [NT][KT][16 rows][16 B]    the block's first 16 bytes verbatim
//            (d, dmin, 12 B packed 6-bit scales and mins)
//
// The nibble placement lets one v_and_or_b32 turn a dword into a pair of f16
// values: bits 0-3 / 16-19 under exponent 0x6400 give 1024+n, bits 4-7 /
// 20-23 under 0x5400 give 64+n; a shift by 8 serves the other four.
#pragma once

#include <cstdint>

namespace air_hip {

enum GgmlType : int {
    kF32 = 0,
    kF16 = 1,
    kQ4_0 = 2,
    kQ5_0 = 6,
    kQ8_0 = 8,
    kQ4_K = 12,
    kQ6_K = 14,
    kBF16 = 30,
};

struct FormatGeometry {
    std::uint32_t block_elements;  // canonical block
    std::uint32_t block_bytes;
    std::uint32_t tile_k;          // k per resident tile
    std::uint32_t code_tile_bytes; // per 16-row tile per k tile
    std::uint32_t scale_tile_bytes;
};

constexpr std::uint32_t kTileRows = 16;

constexpr FormatGeometry geometry_of(int type) {
    switch (type) {
    case kQ8_0: return {32, 34, 64, 1024, 64};
    case kQ4_0: return {32, 18, 128, 1024, 128};
    case kQ4_K: return {256, 144, 256, 2048, 256};
    default: return {0, 0, 0, 0, 0};
    }
}

constexpr bool supported_type(int type) { return geometry_of(type).block_elements != 0; }

// Canonical (GGUF) block of every encoding a matrix may arrive in: the three
// with a resident tile format, Q5_0 (rewritten exactly as Q8_0 blocks) and
// the dense ones (decoded once into f32 rows).
struct CanonicalBlock {
    std::uint32_t elements;
    std::uint32_t bytes;
};

constexpr CanonicalBlock canonical_block(int type) {
    switch (type) {
    case kF32: return {1, 4};
    case kF16: return {1, 2};
    case kBF16: return {1, 2};
    case kQ4_0: return {32, 18};
    case kQ5_0: return {32, 22};
    case kQ8_0: return {32, 34};
    case kQ4_K: return {256, 144};
    case kQ6_K: return {256, 210};
    default: return {0, 0};
    }
}

// Held as dense f32 rows [n][k] (no resident tile format for them).
constexpr bool dense_type(int type) { return type == kF32 || type == kF16 || type == kBF16 || type == kQ6_K; }

constexpr std::uint64_t ceil_div(std::uint64_t a, std::uint64_t b) { return (a + b - 1) / b; }

// Bit position of element e (0..7) of a lane's eight-element run inside one
// nibble dword (4-bit formats).
constexpr std::uint32_t kNibblePos[8] = {0, 16, 4, 20, 8, 24, 12, 28};

} // namespace air_hip

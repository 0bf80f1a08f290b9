// repack.hip -- canonical GGUF blocks <-> resident wavefront tiles, and the
// bit-exact f32 decoders over both.
//
// The repack runs once when a matrix becomes resident (the analogue of the
// per-tensor upload in Impl::initialize, src/cuda/cuda_backend.cu:1790-1822).
// The decoders restate decode_all (src/reference/tensor_reader.cpp:85-196):
// every dequantised value is the same f32 product the reference forms, so the
// results are bit-identical.
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"

namespace air_hip {
namespace {

constexpr unsigned kThreads = 256;

unsigned grid_for(std::uint64_t work) {
    const std::uint64_t blocks = ceil_div(work, kThreads);
    return static_cast<unsigned>(blocks < 65535u * 16u ? blocks : 65535u * 16u);
}

__device__ __forceinline__ std::uint32_t rd16(const std::uint8_t* p) {
    return static_cast<std::uint32_t>(p[0]) | (static_cast<std::uint32_t>(p[1]) << 8);
}

// Q8_0: tile 16 rows x 64 k.  One thread per (row tile, k tile, lane).
__global__ void repack_q8_0_kernel(const std::uint8_t* src, std::uint64_t K, std::uint64_t N,
                                   std::uint32_t NT, std::uint32_t KT,
                                   uint4* codes, std::uint32_t* scales) {
    const std::uint64_t total = static_cast<std::uint64_t>(NT) * KT * 64u;
    const std::uint64_t blocks = K / 32u;
    const std::uint64_t row_bytes = blocks * 34u;
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
        const std::uint32_t lane = static_cast<std::uint32_t>(i & 63u);
        const std::uint64_t tile = i >> 6;
        const std::uint32_t kt = static_cast<std::uint32_t>(tile % KT);
        const std::uint64_t nt = tile / KT;
        const std::uint32_t r = lane & 15u, g = lane >> 4;
        const std::uint64_t n = nt * 16u + r;
        std::uint32_t w[4];
        std::uint32_t d[2];
        for (std::uint32_t hb = 0; hb < 2; ++hb) {
            const std::uint64_t b = 2u * static_cast<std::uint64_t>(kt) + hb;
            const bool live = n < N && b < blocks;
            const std::uint8_t* blk = src + n * row_bytes + b * 34u;
            d[hb] = live ? rd16(blk) : 0u;
            for (std::uint32_t half = 0; half < 2; ++half) {
                std::uint32_t v = 0;
                for (std::uint32_t e = 0; e < 4; ++e) {
                    const std::uint32_t code = live ? (blk[2u + 8u * g + 4u * half + e] ^ 0x80u) : 0x80u;
                    v |= code << (8u * e);
                }
                w[2u * hb + half] = v;
            }
        }
        codes[i] = make_uint4(w[0], w[1], w[2], w[3]);
        if (g == 0u) scales[tile * 16u + r] = d[0] | (d[1] << 16);
    }
}

// Element kl (0..31) of a canonical Q4_0 block: byte kl%16, low nibble for kl<16.
__device__ __forceinline__ std::uint32_t q4_0_nibble(const std::uint8_t* qs, std::uint32_t kl) {
    const std::uint32_t byte = qs[kl & 15u];
    return kl < 16u ? (byte & 0x0fu) : (byte >> 4);
}

// Q4_0: tile 16 rows x 128 k (4 blocks).
__global__ void repack_q4_0_kernel(const std::uint8_t* src, std::uint64_t K, std::uint64_t N,
                                   std::uint32_t NT, std::uint32_t KT,
                                   uint4* codes, uint2* scales) {
    const std::uint64_t total = static_cast<std::uint64_t>(NT) * KT * 64u;
    const std::uint64_t blocks = K / 32u;
    const std::uint64_t row_bytes = blocks * 18u;
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
        const std::uint32_t lane = static_cast<std::uint32_t>(i & 63u);
        const std::uint64_t tile = i >> 6;
        const std::uint32_t kt = static_cast<std::uint32_t>(tile % KT);
        const std::uint64_t nt = tile / KT;
        const std::uint32_t r = lane & 15u, g = lane >> 4;
        const std::uint64_t n = nt * 16u + r;
        std::uint32_t w[4], d[4];
        for (std::uint32_t j = 0; j < 4; ++j) {
            const std::uint64_t b = 4u * static_cast<std::uint64_t>(kt) + j;
            const bool live = n < N && b < blocks;
            const std::uint8_t* blk = src + n * row_bytes + b * 18u;
            d[j] = live ? rd16(blk) : 0u;
            std::uint32_t v = 0;
            for (std::uint32_t e = 0; e < 8; ++e) {
                const std::uint32_t nib = live ? q4_0_nibble(blk + 2, 8u * g + e) : 8u;
                v |= nib << kNibblePos[e];
            }
            w[j] = v;
        }
        codes[i] = make_uint4(w[0], w[1], w[2], w[3]);
        if (g == 0u) scales[tile * 16u + r] = make_uint2(d[0] | (d[1] << 16), d[2] | (d[3] << 16));
    }
}

// Q4_K: tile 16 rows x 256 k (one super-block); two uint4 per lane.
__global__ void repack_q4_k_kernel(const std::uint8_t* src, std::uint64_t K, std::uint64_t N,
                                   std::uint32_t NT, std::uint32_t KT,
                                   uint4* codes, uint4* scales) {
    const std::uint64_t total = static_cast<std::uint64_t>(NT) * KT * 64u;
    const std::uint64_t blocks = K / 256u;
    const std::uint64_t row_bytes = blocks * 144u;
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
        const std::uint32_t lane = static_cast<std::uint32_t>(i & 63u);
        const std::uint64_t tile = i >> 6;
        const std::uint32_t kt = static_cast<std::uint32_t>(tile % KT);
        const std::uint64_t nt = tile / KT;
        const std::uint32_t r = lane & 15u, g = lane >> 4;
        const std::uint64_t n = nt * 16u + r;
        const bool live = n < N && kt < blocks;
        const std::uint8_t* blk = src + n * row_bytes + static_cast<std::uint64_t>(kt) * 144u;
        std::uint32_t w[8];
        for (std::uint32_t j = 0; j < 8; ++j) {
            // sub-block j: 64-element group j/2, low nibbles for even j
            std::uint32_t v = 0;
            for (std::uint32_t e = 0; e < 8; ++e) {
                std::uint32_t nib = 0;
                if (live) {
                    const std::uint32_t byte = blk[16u + (j >> 1) * 32u + 8u * g + e];
                    nib = (j & 1u) ? (byte >> 4) : (byte & 0x0fu);
                }
                v |= nib << kNibblePos[e];
            }
            w[j] = v;
        }
        const std::uint64_t base = (tile * 2u) * 64u + lane;
        codes[base] = make_uint4(w[0], w[1], w[2], w[3]);
        codes[base + 64u] = make_uint4(w[4], w[5], w[6], w[7]);
        if (g == 0u) {
            std::uint32_t s[4] = {0, 0, 0, 0};
            if (live) {
                for (std::uint32_t q = 0; q < 16; ++q) s[q >> 2] |= static_cast<std::uint32_t>(blk[q]) << (8u * (q & 3u));
            }
            scales[tile * 16u + r] = make_uint4(s[0], s[1], s[2], s[3]);
        }
    }
}

// ---- decode of the resident tiles --------------------------------------

__global__ void dequantize_tiles_kernel(int type, const void* codes_, const void* scales_,
                                        std::uint64_t K, std::uint64_t N,
                                        std::uint32_t NT, std::uint32_t KT, float* out) {
    const std::uint64_t total = static_cast<std::uint64_t>(NT) * KT * 64u;
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; i < total;
         i += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
        const std::uint32_t lane = static_cast<std::uint32_t>(i & 63u);
        const std::uint64_t tile = i >> 6;
        const std::uint32_t kt = static_cast<std::uint32_t>(tile % KT);
        const std::uint64_t nt = tile / KT;
        const std::uint32_t r = lane & 15u, g = lane >> 4;
        const std::uint64_t n = nt * 16u + r;
        if (n >= N) continue;
        float* row = out + n * K;
        if (type == kQ8_0) {
            const uint4 c = static_cast<const uint4*>(codes_)[i];
            const std::uint32_t sc = static_cast<const std::uint32_t*>(scales_)[tile * 16u + r];
            const std::uint32_t cw[4] = {c.x, c.y, c.z, c.w};
            for (std::uint32_t hb = 0; hb < 2; ++hb) {
                const float d = f16_bits_to_f32((sc >> (16u * hb)) & 0xffffu);
                for (std::uint32_t e = 0; e < 8; ++e) {
                    const std::uint64_t k = 64u * static_cast<std::uint64_t>(kt) + 32u * hb + 8u * g + e;
                    if (k >= K) continue;
                    const std::uint32_t u = (cw[2u * hb + (e >> 2)] >> (8u * (e & 3u))) & 0xffu;
                    const int q = static_cast<int>(u) - 128;
                    row[k] = d * static_cast<float>(q);
                }
            }
        } else if (type == kQ4_0) {
            const uint4 c = static_cast<const uint4*>(codes_)[i];
            const uint2 sc = static_cast<const uint2*>(scales_)[tile * 16u + r];
            const std::uint32_t cw[4] = {c.x, c.y, c.z, c.w};
            const std::uint32_t sw[2] = {sc.x, sc.y};
            for (std::uint32_t j = 0; j < 4; ++j) {
                const float d = f16_bits_to_f32((sw[j >> 1] >> (16u * (j & 1u))) & 0xffffu);
                for (std::uint32_t e = 0; e < 8; ++e) {
                    const std::uint64_t k = 128u * static_cast<std::uint64_t>(kt) + 32u * j + 8u * g + e;
                    if (k >= K) continue;
                    const int q = static_cast<int>((cw[j] >> kNibblePos[e]) & 0x0fu) - 8;
                    row[k] = d * static_cast<float>(q);
                }
            }
        } else {
            const uint4* c4 = static_cast<const uint4*>(codes_);
            const uint4 c0 = c4[(tile * 2u) * 64u + lane];
            const uint4 c1 = c4[(tile * 2u) * 64u + lane + 64u];
            const uint4 sc = static_cast<const uint4*>(scales_)[tile * 16u + r];
            const std::uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
            const float d = f16_bits_to_f32(sc.x & 0xffffu);
            const float dmin = f16_bits_to_f32(sc.x >> 16);
            const std::uint32_t packed[3] = {sc.y, sc.z, sc.w};
            for (std::uint32_t j = 0; j < 8; ++j) {
                std::uint32_t s = 0, m = 0;
                q4k_scale_min(packed, j, s, m);
                const float dj = d * static_cast<float>(s);
                const float mj = dmin * static_cast<float>(m);
                for (std::uint32_t e = 0; e < 8; ++e) {
                    const std::uint64_t k = 256u * static_cast<std::uint64_t>(kt) + 32u * j + 8u * g + e;
                    const float q = static_cast<float>((cw[j] >> kNibblePos[e]) & 0x0fu);
                    row[k] = dj * q - mj;
                }
            }
        }
    }
}

// ---- decode of canonical blocks (decode_element, cuda_backend.cu:241-344) --

__global__ void dequantize_canonical_kernel(int type, const std::uint8_t* src, std::uint64_t blocks,
                                            float* out) {
    for (std::uint64_t b = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; b < blocks;
         b += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
        if (type == kQ8_0) {
            const std::uint8_t* blk = src + b * 34u;
            const float d = f16_bits_to_f32(rd16(blk));
            for (std::uint32_t i = 0; i < 32; ++i) {
                out[b * 32u + i] = d * static_cast<float>(static_cast<std::int8_t>(blk[2 + i]));
            }
        } else if (type == kQ4_0) {
            const std::uint8_t* blk = src + b * 18u;
            const float d = f16_bits_to_f32(rd16(blk));
            for (std::uint32_t i = 0; i < 16; ++i) {
                const std::uint32_t p = blk[2 + i];
                out[b * 32u + i] = d * static_cast<float>(static_cast<int>(p & 0x0fu) - 8);
                out[b * 32u + i + 16u] = d * static_cast<float>(static_cast<int>(p >> 4) - 8);
            }
        } else if (type == kQ4_K) {
            const std::uint8_t* blk = src + b * 144u;
            const float d = f16_bits_to_f32(rd16(blk));
            const float dmin = f16_bits_to_f32(rd16(blk + 2));
            std::uint32_t packed[3] = {0, 0, 0};
            for (std::uint32_t q = 0; q < 12; ++q) packed[q >> 2] |= static_cast<std::uint32_t>(blk[4 + q]) << (8u * (q & 3u));
            for (std::uint32_t grp = 0; grp < 4; ++grp) {
                std::uint32_t s0, m0, s1, m1;
                q4k_scale_min(packed, 2u * grp, s0, m0);
                q4k_scale_min(packed, 2u * grp + 1u, s1, m1);
                const float d0 = d * static_cast<float>(s0), mm0 = dmin * static_cast<float>(m0);
                const float d1 = d * static_cast<float>(s1), mm1 = dmin * static_cast<float>(m1);
                for (std::uint32_t i = 0; i < 32; ++i) {
                    const std::uint32_t p = blk[16u + grp * 32u + i];
                    out[b * 256u + grp * 64u + i] = d0 * static_cast<float>(p & 0x0fu) - mm0;
                    out[b * 256u + grp * 64u + 32u + i] = d1 * static_cast<float>(p >> 4) - mm1;
                }
            }
        } else if (type == kQ5_0) {   // [d:f16][qh:4][qs:16]; element i's fifth bit is bit i of qh
            const std::uint8_t* blk = src + b * 22u;
            const float d = f16_bits_to_f32(rd16(blk));
            const std::uint32_t qh = rd16(blk + 2) | (rd16(blk + 4) << 16);
            for (std::uint32_t i = 0; i < 16; ++i) {
                const std::uint32_t p = blk[6 + i];
                const int q0 = static_cast<int>((p & 0x0fu) | (((qh >> i) & 1u) << 4)) - 16;
                const int q1 = static_cast<int>((p >> 4) | (((qh >> (i + 16u)) & 1u) << 4)) - 16;
                out[b * 32u + i] = d * static_cast<float>(q0);
                out[b * 32u + i + 16u] = d * static_cast<float>(q1);
            }
        } else if (type == kQ6_K) {   // [ql:128][qh:64][scales:16 x int8][d:f16], two halves of 128
            const std::uint8_t* blk = src + b * 210u;
            const float d = f16_bits_to_f32(rd16(blk + 208));
            for (std::uint32_t half = 0; half < 2; ++half) {
                const std::uint8_t* lo = blk + 64u * half;
                const std::uint8_t* hi = blk + 128u + 32u * half;
                const auto* sc = reinterpret_cast<const std::int8_t*>(blk + 192u + 8u * half);
                float* h = out + b * 256u + 128u * half;
                for (std::uint32_t i = 0; i < 32; ++i) {
                    const std::uint32_t pair = i / 16u;
                    // Element i + 32 j: nibble j >> 1 of lo[i + 32 (j & 1)],
                    // high bits 2j..2j+1 of hi[i]; scale sc[pair + 2j].
                    for (std::uint32_t j = 0; j < 4; ++j) {
                        const std::uint32_t l = lo[i + 32u * (j & 1u)];
                        const std::uint32_t nib = (j >> 1) ? (l >> 4) : (l & 0x0fu);
                        const int q = static_cast<int>(nib | (((hi[i] >> (2u * j)) & 3u) << 4)) - 32;
                        // (d * scale) * q, the order of decode_element
                        h[i + 32u * j] = d * static_cast<float>(sc[pair + 2u * j]) * static_cast<float>(q);
                    }
                }
            }
        } else if (type == kF32) {
            std::uint32_t bits = rd16(src + 4u * b) | (rd16(src + 4u * b + 2u) << 16);
            out[b] = __uint_as_float(bits);
        } else if (type == kF16) {
            out[b] = f16_bits_to_f32(rd16(src + 2u * b));
        } else if (type == kBF16) {
            out[b] = __uint_as_float(rd16(src + 2u * b) << 16);
        }
    }
}

// Q5_0 blocks rewritten as Q8_0 blocks of the same values: the scale is
// kept and each 5-bit code q becomes the int8 q - 16, so d * (q - 16) is
// unchanged bit for bit.
__global__ void q5_0_to_q8_0_kernel(const std::uint8_t* __restrict__ src, std::uint64_t blocks,
                                    std::uint8_t* __restrict__ dst) {
    for (std::uint64_t b = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x; b < blocks;
         b += static_cast<std::uint64_t>(gridDim.x) * blockDim.x) {
        const std::uint8_t* blk = src + b * 22u;
        std::uint8_t* out = dst + b * 34u;
        out[0] = blk[0];
        out[1] = blk[1];
        const std::uint32_t qh = rd16(blk + 2) | (rd16(blk + 4) << 16);
        for (std::uint32_t i = 0; i < 16; ++i) {
            const std::uint32_t p = blk[6 + i];
            const int q0 = static_cast<int>((p & 0x0fu) | (((qh >> i) & 1u) << 4)) - 16;
            const int q1 = static_cast<int>((p >> 4) | (((qh >> (i + 16u)) & 1u) << 4)) - 16;
            out[2 + i] = static_cast<std::uint8_t>(static_cast<std::int8_t>(q0));
            out[18 + i] = static_cast<std::uint8_t>(static_cast<std::int8_t>(q1));
        }
    }
}

} // namespace

hipError_t launch_repack(const TilePlanes& p, const std::uint8_t* canonical, hipStream_t stream) {
    const std::uint64_t work = static_cast<std::uint64_t>(p.nt) * p.kt * 64u;
    const unsigned grid = grid_for(work);
    switch (p.type) {
    case kQ8_0:
        repack_q8_0_kernel<<<grid, kThreads, 0, stream>>>(canonical, p.k, p.n, p.nt, p.kt,
                                                          static_cast<uint4*>(p.codes),
                                                          static_cast<std::uint32_t*>(p.scales));
        break;
    case kQ4_0:
        repack_q4_0_kernel<<<grid, kThreads, 0, stream>>>(canonical, p.k, p.n, p.nt, p.kt,
                                                          static_cast<uint4*>(p.codes),
                                                          static_cast<uint2*>(p.scales));
        break;
    case kQ4_K:
        repack_q4_k_kernel<<<grid, kThreads, 0, stream>>>(canonical, p.k, p.n, p.nt, p.kt,
                                                          static_cast<uint4*>(p.codes),
                                                          static_cast<uint4*>(p.scales));
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequantize_tiles(const TilePlanes& p, float* out, hipStream_t stream) {
    const std::uint64_t work = static_cast<std::uint64_t>(p.nt) * p.kt * 64u;
    dequantize_tiles_kernel<<<grid_for(work), kThreads, 0, stream>>>(p.type, p.codes, p.scales, p.k, p.n,
                                                                     p.nt, p.kt, out);
    return hipGetLastError();
}

hipError_t launch_dequantize_canonical(int type, const std::uint8_t* canonical, std::uint64_t elements,
                                       float* out, hipStream_t stream) {
    const auto geo = canonical_block(type);
    if (geo.elements == 0) return hipErrorInvalidValue;
    const std::uint64_t blocks = elements / geo.elements;
    if (blocks == 0) return hipSuccess;
    dequantize_canonical_kernel<<<grid_for(blocks), kThreads, 0, stream>>>(type, canonical, blocks, out);
    return hipGetLastError();
}

hipError_t launch_q5_0_to_q8_0(const std::uint8_t* q5_0, std::uint64_t blocks, std::uint8_t* q8_0, hipStream_t stream) {
    if (blocks == 0) return hipSuccess;
    q5_0_to_q8_0_kernel<<<grid_for(blocks), kThreads, 0, stream>>>(q5_0, blocks, q8_0);
    return hipGetLastError();
}

} // namespace air_hip

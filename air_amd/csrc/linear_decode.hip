// linear_decode.hip -- the decode linear: y[m][n] = sum_k w[n][k] x[m][k] for
// M = 1..64 rows (and any M, in 64-row groups), over resident tiles.
//
// Replaces specialized_matvec_kernel and specialized_matmul[_batch_reuse]_kernel
// (src/cuda/cuda_backend.cu:501-606).  The reference decodes every element
// with a per-element switch and accumulates f32 lane partials; here the
// integer codes feed the CDNA4 matrix cores directly:
//
//   * the weight tile is the B operand of v_mfma_f32_16x16x32_f16: integer
//     codes are exact in f16 (two v_perm_b32 / v_and_or_b32 per four codes);
//   * the activations are the A operand, split into f16 hi + lo parts after a
//     power-of-two scale per (row, 32-element block), so x is carried to ~21
//     significant bits and every product is exact in the f32 accumulator;
//   * each 32-element block's MFMA partial is multiplied by its f16 block
//     scale and the activation block's inverse scale in f32 (Q4_K:
//     (d*sc_j)*P - (dmin*m_j)*sum(x_block)), i.e. the reference's per-block
//     dequantisation applied after the dot product.
//
// Relative L2 error against the double-accumulating oracle is ~1e-6.
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"

namespace air_hip {
namespace {

// ---- activation split ----------------------------------------------------

__device__ __forceinline__ std::uint64_t xs_index(std::uint64_t block, std::uint32_t mtiles,
                                                  std::uint32_t tile, std::uint32_t part,
                                                  std::uint32_t lane) {
    return ((block * mtiles + tile) * 2u + part) * 64u + lane;
}

// One thread per (row m, 32-block b, eighth g); the four threads of a block
// are adjacent lanes.  Rows M..mp-1 and blocks past K are written as zeros.
__global__ void __launch_bounds__(256)
split_activations_kernel(const float* __restrict__ x, std::uint32_t M, std::uint64_t K, std::uint64_t nb,
                         std::uint32_t mp, uint4* __restrict__ xs, float* __restrict__ block_sums,
                         float* __restrict__ inv_scale) {
    const std::uint64_t idx = blockIdx.x * static_cast<std::uint64_t>(blockDim.x) + threadIdx.x;
    const std::uint64_t total = static_cast<std::uint64_t>(mp) * nb * 4u;
    const bool in_grid = idx < total;
    const std::uint32_t g = static_cast<std::uint32_t>(idx & 3u);
    const std::uint64_t rest = idx >> 2;
    const std::uint64_t b = in_grid ? rest % nb : 0;
    const std::uint32_t m = in_grid ? static_cast<std::uint32_t>(rest / nb) : 0;
    const bool live = in_grid && m < M && (b * 32u) < K;

    float v[8];
    if (live) {
        const float4* src = reinterpret_cast<const float4*>(x + static_cast<std::uint64_t>(m) * K + b * 32u + 8u * g);
        const float4 a = src[0], c = src[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = 0.0f;
    }
    float amax = 0.0f, sum = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        amax = fmaxf(amax, fabsf(v[e]));
        sum += v[e];
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    sum += __shfl_xor(sum, 1);
    sum += __shfl_xor(sum, 2);
    float s, inv;
    block_scale(amax, s, inv);
    half8v hi, lo;
    split8(v, s, hi, lo);
    if (!in_grid) return;
    const std::uint32_t mtiles = mp / 16u;
    const std::uint32_t lane = (m & 15u) + 16u * g;
    xs[xs_index(b, mtiles, m >> 4, 0, lane)] = __builtin_bit_cast(uint4, hi);
    xs[xs_index(b, mtiles, m >> 4, 1, lane)] = __builtin_bit_cast(uint4, lo);
    if (g == 0u) {
        block_sums[b * mp + m] = sum;
        inv_scale[b * mp + m] = inv;
    }
}

// ---- decode linear ----------------------------------------------------------

__device__ __forceinline__ half8v load_half8(const uint4* p) {
    return __builtin_bit_cast(half8v, *p);
}

__device__ __forceinline__ float half_bits_to_float(std::uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(bits16)));
}

__device__ __forceinline__ half8v q8_codes_to_half8(std::uint32_t d0, std::uint32_t d1) {
    half2v p0, p1, p2, p3;
    q8_dword_to_half(d0, p0, p1);
    q8_dword_to_half(d1, p2, p3);
    half8v out;
    out[0] = p0[0]; out[1] = p0[1]; out[2] = p1[0]; out[3] = p1[1];
    out[4] = p2[0]; out[5] = p2[1]; out[6] = p3[0]; out[7] = p3[1];
    return out;
}

// Split activations of block kb for MT m tiles starting at mt0, with the
// inverse scales of the lane's four output rows (D-layout rows 4*(lane/16)+i).
template <int MT>
struct BlockActivations {
    half8v hi[MT], lo[MT];
    float4v inv[MT];
};

template <int MT>
__device__ __forceinline__ void load_block(BlockActivations<MT>& a, const uint4* __restrict__ xs,
                                           const float* __restrict__ inv_scale, std::uint64_t kb,
                                           std::uint32_t mtiles_total, std::uint32_t mt0, std::uint32_t lane) {
    const std::uint32_t mp = mtiles_total * 16u;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        a.hi[t] = load_half8(xs + xs_index(kb, mtiles_total, mt0 + t, 0, lane));
        a.lo[t] = load_half8(xs + xs_index(kb, mtiles_total, mt0 + t, 1, lane));
        a.inv[t] = *reinterpret_cast<const float4v*>(inv_scale + kb * mp + (mt0 + t) * 16u + 4u * (lane >> 4));
    }
}

// acc[t] += (scale * inv[t]) * (A_t . W) for one 16-row tile and one block.
template <int MT>
__device__ __forceinline__ void block_mfma(const BlockActivations<MT>& a, const half8v& w, float scale,
                                           float4v (&acc)[MT]) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        float4v p = mfma16x16x32(a.hi[t], w, float4v{0.0f, 0.0f, 0.0f, 0.0f});
        p = mfma16x16x32(a.lo[t], w, p);
        acc[t] += (scale * a.inv[t]) * p;
    }
}

// Largest workgroup (in waves) a variant is compiled for: small register
// footprints may split K over up to 16 waves, large ones keep 128+ VGPRs.
constexpr int max_waves(int R, int MT) { return R * MT <= 2 ? 16 : (R * MT <= 4 ? 8 : 4); }

// Workgroup = W waves on the same R row tiles; wave w takes k tiles
// [KT*w/W, KT*(w+1)/W).  blockIdx.y selects a group of MT m tiles.
template <int FMT, int R, int MT>
__global__ void __launch_bounds__(64 * max_waves(R, MT))
decode_linear_kernel(const void* __restrict__ codes_, const void* __restrict__ scales_,
                     const uint4* __restrict__ xs, const float* __restrict__ block_sums,
                     const float* __restrict__ inv_scale, const float* __restrict__ bias,
                     float* __restrict__ y, std::uint32_t M, std::uint64_t N,
                     std::uint32_t NT, std::uint32_t KT, std::uint32_t mtiles_total) {
    extern __shared__ float4v partials[];
    const std::uint32_t lane = threadIdx.x & 63u;
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const std::uint32_t W = blockDim.x >> 6;
    const std::uint32_t rt0 = blockIdx.x * R;
    const std::uint32_t mt0 = blockIdx.y * MT;
    const std::uint32_t mp = mtiles_total * 16u;
    const std::uint32_t kt_begin = static_cast<std::uint32_t>((static_cast<std::uint64_t>(KT) * wave) / W);
    const std::uint32_t kt_end = static_cast<std::uint32_t>((static_cast<std::uint64_t>(KT) * (wave + 1u)) / W);

    float4v acc[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[r][t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    bool row_live[R];
#pragma unroll
    for (int r = 0; r < R; ++r) row_live[r] = (rt0 + r) < NT;

    for (std::uint32_t kt = kt_begin; kt < kt_end; ++kt) {
        if constexpr (FMT == kQ8_0) {
            const uint4* codes = static_cast<const uint4*>(codes_);
            const std::uint32_t* scales = static_cast<const std::uint32_t*>(scales_);
            uint4 c[R];
            std::uint32_t sc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const std::uint64_t tile = static_cast<std::uint64_t>(rt0 + r) * KT + kt;
                c[r] = row_live[r] ? codes[tile * 64u + lane] : make_uint4(0x80808080u, 0x80808080u, 0x80808080u, 0x80808080u);
                sc[r] = row_live[r] ? scales[tile * 16u + (lane & 15u)] : 0u;
            }
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                BlockActivations<MT> a;
                load_block<MT>(a, xs, inv_scale, 2u * static_cast<std::uint64_t>(kt) + b, mtiles_total, mt0, lane);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const half8v w = b == 0 ? q8_codes_to_half8(c[r].x, c[r].y) : q8_codes_to_half8(c[r].z, c[r].w);
                    const float d = half_bits_to_float((sc[r] >> (16 * b)) & 0xffffu);
                    block_mfma<MT>(a, w, d, acc[r]);
                }
            }
        } else if constexpr (FMT == kQ4_0) {
            const uint4* codes = static_cast<const uint4*>(codes_);
            const uint2* scales = static_cast<const uint2*>(scales_);
            uint4 c[R];
            uint2 sc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const std::uint64_t tile = static_cast<std::uint64_t>(rt0 + r) * KT + kt;
                c[r] = row_live[r] ? codes[tile * 64u + lane] : make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
                sc[r] = row_live[r] ? scales[tile * 16u + (lane & 15u)] : make_uint2(0u, 0u);
            }
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                BlockActivations<MT> a;
                load_block<MT>(a, xs, inv_scale, 4u * static_cast<std::uint64_t>(kt) + b, mtiles_total, mt0, lane);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const std::uint32_t cw = b == 0 ? c[r].x : b == 1 ? c[r].y : b == 2 ? c[r].z : c[r].w;
                    const half8v w = nibble_dword_to_half8<8>(cw);
                    const std::uint32_t sw = b < 2 ? sc[r].x : sc[r].y;
                    const float d = half_bits_to_float((sw >> (16 * (b & 1))) & 0xffffu);
                    block_mfma<MT>(a, w, d, acc[r]);
                }
            }
        } else { // Q4_K
            const uint4* codes = static_cast<const uint4*>(codes_);
            const uint4* scales = static_cast<const uint4*>(scales_);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                if (!row_live[r]) continue;
                const std::uint64_t tile = static_cast<std::uint64_t>(rt0 + r) * KT + kt;
                const uint4 c0 = codes[(tile * 2u) * 64u + lane];
                const uint4 c1 = codes[(tile * 2u) * 64u + 64u + lane];
                const uint4 sc = scales[tile * 16u + (lane & 15u)];
                const float d = half_bits_to_float(sc.x & 0xffffu);
                const float dmin = half_bits_to_float(sc.x >> 16);
                const std::uint32_t packed[3] = {sc.y, sc.z, sc.w};
                const std::uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const std::uint64_t kb = 8u * static_cast<std::uint64_t>(kt) + j;
                    std::uint32_t s6 = 0, m6 = 0;
                    q4k_scale_min(packed, j, s6, m6);
                    const float dj = d * static_cast<float>(s6);
                    const float mj = dmin * static_cast<float>(m6);
                    const half8v w = nibble_dword_to_half8<0>(cw[j]);
                    BlockActivations<MT> a;
                    load_block<MT>(a, xs, inv_scale, kb, mtiles_total, mt0, lane);
                    block_mfma<MT>(a, w, dj, acc[r]);
#pragma unroll
                    for (int t = 0; t < MT; ++t) {
                        const float4v sx = *reinterpret_cast<const float4v*>(
                            block_sums + kb * mp + (mt0 + t) * 16u + 4u * (lane >> 4));
                        acc[r][t] -= mj * sx;
                    }
                }
            }
        }
    }

    // Deterministic cross-wave reduction: wave 0 adds waves 1..W-1 in order.
    if (W > 1u) {
        if (wave > 0u) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int t = 0; t < MT; ++t)
                    partials[((wave - 1u) * (R * MT) + r * MT + t) * 64u + lane] = acc[r][t];
        }
        __syncthreads();
        if (wave == 0u) {
            for (std::uint32_t w = 1; w < W; ++w) {
#pragma unroll
                for (int r = 0; r < R; ++r)
#pragma unroll
                    for (int t = 0; t < MT; ++t)
                        acc[r][t] += partials[((w - 1u) * (R * MT) + r * MT + t) * 64u + lane];
            }
        }
    }
    if (wave != 0u) return;

#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (!row_live[r]) continue;
        const std::uint64_t n = static_cast<std::uint64_t>(rt0 + r) * 16u + (lane & 15u);
        if (n >= N) continue;
        const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const std::uint32_t m0 = (mt0 + t) * 16u + 4u * (lane >> 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const std::uint32_t m = m0 + i;
                if (m < M) y[static_cast<std::uint64_t>(m) * N + n] = acc[r][t][i] + bn;
            }
        }
    }
}

template <int FMT, int R, int MT>
hipError_t launch_variant(const TilePlanes& p, const SplitWorkspace& ws, const float* bias, float* y,
                          std::uint32_t M, std::uint32_t groups, std::uint32_t W, hipStream_t stream) {
    const std::uint32_t mtiles_total = groups * MT;
    const dim3 grid(static_cast<unsigned>(ceil_div(p.nt, R)), groups, 1);
    const std::size_t lds = static_cast<std::size_t>(W - 1u) * R * MT * 64u * sizeof(float4v);
    decode_linear_kernel<FMT, R, MT><<<grid, 64u * W, lds, stream>>>(
        p.codes, p.scales, static_cast<const uint4*>(ws.xs), ws.block_sums, ws.inv_scale, bias, y, M,
        p.n, p.nt, p.kt, mtiles_total);
    return hipGetLastError();
}

template <int FMT, int R>
hipError_t launch_mt(const TilePlanes& p, const SplitWorkspace& ws, const float* bias, float* y,
                     std::uint32_t M, std::uint32_t MT, std::uint32_t groups, std::uint32_t W, hipStream_t s) {
    switch (MT) {
    case 1: return launch_variant<FMT, R, 1>(p, ws, bias, y, M, groups, W, s);
    case 2: return launch_variant<FMT, R, 2>(p, ws, bias, y, M, groups, W, s);
    case 3: return launch_variant<FMT, R, 3>(p, ws, bias, y, M, groups, W, s);
    default: return launch_variant<FMT, R, 4>(p, ws, bias, y, M, groups, W, s);
    }
}

template <int FMT>
hipError_t launch_fmt(const TilePlanes& p, const SplitWorkspace& ws, const float* bias, float* y,
                      std::uint32_t M, std::uint32_t R, std::uint32_t MT, std::uint32_t groups,
                      std::uint32_t W, hipStream_t s) {
    switch (R) {
    case 1: return launch_mt<FMT, 1>(p, ws, bias, y, M, MT, groups, W, s);
    case 2: return launch_mt<FMT, 2>(p, ws, bias, y, M, MT, groups, W, s);
    default: return launch_mt<FMT, 4>(p, ws, bias, y, M, MT, groups, W, s);
    }
}

} // namespace

// m tiles of 16 rows, grouped four at a time.
static void m_partition(std::uint32_t m, std::uint32_t& mt, std::uint32_t& groups) {
    const std::uint32_t tiles = static_cast<std::uint32_t>(ceil_div(m, 16u));
    mt = tiles < 4u ? tiles : 4u;
    groups = static_cast<std::uint32_t>(ceil_div(tiles, mt));
}

std::uint64_t split_workspace_bytes(std::uint64_t kp, std::uint32_t m) {
    std::uint32_t mt = 0, groups = 0;
    m_partition(m, mt, groups);
    const std::uint64_t mp = static_cast<std::uint64_t>(mt) * groups * 16u;
    const std::uint64_t xs = kp * mp * 4u;                // hi + lo f16
    const std::uint64_t per_block = (kp / 32u) * mp * 4u; // one f32 per (block, row)
    return ceil_div(xs, 256u) * 256u + 2u * (ceil_div(per_block, 256u) * 256u);
}

SplitWorkspace carve_split_workspace(void* base, std::uint64_t kp, std::uint32_t m) {
    std::uint32_t mt = 0, groups = 0;
    m_partition(m, mt, groups);
    const std::uint64_t mp = static_cast<std::uint64_t>(mt) * groups * 16u;
    const std::uint64_t per_block = ceil_div((kp / 32u) * mp * 4u, 256u) * 256u;
    auto* p = static_cast<std::uint8_t*>(base);
    SplitWorkspace ws;
    ws.xs = p;
    p += ceil_div(kp * mp * 4u, 256u) * 256u;
    ws.block_sums = reinterpret_cast<float*>(p);
    p += per_block;
    ws.inv_scale = reinterpret_cast<float*>(p);
    return ws;
}

hipError_t launch_split_activations(const float* x, std::uint32_t m, std::uint64_t k, std::uint64_t kp,
                                    const SplitWorkspace& ws, hipStream_t stream) {
    std::uint32_t mt = 0, groups = 0;
    m_partition(m, mt, groups);
    const std::uint32_t mp = mt * groups * 16u;
    const std::uint64_t nb = kp / 32u;
    const std::uint64_t threads = static_cast<std::uint64_t>(mp) * nb * 4u;
    split_activations_kernel<<<static_cast<unsigned>(ceil_div(threads, 256u)), 256, 0, stream>>>(
        x, m, k, nb, mp, static_cast<uint4*>(ws.xs), ws.block_sums, ws.inv_scale);
    return hipGetLastError();
}

hipError_t launch_decode_linear(const TilePlanes& p, const SplitWorkspace& ws, const float* bias, float* y,
                                std::uint32_t m, const DecodeTuning& tuning, hipStream_t stream) {
    std::uint32_t MT = 0, groups = 0;
    m_partition(m, MT, groups);
    // Enough workgroups to cover 256 CUs several times; split K across the
    // waves of a workgroup when the row tiles alone cannot fill the chip.
    std::uint32_t R = 4;
    while (R > 1u && ceil_div(p.nt, R) * groups < 1024u) R >>= 1;
    if (tuning.rows_per_wave == 1u || tuning.rows_per_wave == 2u || tuning.rows_per_wave == 4u) R = tuning.rows_per_wave;
    const std::uint32_t w_cap = static_cast<std::uint32_t>(max_waves(static_cast<int>(R), static_cast<int>(MT)));
    std::uint32_t W = 1;
    const std::uint64_t wgs = ceil_div(p.nt, R) * groups;
    while (W < w_cap && wgs * W < 8192u && p.kt >= 4u * W && (2u * W - 1u) * R * MT <= 64u) W <<= 1;
    if (tuning.waves_per_group != 0u) {
        // Clamped to what the variant is compiled for and to the LDS partials.
        W = tuning.waves_per_group < w_cap ? tuning.waves_per_group : w_cap;
        while (W > 1u && (W - 1u) * R * MT > 63u) --W;
    }
    switch (p.type) {
    case kQ8_0: return launch_fmt<kQ8_0>(p, ws, bias, y, m, R, MT, groups, W, stream);
    case kQ4_0: return launch_fmt<kQ4_0>(p, ws, bias, y, m, R, MT, groups, W, stream);
    case kQ4_K: return launch_fmt<kQ4_K>(p, ws, bias, y, m, R, MT, groups, W, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace air_hip

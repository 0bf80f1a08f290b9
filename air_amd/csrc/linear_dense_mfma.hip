// linear_dense_mfma.hip -- linears over dense rows (F16, BF16, Q6_K) on the
// matrix cores, for any number of activation rows.
//
// The encodings without a tile format of their own stay resident as the
// file's rows (F16, BF16: 2 bytes per weight; Q6_K: 208-byte super-block
// records plus a plane of f16 d, linear_dense.hip).  Here their weights are
// MFMA operands as they are loaded, with the wave-split arrangement of the
// decode kernel (linear_wsplit.hip): a workgroup owns TN 16-row weight tiles
// and up to 64 activation rows (four 16-row tiles), its waves split K, every
// wave keeps D - 1 steps of weights in flight in registers, and the waves'
// sums meet in LDS in wave order.  Wider inputs run as one launch per 64
// rows, each reading the weights once.
//
//   F16   the weights are exact f16 B operands of v_mfma_f32_16x16x32_f16;
//         the activations are split into f16 hi + lo under one power-of-two
//         scale per (row, 64-k step), undone once per step.
//   BF16  exact bf16 B operands of v_mfma_f32_16x16x32_bf16; the activations
//         as three bf16 limbs (x = x1 + x2 + x3 to 24 bits, each limb the
//         truncated residual of the previous ones; bf16 has f32's exponent
//         range, so no scale).
//   Q6_K  the 6-bit codes become exact f16 integers q - 32 (1024 + q under
//         the f16 exponent byte 0x64, minus 1056); a 16-weight sub-block is
//         one v_mfma_f32_16x16x16_f16, so its product takes its own scale
//         d * sc (exact in f32: 11 x 8 significant bits) in the f32
//         epilogue; activations as for F16.
//
// Replaces decode_element's per-element F16 / BF16 / Q6_K decode inside the
// reference's matvec and matmul kernels (src/cuda/cuda_backend.cu:241-344,
// 501-606).
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"

namespace air_hip {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));

constexpr unsigned kDStepK = 64;          // k per pipeline step
constexpr std::uint32_t kQ6kRec = 208;    // Q6_K record: [ql 128][qh 64][scales 16]

struct DmArgs {
    const float* x;          // activations [m][k] f32
    std::uint64_t k;
    const unsigned char* w;  // rows (F16 / BF16) or Q6_K records + d plane
    std::uint64_t n;
    std::uint32_t nt;        // 16-row tiles
    const float* bias;
    float* y;                // [m][n]
    std::uint32_t m;         // <= 64
    std::uint32_t groups;
    std::uint32_t steps;     // ceil(k / 64)
};

// One lane's weights of one 16-row tile for one 64-k step.  Lane l serves
// row l % 16 of the tile; F16 / BF16 hold elements 8 (l / 16)..+7 of both
// 32-element blocks (the B fragment of the 16x16x32 MFMAs), Q6_K elements
// 16 h2 + 4 (l / 16)..+3 of both halves h2 of both blocks (16x16x16).
template <int WT>
struct DenseW {
    u32x4 v[2];
};
template <>
struct DenseW<kQ6_K> {
    std::uint32_t ql[2][2];   // [block][half]: four low nibbles (in the nibble of the step's quadrant pair)
    std::uint32_t qh[2];      // [half]: four bytes of high-bit pairs
    std::uint32_t sc;         // the step's four int8 sub-block scales
    std::uint32_t d;          // f16 bits of the super-block's d
};

template <int WT>
__device__ __forceinline__ void load_dense_step(const DmArgs& a, std::uint32_t row, std::uint32_t s, std::uint32_t lane,
                                                DenseW<WT>& out) {
    const std::uint32_t g = lane >> 4;
    if constexpr (WT == kQ6_K) {
        if (row >= a.n) {
            out.ql[0][0] = out.ql[0][1] = out.ql[1][0] = out.ql[1][1] = 0u;
            out.qh[0] = out.qh[1] = 0u;
            out.sc = 0u;
            out.d = 0u;
            return;
        }
        // Step s is quadrant pair q = s % 4 of super-block s / 4: half h =
        // q / 2 of the record, quadrants j = 2 (q % 2) + b for its two
        // blocks b (src/reference/tensor_reader.cpp:197-242).
        const std::uint64_t sbs = a.k / 256u;
        const std::uint64_t blk = static_cast<std::uint64_t>(row) * sbs + s / 4u;
        const unsigned char* rec = a.w + blk * kQ6kRec;
        const std::uint32_t q = s & 3u, h = q >> 1;
        // Group g's runs of half-quadrant pair (h, h2): low nibbles of
        // quadrants with j % 2 = 0, then 1, then high pairs (q6k_code_offset).
#pragma unroll
        for (int h2 = 0; h2 < 2; ++h2) {
            const std::uint32_t b = 12u * (2u * h + h2);
            out.ql[0][h2] = *reinterpret_cast<const std::uint32_t*>(rec + q6k_code_offset(g, b));
            out.ql[1][h2] = *reinterpret_cast<const std::uint32_t*>(rec + q6k_code_offset(g, b + 4u));
            out.qh[h2] = *reinterpret_cast<const std::uint32_t*>(rec + q6k_code_offset(g, b + 8u));
        }
        out.sc = *reinterpret_cast<const std::uint32_t*>(rec + 192u + 8u * h + 4u * (q & 1u));
        const std::uint16_t* dplane = reinterpret_cast<const std::uint16_t*>(a.w + static_cast<std::uint64_t>(a.n) * sbs * kQ6kRec);
        out.d = dplane[blk];
    } else {
        const std::uint64_t k0 = static_cast<std::uint64_t>(s) * kDStepK + 8u * g;
        out.v[0] = u32x4{0u, 0u, 0u, 0u};
        out.v[1] = u32x4{0u, 0u, 0u, 0u};
        if (row < a.n) {
            const std::uint16_t* base = reinterpret_cast<const std::uint16_t*>(a.w) + static_cast<std::uint64_t>(row) * a.k;
            if (k0 < a.k) out.v[0] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + k0));
            if (k0 + 32u < a.k) out.v[1] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(base + k0 + 32u));
        }
    }
}

// The lane's f32 activations of one step for MT tiles: F16 / BF16 elements
// 8 (l / 16)..+7 of each block (v[t][2b], v[t][2b + 1]); Q6_K elements
// 16 h2 + 4 (l / 16)..+3 of each block half (v[t][2b + h2]).
template <int WT, int MT>
struct DenseX {
    float4v v[MT][4];
};

template <int WT, int MT>
__device__ __forceinline__ void load_dense_x(const DmArgs& a, std::uint32_t s, std::uint32_t lane, DenseX<WT, MT>& out) {
    const std::uint32_t g = lane >> 4;
    const std::uint64_t base_k = static_cast<std::uint64_t>(s) * kDStepK;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const std::uint32_t row = static_cast<std::uint32_t>(t) * 16u + (lane & 15u);
        const float4v zero{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q = 0; q < 4; ++q) out.v[t][q] = zero;
        if (row >= a.m) continue;
        const float* xr = a.x + static_cast<std::uint64_t>(row) * a.k;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const std::uint64_t kb = base_k + 32u * b;
            if (kb >= a.k) continue;   // k is a multiple of 32: a block is all in or all out
            if constexpr (WT == kQ6_K) {
                out.v[t][2 * b] = *reinterpret_cast<const float4v*>(xr + kb + 4u * g);
                out.v[t][2 * b + 1] = *reinterpret_cast<const float4v*>(xr + kb + 16u + 4u * g);
            } else {
                out.v[t][2 * b] = *reinterpret_cast<const float4v*>(xr + kb + 8u * g);
                out.v[t][2 * b + 1] = *reinterpret_cast<const float4v*>(xr + kb + 8u * g + 4u);
            }
        }
    }
}

__device__ __forceinline__ float lane_float(float v, std::uint32_t src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(static_cast<int>(src << 2), __builtin_bit_cast(int, v)));
}

// bf16 limb: the upper half of the f32 bits (truncation), as a value and as bits.
__device__ __forceinline__ float bf16_trunc(float v) { return __uint_as_float(__float_as_uint(v) & 0xffff0000u); }
__device__ __forceinline__ std::uint32_t bf16_pair(float lo, float hi) {
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// Four Q6_K codes (low nibbles in `nib` bytes, high-bit pairs in bits 4-5 of
// `hib` bytes) as exact f16 values q - 32.
__device__ __forceinline__ half4v q6_codes(std::uint32_t nib, std::uint32_t hib) {
    const std::uint32_t u = (nib & 0x0f0f0f0fu) | (hib & 0x30303030u);
    const half2v bias = {(_Float16)1056.0f, (_Float16)1056.0f};
    const half2v lo = bits_as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
    const half2v hi = bits_as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
    half4v out;
    out[0] = lo[0]; out[1] = lo[1]; out[2] = hi[0]; out[3] = hi[1];
    return out;
}

template <int WT, int MT, int TN, int D>
__global__ __launch_bounds__(512) void dense_mfma_kernel(DmArgs a) {
    extern __shared__ float4v wave_acc[];   // [W][TN][MT][64]
    const std::uint32_t lane = threadIdx.x & 63u;
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const std::uint32_t W = blockDim.x >> 6;
    const std::uint32_t rt0 = blockIdx.x * TN;
    const std::uint32_t s0 = (a.steps * wave) / W;
    const std::uint32_t nsteps = (a.steps * (wave + 1u)) / W - s0;
    const std::uint32_t drow = 4u * (lane >> 4);

    float4v acc[TN][MT];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    DenseW<WT> wr[D][TN];
    const auto load_w = [&](DenseW<WT>(&dst)[TN], std::uint32_t s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            load_dense_step<WT>(a, (rt0 + static_cast<std::uint32_t>(j)) * 16u + (lane & 15u), s, lane, dst[j]);
        }
    };

    const auto compute = [&](const DenseX<WT, MT>& x, const DenseW<WT>(&w)[TN], std::uint32_t s)
        __attribute__((always_inline)) {
        if constexpr (WT == kBF16) {
            // Three bf16 limbs per activation; the products sum in f32.
            bf16x8 xl[3][2][MT];
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    float v[8] = {x.v[t][2 * b][0], x.v[t][2 * b][1], x.v[t][2 * b][2], x.v[t][2 * b][3],
                                  x.v[t][2 * b + 1][0], x.v[t][2 * b + 1][1], x.v[t][2 * b + 1][2], x.v[t][2 * b + 1][3]};
#pragma unroll
                    for (int l = 0; l < 3; ++l) {
                        float limb[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            limb[e] = bf16_trunc(v[e]);
                            v[e] = v[e] - limb[e];   // exact: the residual of a truncation
                        }
                        const u32x4 bits = {bf16_pair(limb[0], limb[1]), bf16_pair(limb[2], limb[3]),
                                            bf16_pair(limb[4], limb[5]), bf16_pair(limb[6], limb[7])};
                        xl[l][b][t] = __builtin_bit_cast(bf16x8, bits);
                    }
                }
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const bf16x8 wv = __builtin_bit_cast(bf16x8, w[j].v[b]);
#pragma unroll
                    for (int t = 0; t < MT; ++t) {
#pragma unroll
                        for (int l = 0; l < 3; ++l) {
                            acc[j][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xl[l][b][t], wv, acc[j][t], 0, 0, 0);
                        }
                    }
                }
        } else {
            // f16 hi + lo under one power-of-two scale per (row, step).
            half8v hi8[2][MT], lo8[2][MT];
            half4v hi4[4][MT], lo4[4][MT];
            float4v inv4[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                float amax = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(x.v[t][q][e]));
                amax = fmaxf(amax, __shfl_xor(amax, 16));
                amax = fmaxf(amax, __shfl_xor(amax, 32));
                float sc, inv;
                block_scale(amax, sc, inv);
                if constexpr (WT == kQ6_K) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        float e8[8] = {x.v[t][q][0], x.v[t][q][1], x.v[t][q][2], x.v[t][q][3], 0.0f, 0.0f, 0.0f, 0.0f};
                        half8v h, l;
                        split8(e8, sc, h, l);
                        hi4[q][t] = half4v{h[0], h[1], h[2], h[3]};
                        lo4[q][t] = half4v{l[0], l[1], l[2], l[3]};
                    }
                } else {
#pragma unroll
                    for (int b = 0; b < 2; ++b) {
                        const float e8[8] = {x.v[t][2 * b][0], x.v[t][2 * b][1], x.v[t][2 * b][2], x.v[t][2 * b][3],
                                             x.v[t][2 * b + 1][0], x.v[t][2 * b + 1][1], x.v[t][2 * b + 1][2],
                                             x.v[t][2 * b + 1][3]};
                        split8(e8, sc, hi8[b][t], lo8[b][t]);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) inv4[t][i] = lane_float(inv, drow + static_cast<std::uint32_t>(i));
            }
            float4v c[TN][MT];
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int t = 0; t < MT; ++t) c[j][t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if constexpr (WT == kQ6_K) {
                        const std::uint32_t q = s & 3u;
                        const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(w[j].d)));
                        const std::uint32_t quad = 2u * (q & 1u) + static_cast<std::uint32_t>(b);
#pragma unroll
                        for (int h2 = 0; h2 < 2; ++h2) {
                            // Low nibble of ql byte i holds quadrant j for j < 2,
                            // the high nibble quadrant j for j >= 2; the high
                            // pair of quadrant j sits at bits 2j, 2j + 1 of qh.
                            const std::uint32_t lq = w[j].ql[b][h2];
                            const std::uint32_t nib = (quad >> 1) != 0u ? (lq >> 4) : lq;
                            const std::uint32_t hq = w[j].qh[h2];
                            const std::uint32_t hib = 2u * quad <= 4u ? (hq << (4u - 2u * quad)) : (hq >> (2u * quad - 4u));
                            const half4v wq = q6_codes(nib, hib);
                            const int sc8 = static_cast<int>(static_cast<std::int8_t>((w[j].sc >> (8u * (2u * b + h2))) & 0xffu));
                            const float ds = d * static_cast<float>(sc8);
#pragma unroll
                            for (int t = 0; t < MT; ++t) {
                                float4v p = __builtin_amdgcn_mfma_f32_16x16x16f16(hi4[2 * b + h2][t], wq,
                                                                                  float4v{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                                p = __builtin_amdgcn_mfma_f32_16x16x16f16(lo4[2 * b + h2][t], wq, p, 0, 0, 0);
                                c[j][t] += ds * p;
                            }
                        }
                    } else {
                        const half8v wv = __builtin_bit_cast(half8v, w[j].v[b]);
#pragma unroll
                        for (int t = 0; t < MT; ++t) {
                            c[j][t] = mfma16x16x32(hi8[b][t], wv, c[j][t]);
                            c[j][t] = mfma16x16x32(lo8[b][t], wv, c[j][t]);
                        }
                    }
                }
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[j][t] += inv4[t] * c[j][t];
        }
    };

#pragma unroll
    for (int q = 0; q < D - 1; ++q) {
        if (static_cast<std::uint32_t>(q) < nsteps) load_w(wr[q], s0 + q);
    }
    DenseX<WT, MT> xa, xb;
    if (nsteps > 0u) load_dense_x<WT, MT>(a, s0, lane, xa);
    const auto step = [&](std::uint32_t q, auto u_tag, DenseX<WT, MT>& cur, DenseX<WT, MT>& next)
        __attribute__((always_inline)) {
        constexpr int U = decltype(u_tag)::value;
        if (q + D - 1u < nsteps) load_w(wr[(U + D - 1) % D], s0 + q + D - 1u);
        if (q + 1u < nsteps) load_dense_x<WT, MT>(a, s0 + q + 1u, lane, next);
        compute(cur, wr[U], s0 + q);
    };
    for (std::uint32_t q = 0; q < nsteps; q += D) {
        step(q, std::integral_constant<int, 0>{}, xa, xb);
        if (q + 1u >= nsteps) break;
        step(q + 1u, std::integral_constant<int, 1>{}, xb, xa);
        if constexpr (D > 2) {
            if (q + 2u >= nsteps) break;
            step(q + 2u, std::integral_constant<int, 2>{}, xa, xb);
            if (q + 3u >= nsteps) break;
            step(q + 3u, std::integral_constant<int, 3>{}, xb, xa);
        }
    }

    // The waves' sums meet in LDS; wave w adds (tile, activation tile)
    // combinations w, w + W, ... over the waves in order.
    if (W > 1u) {
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int t = 0; t < MT; ++t) wave_acc[((wave * TN + j) * MT + t) * 64u + lane] = acc[j][t];
        __syncthreads();
    }
    for (std::uint32_t cmb = wave; cmb < static_cast<std::uint32_t>(TN * MT); cmb += W) {
        const std::uint32_t j = cmb / MT, t = cmb % MT;
        float4v sum = float4v{0.0f, 0.0f, 0.0f, 0.0f};
        if (W > 1u) {
            sum = wave_acc[(j * MT + t) * 64u + lane];
            for (std::uint32_t w = 1; w < W; ++w) sum += wave_acc[((w * TN + j) * MT + t) * 64u + lane];
        } else {
#pragma unroll
            for (int jj = 0; jj < TN; ++jj)
#pragma unroll
                for (int tt = 0; tt < MT; ++tt)
                    if (static_cast<std::uint32_t>(jj) == j && static_cast<std::uint32_t>(tt) == t) sum = acc[jj][tt];
        }
        const std::uint64_t n = static_cast<std::uint64_t>(rt0 + j) * 16u + (lane & 15u);
        if (n >= a.n) continue;
        const float bn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const std::uint32_t m = t * 16u + drow + static_cast<std::uint32_t>(i);
            if (m < a.m) a.y[static_cast<std::uint64_t>(m) * a.n + n] = sum[i] + bn;
        }
    }
}

template <int WT, int MT, int TN>
hipError_t launch_dm_tn(const DmArgs& a, const DenseMfmaShape& s, hipStream_t stream) {
    const std::size_t lds = s.waves > 1u ? static_cast<std::size_t>(s.waves) * TN * MT * 64u * sizeof(float4v) : 0u;
    if (s.depth >= 4u) {
        hipLaunchKernelGGL((dense_mfma_kernel<WT, MT, TN, 4>), dim3(a.groups), dim3(64u * s.waves), lds, stream, a);
    } else {
        hipLaunchKernelGGL((dense_mfma_kernel<WT, MT, TN, 2>), dim3(a.groups), dim3(64u * s.waves), lds, stream, a);
    }
    return hipGetLastError();
}

template <int WT, int MT>
hipError_t launch_dm_mt(const DmArgs& a, const DenseMfmaShape& s, hipStream_t stream) {
    switch (s.tile_n) {
    case 1: return launch_dm_tn<WT, MT, 1>(a, s, stream);
    case 2: return launch_dm_tn<WT, MT, 2>(a, s, stream);
    default: return launch_dm_tn<WT, MT, 4>(a, s, stream);
    }
}

// Three or four activation tiles (F16 only): one weight tile per workgroup,
// one step in flight (the registers of the wider variants spill).
template <int WT>
hipError_t launch_dm(const DmArgs& a, const DenseMfmaShape& s, std::uint32_t mt, hipStream_t stream) {
    switch (mt) {
    case 1: return launch_dm_mt<WT, 1>(a, s, stream);
    case 2: return launch_dm_mt<WT, 2>(a, s, stream);
    default: break;
    }
    if constexpr (WT == kF16) {
        const std::size_t lds = s.waves > 1u ? static_cast<std::size_t>(s.waves) * mt * 64u * sizeof(float4v) : 0u;
        if (mt == 3u) {
            hipLaunchKernelGGL((dense_mfma_kernel<WT, 3, 1, 2>), dim3(a.groups), dim3(64u * s.waves), lds, stream, a);
        } else {
            hipLaunchKernelGGL((dense_mfma_kernel<WT, 4, 1, 2>), dim3(a.groups), dim3(64u * s.waves), lds, stream, a);
        }
        return hipGetLastError();
    }
    return hipErrorInvalidConfiguration;
}

} // namespace

// Activation rows per launch: 64 for F16, 32 for BF16 and Q6_K (three bf16
// limbs or the Q6_K decode leave no registers for more tiles).
std::uint32_t dense_mfma_rows(int storage) { return storage == kF16 ? 64u : 32u; }

DenseMfmaShape plan_dense_mfma(int storage, std::uint64_t k, std::uint64_t n, std::uint32_t m,
                               const DenseMfmaShape& tuning) {
    DenseMfmaShape s;
    const std::uint32_t rows = m < dense_mfma_rows(storage) ? m : dense_mfma_rows(storage);
    const std::uint32_t mt = static_cast<std::uint32_t>(ceil_div(rows, 16u));
    const std::uint64_t nt = ceil_div(n, 16u);
    const std::uint32_t steps = static_cast<std::uint32_t>(ceil_div(k, kDStepK));
    // Measured on the Qwen2-7B shapes (down 3584 x 18944, gate|up 37888 x
    // 3584, o 3584 x 3584; F16, BF16, Q6_K; M = 16, 32, 64): four weight
    // tiles per workgroup on wide matrices with one activation tile (two for
    // Q6_K, whose decode holds more registers), two with two activation
    // tiles, one with more; eight waves splitting K on grids of <= 512
    // workgroups (down, o), four on wider ones (eight cost gate|up 12 %);
    // one step of weights in flight (three were never faster).
    std::uint32_t tn = tuning.tile_n;
    if (tn == 0u) {
        if (mt == 1u) tn = nt >= 2048u ? (storage == kQ6_K ? 2u : 4u) : nt >= 1024u ? 2u : 1u;
        else tn = nt >= 1024u ? 2u : 1u;
    }
    if (mt == 2u && tn > 2u) tn = 2u;
    if (mt >= 3u) tn = 1u;
    s.tile_n = tn >= 4u ? 4u : tn >= 2u ? 2u : 1u;
    const std::uint64_t groups = ceil_div(nt, s.tile_n);
    std::uint32_t w = tuning.waves;
    if (w == 0u) {
        w = groups <= 512u ? 8u : 4u;
        if (w > steps / 2u) w = steps / 2u;
    }
    s.waves = w < 1u ? 1u : (w > 8u ? 8u : w);
    s.depth = tuning.depth >= 4u ? 4u : 2u;
    if (mt >= 3u || (mt == 2u && s.tile_n == 2u)) s.depth = 2u;
    return s;
}

bool dense_mfma_supported(int storage, std::uint64_t k) {
    if (storage == kF16 || storage == kBF16) return k % 32u == 0u;
    return storage == kQ6_K && k % 256u == 0u;
}

hipError_t launch_dense_mfma(const void* w, int storage, std::uint64_t k, std::uint64_t n, const float* x,
                             const float* bias, float* y, std::uint32_t m, const DenseMfmaShape& tuning,
                             hipStream_t stream) {
    if (m == 0u || n == 0u || !dense_mfma_supported(storage, k)) return hipErrorInvalidValue;
    if (ceil_div(n, 16u) > 0x7fffffffu) return hipErrorInvalidValue;
    // One launch per 64 (F16) or 32 activation rows, each over the whole matrix.
    const std::uint32_t chunk = dense_mfma_rows(storage);
    for (std::uint32_t r0 = 0; r0 < m; r0 += chunk) {
        const std::uint32_t rows = m - r0 < chunk ? m - r0 : chunk;
        const DenseMfmaShape s = plan_dense_mfma(storage, k, n, rows, tuning);
        const std::uint32_t mt = static_cast<std::uint32_t>(ceil_div(rows, 16u));
        DmArgs a{};
        a.x = x + static_cast<std::uint64_t>(r0) * k;
        a.k = k;
        a.w = static_cast<const unsigned char*>(w);
        a.n = n;
        a.nt = static_cast<std::uint32_t>(ceil_div(n, 16u));
        a.bias = bias;
        a.y = y + static_cast<std::uint64_t>(r0) * n;
        a.m = rows;
        a.groups = static_cast<std::uint32_t>(ceil_div(a.nt, s.tile_n));
        a.steps = static_cast<std::uint32_t>(ceil_div(k, kDStepK));
        hipError_t err = hipErrorInvalidValue;
        switch (storage) {
        case kF16: err = launch_dm<kF16>(a, s, mt, stream); break;
        case kBF16: err = launch_dm<kBF16>(a, s, mt, stream); break;
        case kQ6_K: err = launch_dm<kQ6_K>(a, s, mt, stream); break;
        default: break;
        }
        if (err != hipSuccess) return err;
    }
    return hipSuccess;
}

} // namespace air_hip

// linear_wsplit.hip -- the decode linear for M = 2..64 rows with K split over
// the waves of a workgroup.
//
// The same arithmetic contract as the other decode kernels (exact integer
// codes as the f16 B operand of v_mfma_f32_16x16x32_f16, activations split
// into f16 hi + lo under a power-of-two scale, f32 weight-scale epilogue),
// arranged like the M = 1 GEMV rather than like a GEMM:
//
//   * a workgroup owns TN 16-row weight tiles and ALL activation rows; its W
//     waves split K into W contiguous ranges, so each wave streams its own
//     weight codes with no barrier between steps and no LDS on the way;
//   * every wave keeps D - 1 steps of weight codes in flight in registers
//     (the M = 1 GEMV's lesson: the launch streams at the rate of the bytes
//     in flight per CU), and the next step's activations;
//   * the wave's activation fragments come straight from L2 and serve its TN
//     weight tiles (activation bytes per weight byte ~ 4 M / (17 TN));
//   * at the end the waves' partial sums meet in LDS and are added in wave
//     order (fixed order: repeat launches are bit-identical); a K split over
//     workgroups (only for matrices too narrow to fill the GPU) writes
//     partials for the deterministic split reduction.
//
// Two activation sources:
//   XF = true   the f32 rows: each wave splits its own steps with one
//               power-of-two scale per (row, 64-k step), undone once per step
//               (acc += inv * step sum), so a linear is one launch and writes
//               no activation workspace;
//   XF = false  the row-scaled split of split_rows_kernel (one scale per row,
//               undone at the end), for matrices whose many workgroups would
//               repeat the in-kernel split too often.
//
// Replaces specialized_matmul_kernel / specialized_matmul_batch_reuse_kernel
// (src/cuda/cuda_backend.cu:501-583) for batched decode.
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"
#include "air_hip_steps.hpp"

namespace air_hip {
namespace {

struct WsArgs {
    const float* x;              // XF: activations [m][k] f32
    std::uint64_t k;
    const u32x4* xs;             // split activations [block][mt][2][64] x 16 B
    const float* inv_scale;      // [mp] inverse power-of-two scale of each row
    const float* block_sums;     // [block][mp] sums of the scaled values (Q4_K)
    const void* codes;
    const void* scales;
    std::uint32_t nt, kt;
    std::uint64_t n;
    const float* bias;           // fused when K is not split over workgroups
    float* out;                  // y, or partials [splits][m][n]
    std::uint32_t m;
    std::uint32_t groups;
    std::uint32_t steps;
    std::uint32_t steps_per_split;
    std::uint32_t partial;
    // K split combined in the kernel (chain_combine): slots [splits-1][m][n],
    // y and the bias the last arrival adds; null: partials for a reduction.
    std::uint64_t* chain;
    float* y;
    const float* chain_bias;
    std::uint32_t splits;
};

// The activations of one 64-k step for one wave: XF holds the lane's f32
// values (row l % 16 of each tile, elements 8 (l / 16)..+7 of both blocks),
// the split source the hi / lo fragments.
template <int MT, bool XF>
struct StepX {
    float4v v[XF ? MT : 1][XF ? 4 : 1];
    u32x4 f[XF ? 1 : 2][XF ? 1 : MT][XF ? 1 : 2];   // [block][tile][hi, lo]
};

template <int MT, bool XF>
__device__ __forceinline__ void load_step_x(const WsArgs& a, std::uint32_t s, std::uint32_t lane, StepX<MT, XF>& out) {
    if constexpr (XF) {
        const std::uint64_t k0 = static_cast<std::uint64_t>(s) * kStepK + 8u * (lane >> 4);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const std::uint32_t row = static_cast<std::uint32_t>(t) * 16u + (lane & 15u);
            const float4v zero{0.0f, 0.0f, 0.0f, 0.0f};
            out.v[t][0] = zero; out.v[t][1] = zero; out.v[t][2] = zero; out.v[t][3] = zero;
            if (row < a.m) {
                const float4v* src = reinterpret_cast<const float4v*>(a.x + static_cast<std::uint64_t>(row) * a.k + k0);
                if (k0 < a.k) { out.v[t][0] = src[0]; out.v[t][1] = src[1]; }
                if (k0 + 32u < a.k) { out.v[t][2] = src[8]; out.v[t][3] = src[9]; }
            }
        }
    } else {
        // Fragment (block 2s + b, tile t, part) of the workspace: 64 lanes x 16 B.
        const u32x4* base = a.xs + static_cast<std::uint64_t>(s) * (4u * MT) * 64u + lane;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int p = 0; p < 2; ++p) out.f[b][t][p] = base[((b * MT + t) * 2 + p) * 64];
    }
}

// Value of lane `src` (a wave-uniform pattern), as ds_bpermute.
__device__ __forceinline__ float lane_float(float v, std::uint32_t src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute(static_cast<int>(src << 2),
                                                                   __builtin_bit_cast(int, v)));
}

template <int FMT, int MT, int TN, int D, bool XF>
__global__ __launch_bounds__(512) void wsplit_kernel(WsArgs a) {
    extern __shared__ float4v wave_acc[];   // [W][TN][MT][64]
    constexpr bool kSums = FMT == kQ4_K;
    const std::uint32_t lane = threadIdx.x & 63u;
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const std::uint32_t W = blockDim.x >> 6;
    const std::uint32_t group = blockIdx.x % a.groups;
    const std::uint32_t split = blockIdx.x / a.groups;
    const std::uint32_t rt0 = group * TN;
    const std::uint32_t sb = split * a.steps_per_split;
    const std::uint32_t se = min(a.steps, sb + a.steps_per_split);
    const std::uint32_t len = se > sb ? se - sb : 0u;
    const std::uint32_t s0 = sb + (len * wave) / W;
    const std::uint32_t nsteps = sb + (len * (wave + 1u)) / W - s0;
    const std::uint32_t mp = MT * 16u;

    float4v acc[TN][MT];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    bool live[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) live[j] = rt0 + static_cast<std::uint32_t>(j) < a.nt;

    StepCodes<FMT> wr[D][TN];
    const auto load_w = [&](StepCodes<FMT>(&dst)[TN], std::uint32_t s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            load_step<FMT, true>(a.codes, a.scales, rt0 + static_cast<std::uint32_t>(j), a.kt, s, lane, live[j], dst[j]);
        }
    };

    // D-row view: lane l holds output rows 4 (l / 16) + i of each tile.
    const std::uint32_t drow = 4u * (lane >> 4);
    const auto compute = [&](const StepX<MT, XF>& x, const StepCodes<FMT>(&w_in)[TN], std::uint32_t s)
        __attribute__((always_inline)) {
        half8v hi[2][MT], lo[2][MT];
        float4v inv4[MT];
        float4v sum4[2][kSums ? MT : 1];
        if constexpr (XF) {
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const float4v* v = x.v[t];
                float amax = 0.0f;
#pragma unroll
                for (int q = 0; q < 4; ++q)
#pragma unroll
                    for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(v[q][e]));
                amax = fmaxf(amax, __shfl_xor(amax, 16));
                amax = fmaxf(amax, __shfl_xor(amax, 32));
                float sc, inv;
                block_scale(amax, sc, inv);
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const float e8[8] = {v[2 * b][0], v[2 * b][1], v[2 * b][2], v[2 * b][3],
                                         v[2 * b + 1][0], v[2 * b + 1][1], v[2 * b + 1][2], v[2 * b + 1][3]};
                    split8(e8, sc, hi[b][t], lo[b][t]);
                    if constexpr (kSums) {
                        // Scaled block sum of the row, moved to the D rows.
                        float sum = ((e8[0] + e8[1]) + (e8[2] + e8[3])) + ((e8[4] + e8[5]) + (e8[6] + e8[7]));
                        sum += __shfl_xor(sum, 16);
                        sum += __shfl_xor(sum, 32);
                        sum *= sc;
#pragma unroll
                        for (int i = 0; i < 4; ++i) sum4[b][t][i] = lane_float(sum, drow + static_cast<std::uint32_t>(i));
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) inv4[t][i] = lane_float(inv, drow + static_cast<std::uint32_t>(i));
            }
        } else {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    hi[b][t] = __builtin_bit_cast(half8v, x.f[b][t][0]);
                    lo[b][t] = __builtin_bit_cast(half8v, x.f[b][t][1]);
                    if constexpr (kSums) {
                        sum4[b][t] = *reinterpret_cast<const float4v*>(
                            a.block_sums + (2u * static_cast<std::uint64_t>(s) + b) * mp + t * 16u + drow);
                    }
                }
        }
        float4v c[TN][MT];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const half8v w = step_codes<FMT>(w_in[j], b);
                float ws, wo;
                step_scale<FMT>(w_in[j], s, b, ws, wo);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    float4v p = mfma16x16x32(hi[b][t], w, float4v{0.0f, 0.0f, 0.0f, 0.0f});
                    p = mfma16x16x32(lo[b][t], w, p);
                    if constexpr (XF) {
                        c[j][t] = b == 0 ? ws * p : c[j][t] + ws * p;
                        if constexpr (kSums) c[j][t] -= wo * sum4[b][t];
                    } else {
                        acc[j][t] += ws * p;
                        if constexpr (kSums) acc[j][t] -= wo * sum4[b][t];
                    }
                }
            }
        }
        if constexpr (XF) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[j][t] += inv4[t] * c[j][t];
        }
    };

    // Weight codes D - 1 steps ahead, activations one step ahead.
#pragma unroll
    for (int q = 0; q < D - 1; ++q) {
        if (static_cast<std::uint32_t>(q) < nsteps) load_w(wr[q], s0 + q);
    }
    StepX<MT, XF> xa, xb;
    if (nsteps > 0u) load_step_x<MT, XF>(a, s0, lane, xa);
    const auto step = [&](std::uint32_t q, auto u_tag, StepX<MT, XF>& cur, StepX<MT, XF>& next)
        __attribute__((always_inline)) {
        constexpr int U = decltype(u_tag)::value;
        if (q + D - 1u < nsteps) load_w(wr[(U + D - 1) % D], s0 + q + D - 1u);
        if (q + 1u < nsteps) load_step_x<MT, XF>(a, s0 + q + 1u, lane, next);
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
    float4v inv_row[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        inv_row[t] = XF ? float4v{1.0f, 1.0f, 1.0f, 1.0f}
                        : *reinterpret_cast<const float4v*>(a.inv_scale + t * 16u + drow);
    }
    float* out = a.out + (a.partial ? static_cast<std::uint64_t>(split) * a.m * a.n : 0u);
    for (std::uint32_t cmb = wave; cmb < static_cast<std::uint32_t>(TN * MT); cmb += W) {
        const std::uint32_t j = cmb / MT, t = cmb % MT;
        float4v sum;
        if (W > 1u) {
            sum = wave_acc[(j * MT + t) * 64u + lane];
            for (std::uint32_t w = 1; w < W; ++w) sum += wave_acc[((w * TN + j) * MT + t) * 64u + lane];
        } else {
            // One wave: its own registers (cmb is then every combination in turn).
            sum = float4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int jj = 0; jj < TN; ++jj)
#pragma unroll
                for (int tt = 0; tt < MT; ++tt)
                    if (static_cast<std::uint32_t>(jj) == j && static_cast<std::uint32_t>(tt) == t) sum = acc[jj][tt];
        }
        const std::uint64_t n = static_cast<std::uint64_t>(rt0 + j) * 16u + (lane & 15u);
        if (rt0 + j >= a.nt || n >= a.n) continue;
        const float bn = (a.bias && !a.partial) ? a.bias[n] : 0.0f;
        float4v invt = inv_row[0];
#pragma unroll
        for (int tt = 1; tt < MT; ++tt) if (static_cast<std::uint32_t>(tt) == t) invt = inv_row[tt];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const std::uint32_t m = t * 16u + drow + static_cast<std::uint32_t>(i);
            if (m >= a.m) continue;
            const std::uint64_t e = static_cast<std::uint64_t>(m) * a.n + n;
            float v = sum[i] * invt[i] + bn;
            if (a.chain) {
                if (chain_combine(a.chain, static_cast<std::uint64_t>(a.m) * a.n, e, split, a.splits, v)) {
                    a.y[e] = a.chain_bias ? v + a.chain_bias[n] : v;
                }
            } else {
                out[e] = v;
            }
        }
    }
}

template <int FMT, int MT, int TN, bool XF>
hipError_t launch_wsplit_tn(const WsArgs& a, const WsplitShape& s, hipStream_t stream) {
    const unsigned blocks = s.groups * s.splits;
    const std::size_t lds = s.waves > 1u ? static_cast<std::size_t>(s.waves) * TN * MT * 64u * sizeof(float4v) : 0u;
    if (s.depth >= 4u) {
        hipLaunchKernelGGL((wsplit_kernel<FMT, MT, TN, 4, XF>), dim3(blocks), dim3(64u * s.waves), lds, stream, a);
    } else {
        hipLaunchKernelGGL((wsplit_kernel<FMT, MT, TN, 2, XF>), dim3(blocks), dim3(64u * s.waves), lds, stream, a);
    }
    return hipGetLastError();
}

template <int FMT, int MT, bool XF>
hipError_t launch_wsplit_mt(const WsArgs& a, const WsplitShape& s, hipStream_t stream) {
    switch (s.tile_n) {
    case 1: return launch_wsplit_tn<FMT, MT, 1, XF>(a, s, stream);
    case 2: return launch_wsplit_tn<FMT, MT, 2, XF>(a, s, stream);
    default: return launch_wsplit_tn<FMT, MT, 4, XF>(a, s, stream);
    }
}

template <int FMT, bool XF>
hipError_t launch_wsplit_fmt(const WsArgs& a, const WsplitShape& s, hipStream_t stream) {
    switch (s.mt) {
    case 1: return launch_wsplit_mt<FMT, 1, XF>(a, s, stream);
    case 2: return launch_wsplit_mt<FMT, 2, XF>(a, s, stream);
    case 3: return launch_wsplit_mt<FMT, 3, XF>(a, s, stream);
    default: return launch_wsplit_mt<FMT, 4, XF>(a, s, stream);
    }
}

template <bool XF>
hipError_t launch_wsplit_any(int type, const WsArgs& a, const WsplitShape& s, hipStream_t stream) {
    switch (type) {
    case kQ8_0: return launch_wsplit_fmt<kQ8_0, XF>(a, s, stream);
    case kQ4_0: return launch_wsplit_fmt<kQ4_0, XF>(a, s, stream);
    case kQ4_K: return launch_wsplit_fmt<kQ4_K, XF>(a, s, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace

bool wsplit_preferred(const TilePlanes& p, std::uint32_t m) {
    // Measured against the skinny kernels on the Qwen2-7B shapes (graph
    // replay, per linear; Q8_0 / Q4_0 / Q4_K at M = 8, 16, 32, 64):
    //  * one activation tile (M <= 16): faster on q|k|v, o, gate|up and
    //    down in every format (down 30.1 -> 23.6 us at M = 8 in Q8_0, gate|up
    //    39.3 -> 34.1, o 12.4 -> 10.7 at M = 16), except Q4_K q|k|v (even at
    //    M = 8, 3 % slower at M = 16);
    //  * two activation tiles: faster on the matrices of <= 256 row tiles (o
    //    16.4 -> 14.4 us, down 37.9 -> 36.0 in Q8_0, 36.3 -> 33.3 in Q4_0);
    //    the wide ones keep the LDS pipeline, which shares each step's
    //    activations among four waves (gate|up 43.8 against 48.2);
    //  * three or four: only o-shaped matrices (<= 256 row tiles, K <= 4096)
    //    outside Q4_K (o 20.1 -> 18.7 us at M = 64).
    // The lm_head (thousands of row tiles) keeps its register kernel.  Q4_K
    // gate|up (2368 row tiles) at M <= 16 is faster on the LDS pipeline with
    // a 2-way K split (36.1-37.6 us against 41.0 at M = 4..16).
    if (m < 2u || m > 64u || p.nt > 4096u) return false;
    const std::uint32_t mt = static_cast<std::uint32_t>(ceil_div(m, 16u));
    const bool short_k = p.k <= 4096u;
    if (mt == 1u) return !(p.type == kQ4_K && ((p.nt > 256u && p.nt <= 512u && short_k) || p.nt >= 2000u));
    if (mt == 2u) return p.nt <= 256u;
    return p.type != kQ4_K && p.nt <= 256u && short_k;
}

WsplitShape plan_wsplit(const TilePlanes& p, std::uint32_t m, const WsplitTuning& tuning) {
    WsplitShape s;
    s.mt = static_cast<std::uint32_t>(ceil_div(m, 16u));
    s.steps = static_cast<std::uint32_t>(p.kp / kStepK);
    const bool short_k = p.k <= 4096u;
    // Automatic shape (the sweep above: tile_n 1/2/4 x waves 1..8 x depth
    // 2/4 x in-kernel or separate split):
    //  * four weight tiles per workgroup, two for short-K matrices of <= 256
    //    row tiles (o), at most two with three or four activation tiles
    //    (registers);
    //  * eight waves for short-K matrices of <= 512 row tiles (q|k|v, o),
    //    four otherwise;
    //  * one step of weight codes in flight (depth 2: depth 4 costs the
    //    registers of a resident wave per SIMD and was slower everywhere);
    //  * the activations split in each wave for one activation tile, except
    //    for wide matrices at M > 8 and wide Q4_K ones (whose many
    //    workgroups would repeat the split, block sums included); split once
    //    into the workspace for two or more tiles, but for Q8_0 down and
    //    o at two tiles (below);
    //  * a K split over workgroups only while the grid holds fewer than 256
    //    workgroups, keeping at least 16 steps per split.
    std::uint32_t tn = tuning.tile_n;
    if (tn == 0u) tn = (p.nt <= 256u && short_k) ? 2u : 4u;
    if (s.mt >= 3u && tn > 2u) tn = 2u;
    s.tile_n = tn >= 4u ? 4u : tn >= 2u ? 2u : 1u;
    s.groups = static_cast<std::uint32_t>(ceil_div(p.nt, s.tile_n));
    std::uint32_t splits = tuning.k_splits;
    if (splits == 0u) {
        splits = 1u;
        while (static_cast<std::uint64_t>(s.groups) * splits < 256u && s.steps / (splits * 2u) >= 16u) splits *= 2u;
    }
    splits = splits < 1u ? 1u : (splits > s.steps ? s.steps : splits);
    s.steps_per_split = static_cast<std::uint32_t>(ceil_div(s.steps, splits));
    s.splits = static_cast<std::uint32_t>(ceil_div(s.steps, s.steps_per_split));
    std::uint32_t w = tuning.waves;
    if (w == 0u) w = (p.nt <= 512u && short_k) ? 8u : 4u;
    s.waves = w < 1u ? 1u : (w > 8u ? 8u : w);
    s.depth = tuning.depth >= 4u ? 4u : 2u;
    if (tuning.split_x != 0u) {
        s.split_x = tuning.split_x == 1u ? 1u : 0u;
    } else {
        // Two Q8_0 activation tiles are also split in each wave for long K
        // (down) and up to 24 rows otherwise (o).  Measured per linear in
        // graph replay, the split launch included: down (K = 18944) 31.9 /
        // 33.3 / 35.3 us at M = 17 / 24 / 32 against 37.7 / 37.9 / 37.8 with
        // split_rows_kernel first, o (K = 3584) 13.3 / 14.0 / 15.0 against
        // 14.5 / 14.5 / 14.8.  Q4_0 is even or slower, Q4_K's in-wave block
        // sums far slower (down 87-90 us against 39).
        const bool wide = p.nt >= 2048u;
        const bool wave_split2 = s.mt == 2u && p.type == kQ8_0 && (!short_k || m <= 24u);
        s.split_x = ((s.mt >= 2u && !wave_split2) || (wide && (m > 8u || p.type == kQ4_K))) ? 1u : 0u;
    }
    return s;
}

std::uint64_t wsplit_partials_bytes(const WsplitShape& s, std::uint32_t m, std::uint64_t n) {
    return s.splits > 1u ? static_cast<std::uint64_t>(s.splits) * m * n * 4u : 0u;
}

hipError_t launch_wsplit_linear(const TilePlanes& p, const float* x, const SplitWorkspace* ws, const float* bias,
                                float* y, std::uint32_t m, const WsplitShape& s, float* partials, hipStream_t stream,
                                const SplitEpilogue* epilogue, std::uint64_t* chain) {
    if (m == 0u || m > 64u || s.mt != ceil_div(m, 16u) || s.waves == 0u || s.waves > 8u) return hipErrorInvalidValue;
    if (!ws && (x == nullptr || p.k % 32u != 0u)) return hipErrorInvalidValue;
    WsArgs a{};
    a.x = x;
    a.k = p.k;
    if (ws) {
        a.xs = static_cast<const u32x4*>(ws->xs);
        a.inv_scale = ws->inv_scale;
        a.block_sums = ws->block_sums;
    }
    a.codes = p.codes;
    a.scales = p.scales;
    a.nt = p.nt;
    a.kt = p.kt;
    a.n = p.n;
    a.m = m;
    a.groups = s.groups;
    a.steps = s.steps;
    a.steps_per_split = s.steps_per_split;
    const bool split = s.splits > 1u;
    const bool chained = split && chain && !epilogue;
    a.partial = split ? 1u : 0u;
    a.bias = split ? nullptr : bias;
    a.out = split ? partials : y;
    if (chained) {
        a.chain = chain;
        a.y = y;
        a.chain_bias = bias;
        a.splits = s.splits;
    }
    const hipError_t err = ws ? launch_wsplit_any<false>(p.type, a, s, stream) : launch_wsplit_any<true>(p.type, a, s, stream);
    if (err != hipSuccess || !split || chained) return err;
    if (epilogue) return launch_split_epilogue(partials, s.splits, m, p.n, bias, *epilogue, stream);
    return launch_split_reduce(partials, s.splits, m, p.n, bias, y, stream);
}

} // namespace air_hip

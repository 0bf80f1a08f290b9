// linear_fused.hip -- single-launch decode linear for M <= 16 rows.
//
// Same arithmetic as decode_linear_kernel (exact integer codes as the f16
// B operand of v_mfma_f32_16x16x32_f16, activations split into f16 hi + lo
// with a power-of-two scale per (row, 32-element block), f32 block-scale
// epilogue), but the activations are read as f32 straight from the caller's
// buffer and split in registers: no workspace, no second launch, and the
// only activation traffic is the live rows' 32 bytes per lane per block.
//
// Lane layout (A operand): lane l carries row m = l % 16 and elements
// 8*(l/16)..+7 of each block; rows >= M load nothing and stay zero.  The
// block's scale is reduced over the four lanes holding that (row, block) and
// broadcast to the D-layout lanes (rows 4*(l/16)+i) that need it.
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"

#include <type_traits>

namespace air_hip {
namespace {

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

// Broadcast of a per-A-row value (held by lanes l with l % 16 == row) to the
// D-layout rows 4*(l/16)+i of this lane.  MR = rows that can be live: 1, 4, 16.
template <int MR>
__device__ __forceinline__ void rows_of_lane(float v, std::uint32_t lane, float (&out)[4]) {
    if constexpr (MR == 1) {
        out[0] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    } else if constexpr (MR == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
            out[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), i));
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = __shfl(v, static_cast<int>(4u * (lane >> 4) + i));
    }
}

// Activations of one 32-element block, split in registers.
struct SplitBlock {
    half8v hi, lo;
    float inv[4];   // inverse scale of the lane's D rows
    float sum[4];   // unscaled block sum of the lane's D rows (Q4_K min term)
};

// The lane's eight activations of block kb (zero for dead rows and blocks
// past K).
__device__ __forceinline__ void load_x8(float4 (&v)[2], const float* __restrict__ xrow, bool live,
                                        std::uint64_t kb, std::uint32_t g) {
    if (live) {
        const float4* src = reinterpret_cast<const float4*>(xrow + kb * 32u + 8u * g);
        v[0] = src[0];
        v[1] = src[1];
    } else {
        v[0] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        v[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

template <int MR, bool WantSum>
__device__ __forceinline__ void split_loaded(SplitBlock& sb, const float4 (&x8)[2], std::uint32_t lane) {
    const float v[8] = {x8[0].x, x8[0].y, x8[0].z, x8[0].w, x8[1].x, x8[1].y, x8[1].z, x8[1].w};
    float amax = fmaxf(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))),
                       fmaxf(fmaxf(fabsf(v[4]), fabsf(v[5])), fmaxf(fabsf(v[6]), fabsf(v[7]))));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    float s, inv;
    block_scale(amax, s, inv);
    split8(v, s, sb.hi, sb.lo);
    rows_of_lane<MR>(inv, lane, sb.inv);
    if constexpr (WantSum) {
        float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
        sum += __shfl_xor(sum, 16);
        sum += __shfl_xor(sum, 32);
        rows_of_lane<MR>(sum, lane, sb.sum);
    }
}

template <int MR, bool WantSum>
__device__ __forceinline__ void split_block(SplitBlock& sb, const float* __restrict__ xrow, bool live,
                                            std::uint64_t kb, std::uint32_t g, std::uint32_t lane) {
    float4 x8[2];
    load_x8(x8, xrow, live, kb, g);
    split_loaded<MR, WantSum>(sb, x8, lane);
}

// Registers of one k tile of the 32-element-block formats: R row tiles'
// codes and scales plus the lane's activations of the tile's blocks.
template <int FMT, int R>
struct BlockTile {
    static constexpr int kBlocks = FMT == kQ8_0 ? 2 : 4;
    using Scale = typename std::conditional<FMT == kQ8_0, std::uint32_t, uint2>::type;
    uint4 c[R];
    Scale sc[R];
    float4 x[kBlocks][2];
};

template <int FMT, int R>
__device__ __forceinline__ void load_block_tile(BlockTile<FMT, R>& t, const void* __restrict__ codes_,
                                                const void* __restrict__ scales_, const bool (&row_live)[R],
                                                std::uint32_t rt0, std::uint32_t KT, std::uint32_t kt,
                                                std::uint32_t lane, const float* __restrict__ xrow,
                                                bool xlive, std::uint64_t nblocks) {
    constexpr int B = BlockTile<FMT, R>::kBlocks;
    const uint4* codes = static_cast<const uint4*>(codes_);
    using Scale = typename BlockTile<FMT, R>::Scale;
    const Scale* scales = static_cast<const Scale*>(scales_);
    const std::uint32_t zero_code = FMT == kQ8_0 ? 0x80808080u : 0x88888888u;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const std::uint64_t tile = static_cast<std::uint64_t>(rt0 + r) * KT + kt;
        if (row_live[r]) {
            // Weight codes are read once per launch: non-temporal loads.
            const u32x4 word = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(codes) + tile * 64u + lane);
            t.c[r] = make_uint4(word.x, word.y, word.z, word.w);
            t.sc[r] = scales[tile * 16u + (lane & 15u)];
        } else {
            t.c[r] = make_uint4(zero_code, zero_code, zero_code, zero_code);
            t.sc[r] = Scale{};
        }
    }
#pragma unroll
    for (int b = 0; b < B; ++b) {
        const std::uint64_t kb = static_cast<std::uint64_t>(B) * kt + b;
        load_x8(t.x[b], xrow, xlive && kb < nblocks, kb, lane >> 4);
    }
}

constexpr int live_rows(int MR) { return MR < 4 ? MR : 4; }

// acc[i] += (d * inv_i) * P[i] over the lane's live D rows.
template <int MR>
__device__ __forceinline__ void block_accumulate(const SplitBlock& sb, const half8v& w, float d, float4v& acc) {
    float4v p = mfma16x16x32(sb.hi, w, float4v{0.0f, 0.0f, 0.0f, 0.0f});
    p = mfma16x16x32(sb.lo, w, p);
#pragma unroll
    for (int i = 0; i < live_rows(MR); ++i) acc[i] += (d * sb.inv[i]) * p[i];
}

template <int FMT, int R, int MR>
__device__ __forceinline__ void compute_block_tile(const BlockTile<FMT, R>& t, std::uint32_t lane,
                                                   float4v (&acc)[R]) {
    constexpr int B = BlockTile<FMT, R>::kBlocks;
#pragma unroll
    for (int b = 0; b < B; ++b) {
        SplitBlock sb;
        split_loaded<MR, false>(sb, t.x[b], lane);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            half8v w;
            std::uint32_t dbits;
            if constexpr (FMT == kQ8_0) {
                w = b == 0 ? q8_codes_to_half8(t.c[r].x, t.c[r].y) : q8_codes_to_half8(t.c[r].z, t.c[r].w);
                dbits = (t.sc[r] >> (16 * b)) & 0xffffu;
            } else {
                const std::uint32_t cw = b == 0 ? t.c[r].x : b == 1 ? t.c[r].y : b == 2 ? t.c[r].z : t.c[r].w;
                w = nibble_dword_to_half8<8>(cw);
                dbits = ((b < 2 ? t.sc[r].x : t.sc[r].y) >> (16 * (b & 1))) & 0xffffu;
            }
            block_accumulate<MR>(sb, w, half_bits_to_float(dbits), acc[r]);
        }
    }
}

// Largest workgroup (in waves) a variant is compiled for; Q4_K's scale
// decode needs more registers than a 16-wave workgroup leaves.
constexpr int fused_max_waves(int FMT, int R, int MR) {
    return FMT == kQ4_K ? ((R > 1 || MR == 16) ? 4 : 16)
         : FMT == kQ4_0 ? (R == 4 ? 4 : (R == 2 ? 8 : 16))
         : (R == 4 ? 8 : 16);
}

// Workgroup = W waves on the same R row tiles, K split across the waves.
template <int FMT, int R, int MR>
__global__ void __launch_bounds__(64 * fused_max_waves(FMT, R, MR))
decode_fused_kernel(const void* __restrict__ codes_, const void* __restrict__ scales_,
                    const float* __restrict__ x, const float* __restrict__ bias, float* __restrict__ y,
                    std::uint32_t M, std::uint64_t K, std::uint64_t N, std::uint32_t NT, std::uint32_t KT,
                    float4v* __restrict__ split_partials, std::uint32_t* __restrict__ split_counters) {
    extern __shared__ float4v partials[];
    const std::uint32_t lane = threadIdx.x & 63u;
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform
    const std::uint32_t W = blockDim.x >> 6;
    const std::uint32_t rt0 = blockIdx.x * R;
    // k tiles of this workgroup's slice, then of this wave within it
    const std::uint64_t slice_begin = (static_cast<std::uint64_t>(KT) * blockIdx.y) / gridDim.y;
    const std::uint64_t slice_len = (static_cast<std::uint64_t>(KT) * (blockIdx.y + 1u)) / gridDim.y - slice_begin;
    const std::uint32_t kt_begin = static_cast<std::uint32_t>(slice_begin + (slice_len * wave) / W);
    const std::uint32_t kt_end = static_cast<std::uint32_t>(slice_begin + (slice_len * (wave + 1u)) / W);
    const std::uint32_t g = lane >> 4;
    const std::uint32_t mrow = lane & 15u;
    const std::uint64_t nblocks = K / 32u;
    const float* xrow = x + static_cast<std::uint64_t>(mrow < M ? mrow : 0u) * K;

    float4v acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    bool row_live[R];
#pragma unroll
    for (int r = 0; r < R; ++r) row_live[r] = (rt0 + r) < NT;

    if constexpr (FMT == kQ8_0 || FMT == kQ4_0) {
        // Software pipeline, one k tile ahead: the loads of tile kt+1 (codes,
        // scales and activations) are in flight while tile kt is computed.
        const bool xlive = mrow < M;
        BlockTile<FMT, R> cur, nxt;
        if (kt_begin < kt_end) load_block_tile<FMT, R>(cur, codes_, scales_, row_live, rt0, KT, kt_begin, lane, xrow, xlive, nblocks);
        for (std::uint32_t kt = kt_begin; kt < kt_end; kt += 2u) {
            if (kt + 1u < kt_end) load_block_tile<FMT, R>(nxt, codes_, scales_, row_live, rt0, KT, kt + 1u, lane, xrow, xlive, nblocks);
            compute_block_tile<FMT, R, MR>(cur, lane, acc);
            if (kt + 1u >= kt_end) break;
            if (kt + 2u < kt_end) load_block_tile<FMT, R>(cur, codes_, scales_, row_live, rt0, KT, kt + 2u, lane, xrow, xlive, nblocks);
            compute_block_tile<FMT, R, MR>(nxt, lane, acc);
        }
    }
    for (std::uint32_t kt = kt_begin; kt < kt_end; ++kt) {
        if constexpr (FMT == kQ8_0 || FMT == kQ4_0) {
            break;
        } else { // Q4_K: one super-block of 8 sub-blocks per k tile
            const uint4* codes = static_cast<const uint4*>(codes_);
            const uint4* scales = static_cast<const uint4*>(scales_);
            uint4 c0[R], c1[R], sc[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const std::uint64_t tile = static_cast<std::uint64_t>(rt0 + r) * KT + kt;
                u32x4 w0 = {0u, 0u, 0u, 0u}, w1 = {0u, 0u, 0u, 0u};
                if (row_live[r]) {
                    const u32x4* rec = reinterpret_cast<const u32x4*>(codes) + (tile * 2u) * 64u + lane;
                    w0 = __builtin_nontemporal_load(rec);
                    w1 = __builtin_nontemporal_load(rec + 64u);
                }
                c0[r] = make_uint4(w0.x, w0.y, w0.z, w0.w);
                c1[r] = make_uint4(w1.x, w1.y, w1.z, w1.w);
                sc[r] = row_live[r] ? scales[tile * 16u + mrow] : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const std::uint64_t kb = 8u * static_cast<std::uint64_t>(kt) + j;
                SplitBlock sb;
                split_block<MR, true>(sb, xrow, mrow < M && kb < nblocks, kb, g, lane);
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const std::uint32_t packed[3] = {sc[r].y, sc[r].z, sc[r].w};
                    std::uint32_t s6 = 0, m6 = 0;
                    q4k_scale_min(packed, static_cast<std::uint32_t>(j), s6, m6);
                    const float dj = half_bits_to_float(sc[r].x & 0xffffu) * static_cast<float>(s6);
                    const float mj = half_bits_to_float(sc[r].x >> 16) * static_cast<float>(m6);
                    const std::uint32_t cw = j < 4 ? (j == 0 ? c0[r].x : j == 1 ? c0[r].y : j == 2 ? c0[r].z : c0[r].w)
                                                   : (j == 4 ? c1[r].x : j == 5 ? c1[r].y : j == 6 ? c1[r].z : c1[r].w);
                    block_accumulate<MR>(sb, nibble_dword_to_half8<0>(cw), dj, acc[r]);
#pragma unroll
                    for (int i = 0; i < live_rows(MR); ++i) acc[r][i] -= mj * sb.sum[i];
                }
            }
        }
    }

    if (W > 1u) {
        if (wave > 0u) {
#pragma unroll
            for (int r = 0; r < R; ++r) partials[((wave - 1u) * R + r) * 64u + lane] = acc[r];
        }
        __syncthreads();
        if (wave == 0u) {
            for (std::uint32_t w = 1; w < W; ++w) {
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] += partials[((w - 1u) * R + r) * 64u + lane];
            }
        }
    }
    if (wave != 0u) return;

    // K split over S workgroups: publish this slice's partial; the workgroup
    // that completes the row group last adds the S partials in slice order
    // (deterministic) and re-arms the counter for the next launch.
    const std::uint32_t S = gridDim.y;
    if (S > 1u) {
        const std::uint32_t rg = blockIdx.x;
        const std::uint64_t groups = gridDim.x;
#pragma unroll
        for (int r = 0; r < R; ++r) split_partials[((blockIdx.y * groups + rg) * R + r) * 64u + lane] = acc[r];
        __threadfence();
        std::uint32_t arrived = 0;
        if (lane == 0u) {
            arrived = __hip_atomic_fetch_add(split_counters + rg, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        }
        arrived = __shfl(arrived, 0);
        if (arrived != S - 1u) return;
        __threadfence();
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
        for (std::uint32_t s = 0; s < S; ++s) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const float4v* src = split_partials + ((s * groups + rg) * R + r) * 64u + lane;
                acc[r] += __builtin_nontemporal_load(src);
            }
        }
        if (lane == 0u) __hip_atomic_store(split_counters + rg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
        if (!row_live[r]) continue;
        const std::uint64_t n = static_cast<std::uint64_t>(rt0 + r) * 16u + mrow;
        if (n >= N) continue;
        const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int i = 0; i < live_rows(MR); ++i) {
            const std::uint32_t m = 4u * g + i;
            if (m < M) y[static_cast<std::uint64_t>(m) * N + n] = acc[r][i] + bn;
        }
    }
}

struct FusedLaunch {
    std::uint32_t R, W, S;
    float4v* partials;
    std::uint32_t* counters;
};

template <int FMT, int R, int MR>
hipError_t launch_fused_variant(const TilePlanes& p, const float* x, const float* bias, float* y,
                                std::uint32_t M, const FusedLaunch& L, hipStream_t stream) {
    if (L.W > static_cast<std::uint32_t>(fused_max_waves(FMT, R, MR))) return hipErrorInvalidConfiguration;
    const dim3 grid(static_cast<unsigned>(ceil_div(p.nt, R)), L.S, 1);
    const std::size_t lds = static_cast<std::size_t>(L.W - 1u) * R * 64u * sizeof(float4v);
    decode_fused_kernel<FMT, R, MR><<<grid, 64u * L.W, lds, stream>>>(
        p.codes, p.scales, x, bias, y, M, p.k, p.n, p.nt, p.kt, L.partials, L.counters);
    return hipGetLastError();
}

template <int FMT, int R>
hipError_t launch_fused_mr(const TilePlanes& p, const float* x, const float* bias, float* y,
                           std::uint32_t M, const FusedLaunch& L, hipStream_t s) {
    if (M == 1u) return launch_fused_variant<FMT, R, 1>(p, x, bias, y, M, L, s);
    if (M <= 4u) return launch_fused_variant<FMT, R, 4>(p, x, bias, y, M, L, s);
    return launch_fused_variant<FMT, R, 16>(p, x, bias, y, M, L, s);
}

template <int FMT>
hipError_t launch_fused_fmt(const TilePlanes& p, const float* x, const float* bias, float* y,
                            std::uint32_t M, const FusedLaunch& L, hipStream_t s) {
    switch (L.R) {
    case 1: return launch_fused_mr<FMT, 1>(p, x, bias, y, M, L, s);
    case 2: return launch_fused_mr<FMT, 2>(p, x, bias, y, M, L, s);
    default: return launch_fused_mr<FMT, 4>(p, x, bias, y, M, L, s);
    }
}

} // namespace

FusedShape plan_decode_fused(const TilePlanes& p, std::uint32_t m, const DecodeTuning& tuning) {
    FusedShape f{};
    // Row tiles per wave: long weight streams per wave where the row tiles
    // alone fill the chip, single tiles where they do not.
    f.rows_per_wave = p.nt >= 2048u ? 4u : (p.nt >= 1024u ? 2u : 1u);
    if (p.type == kQ4_K && f.rows_per_wave > 2u) f.rows_per_wave = 2u;
    if (tuning.rows_per_wave == 1u || tuning.rows_per_wave == 2u || tuning.rows_per_wave == 4u) {
        f.rows_per_wave = tuning.rows_per_wave;
    }
    const std::uint64_t groups = ceil_div(p.nt, f.rows_per_wave);
    const std::uint32_t w_cap = static_cast<std::uint32_t>(
        fused_max_waves(p.type, static_cast<int>(f.rows_per_wave), m == 1u ? 1 : (m <= 4u ? 4 : 16)));
    // Then split K: first over the waves of a workgroup, then over
    // workgroups, aiming at ~8192 waves with >= 3 k tiles each.
    f.waves_per_group = 1;
    f.k_splits = 1;
    while (groups * f.waves_per_group * f.k_splits < 8192u) {
        const std::uint64_t waves_k = static_cast<std::uint64_t>(f.waves_per_group) * f.k_splits;
        if (p.kt < 6u * waves_k) break;
        // Cross-workgroup splits cost an L2 write-back per workgroup, so
        // only waves inside a workgroup split K automatically.
        if (f.waves_per_group < w_cap) {
            f.waves_per_group <<= 1;
        } else {
            break;
        }
    }
    if (tuning.waves_per_group != 0u) f.waves_per_group = tuning.waves_per_group < w_cap ? tuning.waves_per_group : w_cap;
    if (tuning.k_splits != 0u) f.k_splits = tuning.k_splits;
    if (f.k_splits > p.kt) f.k_splits = p.kt;
    f.groups = static_cast<std::uint32_t>(groups);
    return f;
}

std::uint64_t fused_split_workspace_bytes(const FusedShape& f) {
    if (f.k_splits <= 1u) return 0;
    const std::uint64_t partials = static_cast<std::uint64_t>(f.k_splits) * f.groups * f.rows_per_wave * 64u * 16u;
    return ceil_div(partials, 256u) * 256u;
}

hipError_t launch_decode_fused(const TilePlanes& p, const float* x, const float* bias, float* y,
                               std::uint32_t m, const FusedShape& f, void* partials,
                               std::uint32_t* counters, hipStream_t stream) {
    if (m == 0u || m > kFusedMaxRows) return hipErrorInvalidValue;
    if (f.waves_per_group == 0u || f.waves_per_group > 16u || f.k_splits == 0u || f.k_splits > 65535u) {
        return hipErrorInvalidConfiguration;
    }
    if (f.k_splits > 1u && (partials == nullptr || counters == nullptr)) return hipErrorInvalidValue;
    const FusedLaunch L{f.rows_per_wave, f.waves_per_group, f.k_splits, static_cast<float4v*>(partials), counters};
    switch (p.type) {
    case kQ8_0: return launch_fused_fmt<kQ8_0>(p, x, bias, y, m, L, stream);
    case kQ4_0: return launch_fused_fmt<kQ4_0>(p, x, bias, y, m, L, stream);
    case kQ4_K: return launch_fused_fmt<kQ4_K>(p, x, bias, y, m, L, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace air_hip

// linear_skinny.hip -- the decode linear for M = 2..64 rows on exact codes.
//
// Exact integer codes as f16 MFMA operands, activations split into f16 hi +
// lo after one power-of-two scale per row (so the row's largest |x| lands in
// [2^14, 2^15); every value above 2^-17 of it keeps ~22 significant bits),
// per-block f32 weight-scale epilogue, the row scale undone once at the end;
// relative L2 error ~1e-6.  Arranged so that the weights stream once:
//
//   * a workgroup is four waves that own 4 * TN distinct 16-row weight tiles
//     and ALL activation rows (M <= 64: up to four 16-row tiles), so every
//     weight byte is read exactly once per launch;
//   * per 64-k step the split activations of the step (hi, lo, inverse
//     scales, Q4_K block sums) are copied once into LDS by the whole
//     workgroup and read by each wave once per 32-block, then reused for all
//     of that wave's weight tiles;
//   * each wave streams its own weight codes two steps ahead of the MFMAs;
//   * when the weight tiles alone cannot occupy the 256 CUs, K is split over
//     workgroups and the partials are summed by a second, fixed-order pass.
//
// Two activation sources: the row-scaled split written once by
// split_rows_kernel (air_hip_activations_load, shared by several linears),
// or the f32 rows themselves (XF): the workgroup then splits each step's
// activations while staging them, with one power-of-two scale per (row,
// 32-block) applied in the epilogue, so a linear is one launch (plus the
// split reduction) and writes no activation workspace.
//
// Replaces specialized_matmul_kernel / specialized_matmul_batch_reuse_kernel
// (src/cuda/cuda_backend.cu:501-583), which decode every weight M/4 or M/8
// times.
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"
#include "air_hip_steps.hpp"

namespace air_hip {
namespace {

constexpr unsigned kThreads = 256;
constexpr unsigned kSplitThreads = 1024;  // one workgroup per activation row

struct SkinnyArgs {
    const float* x;              // XF: activations [m][k] f32
    std::uint64_t k;             // XF: input width
    const void* codes;
    const void* scales;
    std::uint32_t nt, kt;
    std::uint64_t n;
    const uint4* xs;             // split activations [block][MT][2][64] x 16 B
    const float* inv_scale;      // [mp] inverse power-of-two scale of each row
    const float* block_sums;     // [block][mp] sums of the scaled values (Q4_K)
    const float* bias;           // fused when not split
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

// Stores element (m, n) of a workgroup of split `split`: y (not split), the
// partial for the reduction launch, or the partial into the in-kernel chain.
__device__ __forceinline__ void skinny_store(const SkinnyArgs& a, float* out, std::uint32_t split, std::uint32_t m,
                                             std::uint64_t n, float v) {
    const std::uint64_t e = static_cast<std::uint64_t>(m) * a.n + n;
    if (a.chain) {
        if (!chain_combine(a.chain, static_cast<std::uint64_t>(a.m) * a.n, e, split, a.splits, v)) return;
        a.y[e] = a.chain_bias ? v + a.chain_bias[n] : v;
        return;
    }
    out[e] = v;
}

template <int FMT, int MT, int TN, bool XF>
__global__ __launch_bounds__(kThreads, 2) void skinny_kernel(SkinnyArgs a) {
    constexpr unsigned kMp = 16u * MT;
    constexpr unsigned kChunks = 2u * MT * 2u * 64u / kThreads;  // uint4 of activations per thread per step
    constexpr bool kSums = FMT == kQ4_K;
    constexpr unsigned kFrags = 2u * MT;                          // XF: (block, tile) fragments per step
    constexpr unsigned kFragsPerWave = (kFrags + 3u) / 4u;
    __shared__ u32x4 xa[2][2 * MT * 2 * 64];     // [buf][block][tile][part][lane]
    // [buf][block][row] sums of x (Q4_K): scaled per row, or unscaled (XF).
    __shared__ float4v sm[2][kSums ? 2 * kMp / 4 : 1];
    __shared__ float4v sinv[2][XF ? 2 * kMp / 4 : 1];  // XF: [buf][block][row] inverse scales

    const std::uint32_t tid = threadIdx.x;
    const std::uint32_t lane = tid & 63u;
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    const std::uint32_t group = blockIdx.x % a.groups;
    const std::uint32_t split = blockIdx.x / a.groups;
    const std::uint32_t rt0 = (group * 4u + wave) * TN;
    const std::uint32_t s_begin = split * a.steps_per_split;
    const std::uint32_t s_end = min(a.steps, s_begin + a.steps_per_split);

    float4v acc[TN][MT];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    // Activation staging: step s covers blocks 2s, 2s+1, contiguous in the
    // workspace.  Two register slots: the activations of step s + 2 are
    // loaded while step s computes, so their latency spans two steps.  One
    // slot (load one step ahead) for the Q8_0 f32 variant with two or more
    // activation tiles, where the second slot would cost a wave per SIMD.
    constexpr int kXSlots = (XF && FMT == kQ8_0 && MT >= 2) ? 1 : 2;
    u32x4 xr[kXSlots][XF ? 1 : kChunks];
    float4v mr[kXSlots];
#pragma unroll
    for (int i = 0; i < kXSlots; ++i) mr[i] = float4v{0.f, 0.f, 0.f, 0.f};
    // XF: wave w splits fragments w, w + 4, ...: fragment c is block c / MT,
    // activation tile c % MT; lane l holds row l % 16, elements 8 (l / 16)..+7.
    float4 xfs[kXSlots][XF ? kFragsPerWave : 1][2];
    const auto load_x = [&](std::uint32_t s, int slot) __attribute__((always_inline)) {
        auto& xf = xfs[slot];
        if constexpr (XF) {
#pragma unroll
            for (unsigned r = 0; r < kFragsPerWave; ++r) {
                const unsigned c = wave + 4u * r;
                const unsigned row = (c % MT) * 16u + (lane & 15u);
                const std::uint64_t col = (2u * static_cast<std::uint64_t>(s) + c / MT) * 32u + 8u * (lane >> 4);
                xf[r][0] = make_float4(0.f, 0.f, 0.f, 0.f);
                xf[r][1] = xf[r][0];
                if (c < kFrags && row < a.m && col < a.k) {
                    const float4* src = reinterpret_cast<const float4*>(a.x + static_cast<std::uint64_t>(row) * a.k + col);
                    xf[r][0] = src[0];
                    xf[r][1] = src[1];
                }
            }
        } else {
            const u32x4* src = reinterpret_cast<const u32x4*>(a.xs) + static_cast<std::uint64_t>(s) * (2u * MT * 2u * 64u);
#pragma unroll
            for (unsigned j = 0; j < kChunks; ++j) xr[slot][j] = src[tid + kThreads * j];
            if constexpr (kSums) {
                if (tid < 2u * kMp / 4u) mr[slot] = reinterpret_cast<const float4v*>(a.block_sums + static_cast<std::uint64_t>(s) * 2u * kMp)[tid];
            }
        }
    };
    const auto store_x = [&](unsigned buf, int slot) __attribute__((always_inline)) {
        auto& xf = xfs[slot];
        if constexpr (XF) {
#pragma unroll
            for (unsigned r = 0; r < kFragsPerWave; ++r) {
                const unsigned c = wave + 4u * r;
                if (c >= kFrags) continue;  // uniform per wave
                const float v[8] = {xf[r][0].x, xf[r][0].y, xf[r][0].z, xf[r][0].w,
                                    xf[r][1].x, xf[r][1].y, xf[r][1].z, xf[r][1].w};
                float amax = fmaxf(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))),
                                   fmaxf(fmaxf(fabsf(v[4]), fabsf(v[5])), fmaxf(fabsf(v[6]), fabsf(v[7]))));
                amax = fmaxf(amax, __shfl_xor(amax, 16));
                amax = fmaxf(amax, __shfl_xor(amax, 32));
                float sc, inv;
                block_scale(amax, sc, inv);
                half8v hi, lo;
                split8(v, sc, hi, lo);
                const unsigned base = (c * 2u) * 64u + lane;   // c = block * MT + tile
                xa[buf][base] = __builtin_bit_cast(u32x4, hi);
                xa[buf][base + 64u] = __builtin_bit_cast(u32x4, lo);
                const unsigned slot = (c / MT) * kMp + (c % MT) * 16u + lane;   // [block][row]
                if (lane < 16u) reinterpret_cast<float*>(&sinv[buf][0])[slot] = inv;
                if constexpr (kSums) {
                    float sum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
                    sum += __shfl_xor(sum, 16);
                    sum += __shfl_xor(sum, 32);
                    if (lane < 16u) reinterpret_cast<float*>(&sm[buf][0])[slot] = sum;
                }
            }
        } else {
#pragma unroll
            for (unsigned j = 0; j < kChunks; ++j) xa[buf][tid + kThreads * j] = xr[slot][j];
            if constexpr (kSums) {
                if (tid < 2u * kMp / 4u) sm[buf][tid] = mr[slot];
            }
        }
    };
    StepCodes<FMT> wa[TN], wb[TN];
    const auto load_w = [&](StepCodes<FMT>(&dst)[TN], std::uint32_t s) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const std::uint32_t rt = rt0 + static_cast<std::uint32_t>(j);
            load_step<FMT, true>(a.codes, a.scales, rt, a.kt, s, lane, rt < a.nt, dst[j]);
        }
    };
    // slot: the register slot of step s's activations ((s - s_begin) % 2 with
    // two slots).
    const auto step = [&](std::uint32_t s, StepCodes<FMT>(&cur)[TN], int slot) __attribute__((always_inline)) {
        const unsigned buf = (s - s_begin) & 1u;
        const bool more = s + 1u < s_end;
        if constexpr (kXSlots == 2) {
            if (s + 2u < s_end) load_x(s + 2u, slot);   // step s's slot is free: staged already
        } else {
            if (more) load_x(s + 1u, 0);
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            half8v w[TN];
            float ws[TN], wo[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                w[j] = step_codes<FMT>(cur[j], b);
                step_scale<FMT>(cur[j], s, b, ws[j], wo[j]);
            }
            if (b == 1 && s + 2u < s_end) load_w(cur, s + 2u);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const unsigned base = ((static_cast<unsigned>(b) * MT + t) * 2u) * 64u + lane;
                const half8v hi = __builtin_bit_cast(half8v, xa[buf][base]);
                const half8v lo = __builtin_bit_cast(half8v, xa[buf][base + 64u]);
                float4v sum4 = {0.f, 0.f, 0.f, 0.f};
                if constexpr (kSums) sum4 = sm[buf][(static_cast<unsigned>(b) * kMp + t * 16u) / 4u + (lane >> 4)];
                float4v inv4 = {1.f, 1.f, 1.f, 1.f};
                if constexpr (XF) inv4 = sinv[buf][(static_cast<unsigned>(b) * kMp + t * 16u) / 4u + (lane >> 4)];
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    float4v p = mfma16x16x32(hi, w[j], float4v{0.f, 0.f, 0.f, 0.f});
                    p = mfma16x16x32(lo, w[j], p);
                    if constexpr (XF) {
                        acc[j][t] += (ws[j] * inv4) * p;
                    } else {
                        acc[j][t] += ws[j] * p;
                    }
                    if constexpr (kSums) acc[j][t] -= wo[j] * sum4;
                }
            }
        }
        if (more) store_x(buf ^ 1u, kXSlots == 2 ? slot ^ 1 : 0);
        __syncthreads();
    };

    if (s_begin < s_end) {
        load_x(s_begin, 0);
        load_w(wa, s_begin);
        if (s_begin + 1u < s_end) {
            if constexpr (kXSlots == 2) load_x(s_begin + 1u, 1);
            load_w(wb, s_begin + 1u);
        }
        store_x(0, 0);
    }
    __syncthreads();
    std::uint32_t s = s_begin;
    for (; s + 1u < s_end; s += 2u) {
        step(s, wa, 0);
        step(s + 1u, wb, 1);
    }
    if (s < s_end) step(s, wa, 0);

    // D[row = activation row][col = weight row]: lane holds rows 4(l/16)+i of
    // column l%16; the rows' power-of-two activation scales are undone here.
    float4v inv[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        inv[t] = XF ? float4v{1.f, 1.f, 1.f, 1.f} : reinterpret_cast<const float4v*>(a.inv_scale)[t * 4 + (lane >> 4)];
    }
    float* out = a.out + (a.partial ? static_cast<std::uint64_t>(split) * a.m * a.n : 0u);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const std::uint64_t n = static_cast<std::uint64_t>(rt0 + static_cast<std::uint32_t>(j)) * 16u + (lane & 15u);
        if (n >= a.n) continue;
        const float bn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const std::uint32_t m = static_cast<std::uint32_t>(t) * 16u + 4u * (lane >> 4) + static_cast<std::uint32_t>(i);
                if (m < a.m) skinny_store(a, out, split, m, n, acc[j][t][i] * inv[t][i] + bn);
            }
        }
    }
}

// ---- LDS-pipelined variant (split activations) ------------------------------
//
// The same arithmetic as skinny_kernel<FMT, MT, TN, false>, with every
// operand of a 64-k step moved by direct global -> LDS loads into one of NS
// stages, so up to NS - 1 steps of weight codes per wave are in flight
// without holding registers (the register pipeline above has room for two).
// A stage holds the step's 4 MT activation fragments (each wave loads MT of
// them), then each wave's TN weight-code records and scale records, then
// (Q4_K) the step's activation block sums.  Per 16-row tile and step the
// codes are one 64-lane x 16-byte fragment (Q8_0), or the lane's half of its
// 16-byte record (Q4_0, Q4_K: two 64-lane x 4-byte loads); the scales are
// 64 lanes x 4 bytes (Q8_0, Q4_0: the lane's row's two block scales; Q4_K:
// the tile's 16 super-block headers, 256 contiguous bytes).  Everything is
// read back in lane order (no bank conflicts).  One bare barrier per step
// publishes the stage and frees the oldest one; a wave waits only for its
// own loads of the stage (vmcnt).
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// Lane l's 16 (or 4) bytes land at lds_wave_base + l * 16 (l * 4).
__device__ __forceinline__ void lds_load16(const void* src, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds((global_void_t*)(const_cast<void*>(src)), (lds_void_t*)(lds_wave_base), 16, 0, 0);
}
__device__ __forceinline__ void lds_load4(const void* src, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds((global_void_t*)(const_cast<void*>(src)), (lds_void_t*)(lds_wave_base), 4, 0, 0);
}

// s_waitcnt for vmcnt <= n only (expcnt and lgkmcnt at their maxima).
template <unsigned n>
__device__ __forceinline__ void wait_vm() {
    static_assert(n < 64u, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((n & 0xfu) | ((n >> 4) << 14) | (0x7u << 4) | (0xfu << 8));
}

template <int FMT>
constexpr unsigned lds_code_bytes() {
    return FMT == kQ8_0 ? 1024u : 512u;   // per tile and step
}

template <int FMT, int MT, int TN, int W = 4>
constexpr unsigned skinny_stage_bytes() {
    return 4u * MT * 1024u + W * TN * (lds_code_bytes<FMT>() + 256u) + (FMT == kQ4_K ? W * 256u : 0u);
}

// W waves per workgroup (4, or 8 with two or four activation tiles): the
// workgroup covers W * TN weight tiles, so eight waves read each step's
// activations into LDS once for twice the weight rows.
template <int FMT, int MT, int TN, int NS, int W = 4>
__global__ __launch_bounds__(64 * W, W == 4 ? 2 : 1) void skinny_lds_kernel(SkinnyArgs a) {
    constexpr unsigned kStage = skinny_stage_bytes<FMT, MT, TN, W>();
    constexpr unsigned kCodeBytes = lds_code_bytes<FMT>();
    constexpr unsigned kCodes = 4u * MT * 1024u;                  // offset of the weight codes in a stage
    constexpr unsigned kScales = kCodes + W * TN * kCodeBytes;    // offset of the weight scales
    constexpr unsigned kSumsAt = kScales + W * TN * 256u;         // offset of the block sums (Q4_K)
    constexpr bool kSums = FMT == kQ4_K;
    constexpr unsigned kMp = 16u * MT;
    constexpr unsigned kActLoads = 4u * MT / W;                   // activation fragments per wave per step
    // Load instructions per wave per stage (the same for every wave).
    constexpr unsigned kLoads = kActLoads + TN * (FMT == kQ8_0 ? 2u : 3u) + (kSums ? 1u : 0u);
    static_assert(W == 4 || W == 8, "four or eight waves");
    static_assert((4u * MT) % W == 0u, "activation fragments split evenly over the waves");
    static_assert(NS >= 2 && NS <= 4, "two to four stages");
    static_assert(2u * kMp <= W * 64u, "one block-sum load per wave covers a step");
    // One LDS object per stage, addressed with compile-time stage numbers:
    // the compiler's wait-count pass then sees that a stage's direct loads
    // and another stage's reads touch different objects.
    __shared__ __attribute__((aligned(1024))) unsigned char stage0[kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage1[kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage2[NS > 2 ? kStage : 16];
    __shared__ __attribute__((aligned(1024))) unsigned char stage3[NS > 3 ? kStage : 16];
    const auto stage = [&](unsigned st) __attribute__((always_inline)) -> unsigned char* {
        return st == 0u ? stage0 : st == 1u ? stage1 : st == 2u ? stage2 : stage3;
    };

    const std::uint32_t lane = threadIdx.x & 63u;
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const std::uint32_t group = blockIdx.x % a.groups;
    const std::uint32_t split = blockIdx.x / a.groups;
    const std::uint32_t rt0 = (group * W + wave) * TN;
    const std::uint32_t s_begin = split * a.steps_per_split;
    const std::uint32_t s_end = min(a.steps, s_begin + a.steps_per_split);

    float4v acc[TN][MT];
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    // Padded weight rows (rt >= nt) read the last real tile: their outputs
    // are never stored.
    std::uint64_t wtile[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const std::uint32_t rt = min(rt0 + static_cast<std::uint32_t>(j), a.nt - 1u);
        wtile[j] = static_cast<std::uint64_t>(rt) * a.kt;
    }
    const u32x4* xs = reinterpret_cast<const u32x4*>(a.xs);
    const std::uint32_t* codes32 = static_cast<const std::uint32_t*>(a.codes);
    const std::uint32_t* scales32 = static_cast<const std::uint32_t*>(a.scales);
    // Q4_K: this lane's block-sum load, the step's 2 * kMp sums spread over
    // the four waves (lanes past them repeat the last one into unused slots).
    const std::uint32_t sum_slot = wave * 64u + lane;
    const std::uint32_t sum_src = min(sum_slot, 2u * kMp - 1u);
    const auto issue = [&](std::uint32_t s, unsigned st) __attribute__((always_inline)) {
        unsigned char* base = stage(st);
        // Fragment f of the step: block f / (2 MT), tile (f / 2) % MT, part f % 2.
#pragma unroll
        for (unsigned j = 0; j < kActLoads; ++j) {
            const unsigned f = wave + W * j;
            lds_load16(xs + (static_cast<std::uint64_t>(s) * (4u * MT) + f) * 64u + lane, base + f * 1024u);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const unsigned slot = wave * TN + static_cast<unsigned>(j);
            unsigned char* code_dst = base + kCodes + slot * kCodeBytes;
            unsigned char* scale_dst = base + kScales + slot * 256u;
            if constexpr (FMT == kQ8_0) {
                const std::uint64_t tile = wtile[j] + s;
                lds_load16(static_cast<const u32x4*>(a.codes) + tile * 64u + lane, code_dst);
                lds_load4(scales32 + tile * 16u + (lane & 15u), scale_dst);
            } else if constexpr (FMT == kQ4_0) {
                // 128-k tiles: the step is half (s & 1) of the lane's record.
                const std::uint64_t tile = wtile[j] + (s >> 1);
                const std::uint64_t rec = ((tile * 64u + lane) * 2u + (s & 1u)) * 2u;   // dword index
                lds_load4(codes32 + rec, code_dst);
                lds_load4(codes32 + rec + 1u, code_dst + 256u);
                lds_load4(scales32 + (tile * 16u + (lane & 15u)) * 2u + (s & 1u), scale_dst);
            } else {
                // 256-k super-blocks: sub-block pair s & 3 of two 16-byte records.
                const std::uint64_t tile = wtile[j] + (s >> 2);
                const std::uint32_t sub = s & 3u;
                const std::uint64_t rec = (((tile * 2u + (sub >> 1)) * 64u + lane) * 2u + (sub & 1u)) * 2u;
                lds_load4(codes32 + rec, code_dst);
                lds_load4(codes32 + rec + 1u, code_dst + 256u);
                lds_load4(scales32 + tile * 64u + lane, scale_dst);   // the 16 rows' headers
            }
        }
        if constexpr (kSums) {
            lds_load4(a.block_sums + static_cast<std::uint64_t>(s) * 2u * kMp + sum_src, base + kSumsAt + wave * 256u);
        }
    };
    const auto compute = [&](std::uint32_t s, unsigned st) __attribute__((always_inline)) {
        const unsigned char* base = stage(st);
        StepCodes<FMT> w_in[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const unsigned slot = wave * TN + static_cast<unsigned>(j);
            const unsigned char* code_src = base + kCodes + slot * kCodeBytes;
            const unsigned char* scale_src = base + kScales + slot * 256u;
            if constexpr (FMT == kQ8_0) {
                w_in[j].c = *reinterpret_cast<const u32x4*>(code_src + lane * 16u);
                w_in[j].d = *reinterpret_cast<const std::uint32_t*>(scale_src + lane * 4u);
            } else {
                w_in[j].c.x = *reinterpret_cast<const std::uint32_t*>(code_src + lane * 4u);
                w_in[j].c.y = *reinterpret_cast<const std::uint32_t*>(code_src + 256u + lane * 4u);
                if constexpr (FMT == kQ4_0) {
                    w_in[j].d = *reinterpret_cast<const std::uint32_t*>(scale_src + lane * 4u);
                } else {
                    w_in[j].h = *reinterpret_cast<const u32x4*>(scale_src + (lane & 15u) * 16u);
                }
            }
        }
        half8v xf[2][MT][2];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int part = 0; part < 2; ++part) {
                    const unsigned f = (static_cast<unsigned>(b) * MT + t) * 2u + part;
                    xf[b][t][part] = *reinterpret_cast<const half8v*>(base + f * 1024u + lane * 16u);
                }
        float4v sum4[kSums ? 2 : 1][kSums ? MT : 1];
        if constexpr (kSums) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const unsigned at = (static_cast<unsigned>(b) * kMp + t * 16u + 4u * (lane >> 4)) * 4u;
                    sum4[b][t] = *reinterpret_cast<const float4v*>(base + kSumsAt + at);
                }
        }
        __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the arithmetic
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const half8v w = step_codes<FMT>(w_in[j], b);
                float ws, wo;
                step_scale<FMT>(w_in[j], s, b, ws, wo);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    float4v p = mfma16x16x32(xf[b][t][0], w, float4v{0.f, 0.f, 0.f, 0.f});
                    p = mfma16x16x32(xf[b][t][1], w, p);
                    acc[j][t] += ws * p;
                    if constexpr (kSums) acc[j][t] -= wo * sum4[b][t];
                }
            }
        }
    };

    const std::uint32_t steps = s_end > s_begin ? s_end - s_begin : 0u;
#pragma unroll
    for (unsigned q = 0; q + 1u < NS; ++q) {
        if (q < steps) issue(s_begin + q, q);
    }
    // Step q of the split computes stage q mod NS (ST, a constant).
    const auto step = [&](std::uint32_t q, auto st_tag) __attribute__((always_inline)) {
        constexpr unsigned ST = decltype(st_tag)::value;
        // Stage ST is complete once at most the later stages' loads are in
        // flight; near the end fewer follow it, so wait for everything.
        if (q + NS - 2u < steps) {
            wait_vm<kLoads * (NS - 2u)>();
        } else {
            wait_vm<0u>();
        }
        // Every wave's reads of the previous stage are complete before the
        // barrier, after which that stage takes new loads; a bare s_barrier
        // (a fence would also wait for the loads still in flight).
        __builtin_amdgcn_s_waitcnt(0xc07fu);   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        if (q + NS - 1u < steps) issue(s_begin + q + NS - 1u, (ST + NS - 1u) % NS);
        compute(s_begin + q, ST);
    };
    for (std::uint32_t q = 0; q < steps; q += NS) {
        step(q, std::integral_constant<unsigned, 0>{});
        if (q + 1u < steps) step(q + 1u, std::integral_constant<unsigned, 1>{});
        if constexpr (NS > 2) {
            if (q + 2u < steps) step(q + 2u, std::integral_constant<unsigned, 2>{});
        }
        if constexpr (NS > 3) {
            if (q + 3u < steps) step(q + 3u, std::integral_constant<unsigned, 3>{});
        }
    }

    // D[row = activation row][col = weight row], as skinny_kernel.
    float4v inv[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) inv[t] = reinterpret_cast<const float4v*>(a.inv_scale)[t * 4 + (lane >> 4)];
    float* out = a.out + (a.partial ? static_cast<std::uint64_t>(split) * a.m * a.n : 0u);
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const std::uint64_t n = static_cast<std::uint64_t>(rt0 + static_cast<std::uint32_t>(j)) * 16u + (lane & 15u);
        if (n >= a.n) continue;
        const float bn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const std::uint32_t m = static_cast<std::uint32_t>(t) * 16u + 4u * (lane >> 4) + static_cast<std::uint32_t>(i);
                if (m < a.m) skinny_store(a, out, split, m, n, acc[j][t][i] * inv[t][i] + bn);
            }
        }
    }
}

// Row-scaled activation split: one workgroup per padded row.  Pass 1 finds
// the row's max |x|; pass 2 writes the hi/lo fragments of every (block,
// eighth) run and the block sums of the scaled values.
__global__ __launch_bounds__(kSplitThreads) void split_rows_kernel(const float* __restrict__ x, std::uint32_t M,
                                                              std::uint64_t K, std::uint64_t nb, std::uint32_t mp,
                                                              uint4* __restrict__ xs, float* __restrict__ block_sums,
                                                              float* __restrict__ inv_scale) {
    __shared__ float red[kSplitThreads / 64];
    const std::uint32_t m = blockIdx.x;
    const bool row_live = m < M;
    const float* in = x + static_cast<std::uint64_t>(m) * K;
    // Rows of up to kHeldRuns * 1024 runs (K <= 32768) are read once and held
    // in registers for the split; longer rows are read twice.
    constexpr unsigned kHeldRuns = 4;
    const bool held = nb * 4u <= kHeldRuns * kSplitThreads;
    float4v part[kHeldRuns][2];
    float amax = 0.0f;
    if (held) {
#pragma unroll
        for (unsigned i = 0; i < kHeldRuns; ++i) {
            const std::uint64_t r = threadIdx.x + kSplitThreads * i;
            const std::uint64_t b = r >> 2;
            if (row_live && r < nb * 4u && b * 32u < K) {
                const float4v* src = reinterpret_cast<const float4v*>(in + b * 32u + 8u * (r & 3u));
                part[i][0] = src[0];
                part[i][1] = src[1];
            } else {
                part[i][0] = float4v{0.f, 0.f, 0.f, 0.f};
                part[i][1] = float4v{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int h = 0; h < 2; ++h)
#pragma unroll
                for (int e = 0; e < 4; ++e) amax = fmaxf(amax, fabsf(part[i][h][e]));
        }
    } else if (row_live) {
        for (std::uint64_t c = threadIdx.x * 4u; c < K; c += kSplitThreads * 4u) {
            const float4 v = *reinterpret_cast<const float4*>(in + c);
            amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
        }
    }
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (unsigned w = 1; w < kSplitThreads / 64; ++w) amax = fmaxf(amax, red[w]);
    float s, inv;
    block_scale(amax, s, inv);
    const auto emit = [&](std::uint64_t r, const float (&v)[8]) __attribute__((always_inline)) {
        emit_split_run(r, v, s, m, mp, xs, block_sums);
    };
    if (held) {
#pragma unroll
        for (unsigned i = 0; i < kHeldRuns; ++i) {
            const std::uint64_t r = threadIdx.x + kSplitThreads * i;
            if (r >= nb * 4u) break;  // uniform per aligned group of four lanes
            const float v[8] = {part[i][0][0], part[i][0][1], part[i][0][2], part[i][0][3],
                                part[i][1][0], part[i][1][1], part[i][1][2], part[i][1][3]};
            emit(r, v);
        }
        if (threadIdx.x == 0) inv_scale[m] = inv;
        return;
    }
    // Runs of 8: run r = 4 * block + g; the four runs of a block are adjacent lanes.
    for (std::uint64_t r = threadIdx.x; r < nb * 4u; r += kSplitThreads) {
        const std::uint64_t b = r >> 2;
        const std::uint32_t g = static_cast<std::uint32_t>(r & 3u);
        float v[8];
        if (row_live && b * 32u < K) {
            const float4* src = reinterpret_cast<const float4*>(in + b * 32u + 8u * g);
            const float4 p = src[0], q = src[1];
            v[0] = p.x; v[1] = p.y; v[2] = p.z; v[3] = p.w;
            v[4] = q.x; v[5] = q.y; v[6] = q.z; v[7] = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = 0.0f;
        }
        (void)g;
        emit(r, v);
    }
    if (threadIdx.x == 0) inv_scale[m] = inv;
}

template <int FMT, int MT, bool XF>
hipError_t launch_mt(const SkinnyArgs& a, std::uint32_t tn, std::uint32_t blocks, hipStream_t stream) {
    if (tn == 2u) {
        hipLaunchKernelGGL((skinny_kernel<FMT, MT, 2, XF>), dim3(blocks), dim3(kThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL((skinny_kernel<FMT, MT, 1, XF>), dim3(blocks), dim3(kThreads), 0, stream, a);
    }
    return hipGetLastError();
}

template <int FMT, bool XF>
hipError_t launch_fmt(const SkinnyArgs& a, const SkinnyShape& shape, std::uint32_t blocks, hipStream_t stream) {
    if (shape.waves != 4u) return hipErrorInvalidConfiguration;   // eight waves: the LDS pipeline only
    switch (shape.mt) {
    case 1: return launch_mt<FMT, 1, XF>(a, shape.tile_n, blocks, stream);
    case 2: return launch_mt<FMT, 2, XF>(a, shape.tile_n, blocks, stream);
    case 3: return launch_mt<FMT, 3, XF>(a, shape.tile_n, blocks, stream);
    default: return launch_mt<FMT, 4, XF>(a, shape.tile_n, blocks, stream);
    }
}

template <int FMT, int MT>
hipError_t launch_lds_mt(const SkinnyArgs& a, const SkinnyShape& shape, std::uint32_t blocks, hipStream_t stream) {
    const bool two = shape.tile_n == 2u;
    if (shape.waves == 8u) {
        // Eight waves: two or four activation tiles, two stages.
        if constexpr (MT == 2 || MT == 4) {
            if (shape.lds_stages != 2u) return hipErrorInvalidConfiguration;
            if (two) hipLaunchKernelGGL((skinny_lds_kernel<FMT, MT, 2, 2, 8>), dim3(blocks), dim3(512), 0, stream, a);
            else hipLaunchKernelGGL((skinny_lds_kernel<FMT, MT, 1, 2, 8>), dim3(blocks), dim3(512), 0, stream, a);
            return hipGetLastError();
        }
        return hipErrorInvalidConfiguration;
    }
    if (shape.waves != 4u) return hipErrorInvalidConfiguration;
    switch (shape.lds_stages) {
    case 2:
        if (two) hipLaunchKernelGGL((skinny_lds_kernel<FMT, MT, 2, 2>), dim3(blocks), dim3(kThreads), 0, stream, a);
        else hipLaunchKernelGGL((skinny_lds_kernel<FMT, MT, 1, 2>), dim3(blocks), dim3(kThreads), 0, stream, a);
        break;
    case 3:
        if (two) hipLaunchKernelGGL((skinny_lds_kernel<FMT, MT, 2, 3>), dim3(blocks), dim3(kThreads), 0, stream, a);
        else hipLaunchKernelGGL((skinny_lds_kernel<FMT, MT, 1, 3>), dim3(blocks), dim3(kThreads), 0, stream, a);
        break;
    default:
        if (two) hipLaunchKernelGGL((skinny_lds_kernel<FMT, MT, 2, 4>), dim3(blocks), dim3(kThreads), 0, stream, a);
        else hipLaunchKernelGGL((skinny_lds_kernel<FMT, MT, 1, 4>), dim3(blocks), dim3(kThreads), 0, stream, a);
        break;
    }
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_lds_fmt(const SkinnyArgs& a, const SkinnyShape& shape, std::uint32_t blocks, hipStream_t stream) {
    switch (shape.mt) {
    case 1: return launch_lds_mt<FMT, 1>(a, shape, blocks, stream);
    case 2: return launch_lds_mt<FMT, 2>(a, shape, blocks, stream);
    case 3: return launch_lds_mt<FMT, 3>(a, shape, blocks, stream);
    default: return launch_lds_mt<FMT, 4>(a, shape, blocks, stream);
    }
}

hipError_t launch_lds(int type, const SkinnyArgs& a, const SkinnyShape& shape, std::uint32_t blocks,
                      hipStream_t stream) {
    switch (type) {
    case kQ8_0: return launch_lds_fmt<kQ8_0>(a, shape, blocks, stream);
    case kQ4_0: return launch_lds_fmt<kQ4_0>(a, shape, blocks, stream);
    case kQ4_K: return launch_lds_fmt<kQ4_K>(a, shape, blocks, stream);
    default: return hipErrorInvalidValue;
    }
}

template <bool XF>
hipError_t launch_any(const TilePlanes& p, const SkinnyArgs& a, const SkinnyShape& shape, std::uint32_t blocks,
                      hipStream_t stream) {
    switch (p.type) {
    case kQ8_0: return launch_fmt<kQ8_0, XF>(a, shape, blocks, stream);
    case kQ4_0: return launch_fmt<kQ4_0, XF>(a, shape, blocks, stream);
    case kQ4_K: return launch_fmt<kQ4_K, XF>(a, shape, blocks, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace

hipError_t launch_split_activations_rows(const float* x, std::uint32_t m, std::uint64_t k, std::uint64_t kp,
                                         const SplitWorkspace& ws, hipStream_t stream) {
    if (m == 0u || m > 64u) return hipErrorInvalidValue;
    const std::uint32_t mp = static_cast<std::uint32_t>(ceil_div(m, 16u) * 16u);
    hipLaunchKernelGGL(split_rows_kernel, dim3(mp), dim3(kSplitThreads), 0, stream, x, m, k, kp / 32u, mp,
                       static_cast<uint4*>(ws.xs), ws.block_sums, ws.inv_scale);
    return hipGetLastError();
}

SkinnyShape plan_skinny(const TilePlanes& p, std::uint32_t m, std::uint32_t tile_n, std::uint32_t k_splits,
                        std::uint32_t lds_stages, std::uint32_t waves) {
    SkinnyShape s;
    s.mt = static_cast<std::uint32_t>(ceil_div(m, 16u));
    // The LDS pipeline (split activations): two stages measured best (three
    // and four never helped).  Q8_0 takes it on every 7B matrix except the
    // lm_head at M <= 32, where the register pipeline with two tiles per wave
    // wins (132 vs 146 us); Q4_K everywhere (gate|up 70 -> 48 us at M = 32,
    // 105 -> 75 at M = 64; down 55 -> 37 at M = 32; lm_head M = 32 157 us
    // against 208); Q4_0 from 17 rows (M = 64: q|k|v 31 -> 21 us, gate|up
    // 66 -> 57, down 51 -> 44), except its lm_head at M <= 32 (132 us on
    // registers with two tiles, 157 on LDS) and its gate|up below 33 rows
    // (registers with two tiles: 42.4 / 44.8 us at M = 17 / 32 against 46.0 /
    // 46.5 on LDS; at M <= 16 29 vs 33 us).
    if (lds_stages == 0u) {
        const bool narrow_or_tall = p.nt <= 4096u || s.mt >= 3u;
        const bool q4_0_gate_up = p.nt >= 2000u && p.nt <= 4096u && s.mt <= 2u;
        const bool lds = p.type == kQ8_0   ? narrow_or_tall
                         : p.type == kQ4_0 ? s.mt >= 2u && narrow_or_tall && !q4_0_gate_up
                                           : true;
        lds_stages = lds ? 2u : 1u;
    }
    s.lds_stages = lds_stages >= 2u ? lds_stages : 0u;
    // Two weight tiles per wave halve the LDS activation reads per weight
    // byte; with three or more activation tiles they would spill registers
    // (the in-workgroup split of the f32 variant holds more live values).
    // Automatic choice, measured on the Qwen2-7B shapes: two tiles only pay
    // for matrices of 2000..4096 row tiles (gate|up) at M <= 32, and not for
    // the 4-bit formats on the LDS pipeline (Q4_K gate|up M = 32: 52 vs 48 us).
    // lm_head-sized matrices (9504 row tiles) also take two at M <= 32 on the
    // register pipeline (M = 32: 155 -> 132 us), and so does the Q4_K one on
    // the LDS pipeline (M = 17 / 32: 154.8 -> 145.5 / 165.6 -> 154.4 us).
    const std::uint32_t tn2_max_mt = 2u;
    const bool tn2_auto = s.mt <= 2u && p.nt >= 2000u &&
                          (p.type == kQ8_0 || s.lds_stages == 0u || (p.type == kQ4_K && p.nt > 4096u));
    const std::uint32_t want = tile_n != 0u ? tile_n : (tn2_auto ? 2u : 1u);
    s.tile_n = (want == 2u && s.mt <= tn2_max_mt) ? 2u : 1u;
    // Eight waves per workgroup: the LDS pipeline with two stages and two or
    // four activation tiles.  Automatic for Q8_0 gate|up-sized matrices at
    // 17..32 rows, with one weight tile per wave (45.5 -> 44.0 us at M = 32),
    // and for lm_head-sized Q8_0 and Q4_0 matrices at 49..64 rows (229 -> 199
    // us and 216 -> 192); measured even or slower on every other 7B matrix,
    // width and format (Q4_K lm_head at 64 rows 251 -> 298).
    const bool eight_auto = waves == 0u && tile_n == 0u &&
                            ((p.type == kQ8_0 && s.mt == 2u && p.nt >= 2000u && p.nt <= 4096u) ||
                             ((p.type == kQ8_0 || p.type == kQ4_0) && s.mt == 4u && p.nt > 4096u));
    const bool eight = (waves == 8u || eight_auto) && s.lds_stages == 2u && (s.mt == 2u || s.mt == 4u);
    s.waves = eight ? 8u : 4u;
    if (eight_auto && eight) s.tile_n = 1u;
    s.groups = static_cast<std::uint32_t>(ceil_div(p.nt, s.waves * s.tile_n));
    s.steps = static_cast<std::uint32_t>(p.kp / kStepK);
    std::uint32_t splits = k_splits;
    if (splits == 0u) {
        // Up to about four workgroups per CU (two with three or four
        // activation tiles, whose registers and LDS halve the resident
        // workgroups), keeping at least 4 steps per split and the partials'
        // round trip (mostly cache-resident) within twice the weight bytes.
        // Measured on the Qwen2-7B shapes at M = 16..64 in all three formats.
        const std::uint64_t weight_bytes = static_cast<std::uint64_t>(p.nt) * p.kt * geometry_of(p.type).code_tile_bytes;
        const std::uint64_t partial_trip = 2u * static_cast<std::uint64_t>(m) * p.n * 4u;
        const std::uint64_t max_groups = s.mt <= 2u ? 1024u : 512u;
        splits = 1u;
        while (static_cast<std::uint64_t>(s.groups) * splits * 2u <= max_groups && s.steps / (splits * 2u) >= 4u &&
               partial_trip * splits * 2u <= 2u * weight_bytes) {
            splits *= 2u;
        }
        // Q4_K on wide grids (gate|up, 592 groups of one tile) at M <= 32
        // takes two splits past that limit: 45.1 -> 37.6 us at M = 16, 54.8
        // -> 50.6 at M = 32 (three or four splits slower; M = 64 even).
        if (p.type == kQ4_K && s.mt <= 2u && p.nt >= 2000u && p.nt <= 4096u && s.lds_stages >= 2u && splits < 2u) {
            splits = 2u;
        }
    }
    splits = splits < 1u ? 1u : (splits > s.steps ? s.steps : splits);
    s.steps_per_split = static_cast<std::uint32_t>(ceil_div(s.steps, splits));
    s.splits = static_cast<std::uint32_t>(ceil_div(s.steps, s.steps_per_split));
    return s;
}

std::uint64_t skinny_partials_bytes(const SkinnyShape& shape, std::uint32_t m, std::uint64_t n) {
    return shape.splits > 1u ? static_cast<std::uint64_t>(shape.splits) * m * n * 4u : 0u;
}

hipError_t launch_skinny_linear(const TilePlanes& p, const SplitWorkspace& ws, const float* bias, float* y,
                                std::uint32_t m, const SkinnyShape& shape, float* partials, hipStream_t stream,
                                const SplitEpilogue* epilogue, std::uint64_t* chain) {
    if (m == 0u || m > 64u || shape.mt != ceil_div(m, 16u)) return hipErrorInvalidValue;
    SkinnyArgs a{};
    a.codes = p.codes;
    a.scales = p.scales;
    a.nt = p.nt;
    a.kt = p.kt;
    a.n = p.n;
    a.xs = static_cast<const uint4*>(ws.xs);
    a.inv_scale = ws.inv_scale;
    a.block_sums = ws.block_sums;
    a.m = m;
    a.groups = shape.groups;
    a.steps = shape.steps;
    a.steps_per_split = shape.steps_per_split;
    const bool split = shape.splits > 1u;
    const bool chained = split && chain && !epilogue;
    a.partial = split ? 1u : 0u;
    a.bias = split ? nullptr : bias;
    a.out = split ? partials : y;
    if (chained) {
        a.chain = chain;
        a.y = y;
        a.chain_bias = bias;
        a.splits = shape.splits;
    }
    const std::uint32_t blocks = shape.groups * shape.splits;
    const hipError_t err = shape.lds_stages >= 2u ? launch_lds(p.type, a, shape, blocks, stream)
                                                  : launch_any<false>(p, a, shape, blocks, stream);
    if (err != hipSuccess || !split || chained) return err;
    if (epilogue) return launch_split_epilogue(partials, shape.splits, m, p.n, bias, *epilogue, stream);
    return launch_split_reduce(partials, shape.splits, m, p.n, bias, y, stream);
}

hipError_t launch_skinny_linear_x(const TilePlanes& p, const float* x, const float* bias, float* y, std::uint32_t m,
                                  const SkinnyShape& shape, float* partials, hipStream_t stream,
                                  const SplitEpilogue* epilogue, std::uint64_t* chain) {
    if (m == 0u || m > 64u || shape.mt != ceil_div(m, 16u) || p.k % 32u != 0u) return hipErrorInvalidValue;
    SkinnyArgs a{};
    a.x = x;
    a.k = p.k;
    a.codes = p.codes;
    a.scales = p.scales;
    a.nt = p.nt;
    a.kt = p.kt;
    a.n = p.n;
    a.m = m;
    a.groups = shape.groups;
    a.steps = shape.steps;
    a.steps_per_split = shape.steps_per_split;
    const bool split = shape.splits > 1u;
    const bool chained = split && chain && !epilogue;
    a.partial = split ? 1u : 0u;
    a.bias = split ? nullptr : bias;
    a.out = split ? partials : y;
    if (chained) {
        a.chain = chain;
        a.y = y;
        a.chain_bias = bias;
        a.splits = shape.splits;
    }
    const std::uint32_t blocks = shape.groups * shape.splits;
    const hipError_t err = launch_any<true>(p, a, shape, blocks, stream);
    if (err != hipSuccess || !split || chained) return err;
    if (epilogue) return launch_split_epilogue(partials, shape.splits, m, p.n, bias, *epilogue, stream);
    return launch_split_reduce(partials, shape.splits, m, p.n, bias, y, stream);
}

} // namespace air_hip

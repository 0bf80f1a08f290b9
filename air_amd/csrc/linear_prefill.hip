// linear_prefill.hip -- prefill-sized linears (M = 65..4096) on f16 MFMA.
//
// The reference runs prefill linears through the same f32 kernels as decode
// (specialized_matmul / batch_reuse, src/cuda/cuda_backend.cu:501-583), so a
// 512-token prefill decodes every weight 64 times.  Here a prefill linear is a
// GEMM on the matrix cores:
//
//   1. prefill_activations_kernel: x f32 [M][K] -> xh f16 [Mp][Kx], each row
//      scaled by a power of two so that its max |x| lies in [2^14, 2^15)
//      (no f16 overflow, no needless subnormals); row_inv[m] undoes it.
//   2. prefill_gemm_kernel: each workgroup owns BM = 16*TM activation rows and
//      4*TN 16-row weight tiles; each of its four waves owns TN weight tiles.
//      Per 64-k step the activation tile is staged through LDS (it is shared
//      by all four waves) while every wave streams its own weight codes from
//      the resident tile layout, dequantizes them to f16 in registers
//      (w = code * f16(d * 2^-e), exact codes, one rounding) and feeds them as
//      the A operand of v_mfma_f32_16x16x32_f16; the LDS activation fragments
//      are the B operand.  The lane layout of the resident records is the MFMA
//      operand layout, so weights never pass through LDS: no wave reads
//      another wave's weights.  Accumulation is f32.
//   3. With a K split, prefill_reduce_kernel sums the split partials in a
//      fixed order (deterministic) and adds the bias.
//
// The weight exponent e is chosen per matrix when it becomes resident
// (prefill_bound_kernel): max |w| * 2^-e <= 2^15.  Outputs are
// acc * row_inv[m] * 2^e + bias[n].
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"
#include "air_hip_steps.hpp"

#include <algorithm>
#include <cmath>
#include <type_traits>
#include <cstring>

namespace air_hip {
namespace {

constexpr unsigned kThreads = 256;       // four waves
constexpr unsigned kLdsStride = kStepK + 8;  // halfs per staged activation row

// ---- 1. activations ----------------------------------------------------

// One workgroup per padded row.  Row scale as block_scale, over the whole row.
__global__ __launch_bounds__(kThreads) void prefill_activations_kernel(const float* __restrict__ x, std::uint32_t m,
                                                                       std::uint64_t k, std::uint64_t ldx,
                                                                       _Float16* __restrict__ xh,
                                                                       float* __restrict__ row_inv) {
    __shared__ float red[kThreads / 64];
    const std::uint32_t row = blockIdx.x;
    _Float16* out = xh + static_cast<std::uint64_t>(row) * ldx;
    if (row >= m) {
        for (std::uint64_t c = threadIdx.x * 8u; c < ldx; c += kThreads * 8u) {
            *reinterpret_cast<uint4*>(out + c) = make_uint4(0u, 0u, 0u, 0u);
        }
        if (threadIdx.x == 0) row_inv[row] = 1.0f;
        return;
    }
    const float* in = x + static_cast<std::uint64_t>(row) * k;
    float amax = 0.0f;
    for (std::uint64_t c = threadIdx.x * 4u; c < k; c += kThreads * 4u) {
        const float4 v = *reinterpret_cast<const float4*>(in + c);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float s, inv;
    block_scale(amax, s, inv);
    for (std::uint64_t c = threadIdx.x * 8u; c < ldx; c += kThreads * 8u) {
        half8v h;
        if (c < k) {  // k is a multiple of 32, so a run of 8 is all in or all out
            const float4 a = *reinterpret_cast<const float4*>(in + c);
            const float4 b = *reinterpret_cast<const float4*>(in + c + 4);
            h[0] = static_cast<_Float16>(a.x * s); h[1] = static_cast<_Float16>(a.y * s);
            h[2] = static_cast<_Float16>(a.z * s); h[3] = static_cast<_Float16>(a.w * s);
            h[4] = static_cast<_Float16>(b.x * s); h[5] = static_cast<_Float16>(b.y * s);
            h[6] = static_cast<_Float16>(b.z * s); h[7] = static_cast<_Float16>(b.w * s);
        } else {
            for (int e = 0; e < 8; ++e) h[e] = static_cast<_Float16>(0.0f);
        }
        *reinterpret_cast<half8v*>(out + c) = h;
    }
    if (threadIdx.x == 0) row_inv[row] = inv;
}

// The same conversion reading the row once: thread t holds the runs of 8
// floats at (t + 256 j) * 8 for j < C in registers, so the row's max and
// its conversion take one pass over memory instead of two (same scale, same
// per-element arithmetic: bit-identical).  Rows with ldx <= 2048 * C.
template <int C>
__global__ __launch_bounds__(kThreads) void prefill_activations_reg_kernel(const float* __restrict__ x,
                                                                           std::uint32_t m, std::uint64_t k,
                                                                           std::uint64_t ldx,
                                                                           _Float16* __restrict__ xh,
                                                                           float* __restrict__ row_inv) {
    __shared__ float red[kThreads / 64];
    const std::uint32_t row = blockIdx.x;
    _Float16* out = xh + static_cast<std::uint64_t>(row) * ldx;
    if (row >= m) {
        for (std::uint64_t c = threadIdx.x * 8u; c < ldx; c += kThreads * 8u) {
            *reinterpret_cast<uint4*>(out + c) = make_uint4(0u, 0u, 0u, 0u);
        }
        if (threadIdx.x == 0) row_inv[row] = 1.0f;
        return;
    }
    const float* in = x + static_cast<std::uint64_t>(row) * k;
    float4 v[C][2];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const std::uint64_t c = (threadIdx.x + kThreads * static_cast<std::uint64_t>(j)) * 8u;
        if (c < k) {  // k is a multiple of 32, so a run of 8 is all in or all out
            v[j][0] = *reinterpret_cast<const float4*>(in + c);
            v[j][1] = *reinterpret_cast<const float4*>(in + c + 4);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[j][h].x), fabsf(v[j][h].y)),
                                         fmaxf(fabsf(v[j][h].z), fabsf(v[j][h].w))));
            }
        }
    }
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float s, inv;
    block_scale(amax, s, inv);
#pragma unroll
    for (int j = 0; j < C; ++j) {
        const std::uint64_t c = (threadIdx.x + kThreads * static_cast<std::uint64_t>(j)) * 8u;
        if (c >= ldx) continue;
        half8v h;
        if (c < k) {
            const float4 a = v[j][0], b = v[j][1];
            h[0] = static_cast<_Float16>(a.x * s); h[1] = static_cast<_Float16>(a.y * s);
            h[2] = static_cast<_Float16>(a.z * s); h[3] = static_cast<_Float16>(a.w * s);
            h[4] = static_cast<_Float16>(b.x * s); h[5] = static_cast<_Float16>(b.y * s);
            h[6] = static_cast<_Float16>(b.z * s); h[7] = static_cast<_Float16>(b.w * s);
        } else {
            for (int e = 0; e < 8; ++e) h[e] = static_cast<_Float16>(0.0f);
        }
        *reinterpret_cast<half8v*>(out + c) = h;
    }
    if (threadIdx.x == 0) row_inv[row] = inv;
}

// One launch converting rows [0, mp) of x (rows >= m zero-filled).
hipError_t launch_prefill_activations(const float* x, std::uint32_t m, std::uint64_t k, std::uint64_t ldx,
                                      std::uint64_t mp, _Float16* xh, float* row_inv, hipStream_t stream) {
    const dim3 grid(static_cast<unsigned>(mp)), block(kThreads);
    const std::uint64_t chunks = ceil_div(ldx, 8u * kThreads);
    if (chunks <= 2u) {
        hipLaunchKernelGGL(prefill_activations_reg_kernel<2>, grid, block, 0, stream, x, m, k, ldx, xh, row_inv);
    } else if (chunks <= 4u) {
        hipLaunchKernelGGL(prefill_activations_reg_kernel<4>, grid, block, 0, stream, x, m, k, ldx, xh, row_inv);
    } else if (chunks <= 8u) {
        hipLaunchKernelGGL(prefill_activations_reg_kernel<8>, grid, block, 0, stream, x, m, k, ldx, xh, row_inv);
    } else if (chunks <= 12u) {
        hipLaunchKernelGGL(prefill_activations_reg_kernel<12>, grid, block, 0, stream, x, m, k, ldx, xh, row_inv);
    } else {
        hipLaunchKernelGGL(prefill_activations_kernel, grid, block, 0, stream, x, m, k, ldx, xh, row_inv);
    }
    return hipGetLastError();
}

// ---- weight fragments -----------------------------------------------------

__device__ __forceinline__ _Float16 scaled_half(std::uint32_t bits, float w_scale) {
    const float v = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(bits))) * w_scale;
    return static_cast<_Float16>(v);
}

// f16 weights of block b (0, 1) of the step (A fragment: row l%16, k 8(l/16)+e).
template <int FMT>
__device__ __forceinline__ half8v dequant_block(const StepCodes<FMT>& in, std::uint32_t s, int b, float w_scale) {
    half8v w;
    if constexpr (FMT == kQ8_0) {
        const std::uint32_t lo = b == 0 ? in.c.x : in.c.z;
        const std::uint32_t hi = b == 0 ? in.c.y : in.c.w;
        half2v p0, p1, p2, p3;
        q8_dword_to_half(lo, p0, p1);
        q8_dword_to_half(hi, p2, p3);
        const _Float16 d = scaled_half((in.d >> (16 * b)) & 0xffffu, w_scale);
        const half2v dd = {d, d};
        p0 *= dd; p1 *= dd; p2 *= dd; p3 *= dd;
        w[0] = p0[0]; w[1] = p0[1]; w[2] = p1[0]; w[3] = p1[1];
        w[4] = p2[0]; w[5] = p2[1]; w[6] = p3[0]; w[7] = p3[1];
    } else if constexpr (FMT == kQ4_0) {
        const _Float16 d = scaled_half((in.d >> (16 * b)) & 0xffffu, w_scale);
        w = nibble_dword_to_half8<8>(b == 0 ? in.c.x : in.c.y) * d;
    } else if constexpr (FMT == kF16) {
        // Exact f16 rows: the weight exponent of F16 storage is 0.
        (void)w_scale;
        w = __builtin_bit_cast(half8v, in.v[b]);
    } else if constexpr (FMT == kBF16) {
        // bf16 -> f32 (exact) -> scaled -> f16 (one rounding).
        const u32x4 v = in.v[b];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            w[2 * e] = static_cast<_Float16>(__uint_as_float(v[e] << 16) * w_scale);
            w[2 * e + 1] = static_cast<_Float16>(__uint_as_float(v[e] & 0xffff0000u) * w_scale);
        }
    } else if constexpr (FMT == kQ6_K) {
        // Codes q - 32 as exact f16 (1024 + q under the exponent byte 0x64,
        // minus 1056) times f16(d * sc * 2^-e): one rounding per weight.
        const std::uint32_t q = s & 3u;
        const std::uint32_t j = 2u * (q & 1u) + static_cast<std::uint32_t>(b);
        const std::uint32_t g = (threadIdx.x & 63u) >> 4;
        const int sc = static_cast<int>(static_cast<std::int8_t>((in.sc >> (8u * (2u * b + (g >> 1)))) & 0xffu));
        const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(in.d)));
        const _Float16 ds = static_cast<_Float16>(d * static_cast<float>(sc) * w_scale);
        const half2v dd = {ds, ds};
        const half2v bias = {(_Float16)1056.0f, (_Float16)1056.0f};
        const u32x2 lq = in.ql[b];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const std::uint32_t nib = ((q & 1u) ? (lq[e] >> 4) : lq[e]) & 0x0f0f0f0fu;
            const std::uint32_t hq = in.qh[e];
            const std::uint32_t hib = (j <= 2u ? (hq << (4u - 2u * j)) : (hq >> (2u * j - 4u))) & 0x30303030u;
            const std::uint32_t u = nib | hib;
            const half2v lo = (bits_as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias) * dd;
            const half2v hi = (bits_as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias) * dd;
            w[4 * e] = lo[0]; w[4 * e + 1] = lo[1]; w[4 * e + 2] = hi[0]; w[4 * e + 3] = hi[1];
        }
    } else {
        const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(in.h.x & 0xffffu)));
        const float dmin = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(in.h.x >> 16)));
        const std::uint32_t packed[3] = {in.h.y, in.h.z, in.h.w};
        std::uint32_t sc = 0, mn = 0;
        q4k_scale_min(packed, 2u * (s & 3u) + static_cast<std::uint32_t>(b), sc, mn);
        const _Float16 a = static_cast<_Float16>(d * static_cast<float>(sc) * w_scale);
        const _Float16 o = static_cast<_Float16>(dmin * static_cast<float>(mn) * w_scale);
        w = nibble_dword_to_half8<0>(b == 0 ? in.c.x : in.c.y) * a - o;
    }
    return w;
}

// ---- 2. GEMM --------------------------------------------------------------

struct GemmArgs {
    const void* codes;
    const void* scales;
    std::uint32_t nt, kt;        // tile grid of the matrix
    std::uint64_t n;
    const _Float16* xh;          // [Mp][ldx]
    std::uint64_t ldx;
    const float* row_inv;        // [Mp]
    float w_scale, w_unscale;
    const float* bias;           // [n] or null (ignored when splits > 1)
    float* out;                  // y [m][ldo], or partials [splits][m][ldo]
    std::uint64_t ldo;           // row stride of out (n, or the partials' column count)
    std::uint64_t col0;          // first column that out holds
    std::uint32_t m;
    std::uint32_t m_tiles;       // ceil(m / BM)
    std::uint32_t groups;        // ceil(nt / (4 * TN))
    std::uint32_t steps;         // 64-k steps of the padded k
    std::uint32_t steps_per_split;
    std::uint32_t partial;       // 1: write split partials (no bias)
    std::uint32_t blocks;        // logical workgroups: m_tiles * groups * splits
    std::uint32_t rt_base;       // first row tile of the launch
};

// D[row = weight row][col = activation row]: lane holds rows 4(l/16)+r of
// column l%16; outputs are acc * row_inv[m] * 2^e (+ bias[n]).
template <int TM, int TN>
__device__ __forceinline__ void store_tile(const GemmArgs& a, const float4v (&acc)[TM][TN], std::uint32_t m0,
                                           std::uint32_t rt0, std::uint32_t split, std::uint32_t lane) {
    float* out = a.out + (a.partial ? static_cast<std::uint64_t>(split) * a.m * a.ldo : 0u);
    const bool vec = (a.n & 3u) == 0u && (a.ldo & 3u) == 0u && (a.col0 & 3u) == 0u;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const std::uint32_t m = m0 + static_cast<std::uint32_t>(i) * 16u + (lane & 15u);
        if (m >= a.m) continue;
        const float scale = a.row_inv[m] * a.w_unscale;
        float* yrow = out + static_cast<std::uint64_t>(m) * a.ldo;
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const std::uint64_t n0 = static_cast<std::uint64_t>(rt0 + static_cast<std::uint32_t>(t)) * 16u + 4u * (lane >> 4);
            if (n0 >= a.n) continue;
            float v[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                v[r] = acc[i][t][r] * scale;
                if (a.bias && n0 + r < a.n) v[r] += a.bias[n0 + r];
            }
            float* dst = yrow + (n0 - a.col0);   // n0 >= col0: the launch covers columns from col0 on
            if (vec && n0 + 4u <= a.n) {
                *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
                for (int r = 0; r < 4; ++r)
                    if (n0 + r < a.n) dst[r] = v[r];
            }
        }
    }
}

// The workgroup's tile of the logical grid (m-tiles fastest, then weight
// groups, then K splits), dealt to the eight XCDs in contiguous runs:
// hardware hands workgroup i to XCD i % 8, so the m-tiles of one weight
// group share that XCD's L2.  False for the padding workgroups of the last
// round.
struct GemmTile {
    std::uint32_t m0, rt0, split, s_begin, s_end;
};
template <int TM, int TN>
__device__ __forceinline__ bool gemm_tile(const GemmArgs& a, std::uint32_t wave, GemmTile& g) {
    const std::uint32_t per_xcd = (a.blocks + 7u) / 8u;
    std::uint32_t bid = (blockIdx.x & 7u) * per_xcd + (blockIdx.x >> 3);
    if (bid >= a.blocks) return false;
    const std::uint32_t mt = bid % a.m_tiles;
    bid /= a.m_tiles;
    const std::uint32_t group = bid % a.groups;
    g.split = bid / a.groups;
    g.m0 = mt * 16u * TM;
    g.rt0 = a.rt_base + (group * 4u + wave) * TN;
    g.s_begin = g.split * a.steps_per_split;
    g.s_end = min(a.steps, g.s_begin + a.steps_per_split);
    return true;
}

// PF = how many steps ahead the weight codes are fetched (1 or 2).  The
// largest register tile with PF = 2 runs at one wave per SIMD so that its
// accumulators fit (VGPR + AGPR).
template <int FMT, int TM, int TN, int PF>
__global__ __launch_bounds__(kThreads, (TM * TN >= 32 && PF == 2) ? 1 : 2) void prefill_gemm_kernel(GemmArgs a) {
    constexpr unsigned BM = 16u * TM;
    constexpr unsigned kChunks = BM * (kStepK / 8u) / kThreads;  // 16-byte activation chunks per thread
    static_assert(kChunks * kThreads == BM * (kStepK / 8u), "activation tile must split evenly");
    __shared__ __attribute__((aligned(16))) _Float16 xs[2][BM * kLdsStride];

    const std::uint32_t tid = threadIdx.x;
    const std::uint32_t lane = tid & 63u;
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
    GemmTile g;
    if (!gemm_tile<TM, TN>(a, wave, g)) return;
    const std::uint32_t m0 = g.m0, rt0 = g.rt0, split = g.split, s_begin = g.s_begin, s_end = g.s_end;

    float4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t) acc[i][t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    u32x4 xr[kChunks];
    const auto load_x = [&](std::uint32_t s) __attribute__((always_inline)) {
#pragma unroll
        for (unsigned j = 0; j < kChunks; ++j) {
            const std::uint32_t c = tid + kThreads * j;
            const std::uint32_t row = c >> 3, col = (c & 7u) * 8u;
            xr[j] = *reinterpret_cast<const u32x4*>(a.xh + static_cast<std::uint64_t>(m0 + row) * a.ldx +
                                                    static_cast<std::uint64_t>(s) * kStepK + col);
        }
    };
    const auto store_x = [&](unsigned buf) __attribute__((always_inline)) {
#pragma unroll
        for (unsigned j = 0; j < kChunks; ++j) {
            const std::uint32_t c = tid + kThreads * j;
            const std::uint32_t row = c >> 3, col = (c & 7u) * 8u;
            *reinterpret_cast<u32x4*>(&xs[buf][row * kLdsStride + col]) = xr[j];
        }
    };
    // Weight codes run PF steps ahead of the MFMAs: with PF = 2, while step
    // s computes, the codes of s+1 are resident and those of s+2 in flight.
    StepCodes<FMT> wa[TN], wb[TN];
    const auto load_w = [&](StepCodes<FMT>(&dst)[TN], std::uint32_t s) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const std::uint32_t rt = rt0 + static_cast<std::uint32_t>(t);
            if constexpr (dense_storage(FMT)) {
                load_dense_step<FMT>(a.codes, a.n, a.kt, rt, s, lane, dst[t]);
            } else {
                load_step<FMT>(a.codes, a.scales, rt, a.kt, s, lane, rt < a.nt, dst[t]);
            }
        }
    };
    // One pipeline step over codes `cur`; refills `cur` with step s+PF once
    // its last block is dequantized.
    const auto step = [&](std::uint32_t s, StepCodes<FMT>(&cur)[TN]) __attribute__((always_inline)) {
        const unsigned buf = (s - s_begin) & 1u;
        const bool more = s + 1u < s_end;
        if (more) load_x(s + 1u);
        const _Float16* xb = xs[buf];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            half8v w[TN];
#pragma unroll
            for (int t = 0; t < TN; ++t) w[t] = dequant_block<FMT>(cur[t], s, b, a.w_scale);
            if (b == 1 && s + PF < s_end) load_w(cur, s + PF);
            half8v xf[TM];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                xf[i] = *reinterpret_cast<const half8v*>(
                    xb + (static_cast<unsigned>(i) * 16u + (lane & 15u)) * kLdsStride + 32u * b + 8u * (lane >> 4));
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int t = 0; t < TN; ++t) acc[i][t] = mfma16x16x32(w[t], xf[i], acc[i][t]);
        }
        if (more) store_x(buf ^ 1u);
        __syncthreads();
    };

    if (s_begin < s_end) {
        load_x(s_begin);
        load_w(wa, s_begin);
        if (PF == 2 && s_begin + 1u < s_end) load_w(wb, s_begin + 1u);
        store_x(0);
    }
    __syncthreads();
    if constexpr (PF == 2) {
        std::uint32_t s = s_begin;
        for (; s + 1u < s_end; s += 2u) {
            step(s, wa);
            step(s + 1u, wb);
        }
        if (s < s_end) step(s, wa);
    } else {
        for (std::uint32_t s = s_begin; s < s_end; ++s) step(s, wa);
    }

    store_tile<TM, TN>(a, acc, m0, rt0, split, lane);
}

// ---- 2b. GEMM with an LDS load pipeline ------------------------------------
//
// The same workgroup tile and arithmetic as prefill_gemm_kernel, but every
// operand streams global -> LDS directly (global_load_lds_dwordx4: no
// staging registers), through a ring of NS stages of one 64-k step each, so
// loads run NS - 1 steps ahead of the MFMAs without holding VGPRs:
//
//   stage = [activation fragments: TM m-tiles x 2 blocks x 1 KiB]
//           [weight codes: 4 waves x TN tiles x 1 KiB]
//           [weight scales: 4 waves x TN tiles x 64 lanes x 4 B]
//
// Each KiB is one 64-lane x 16-byte MFMA fragment in lane order, exactly as
// a wave reads it back (ds_read_b128 at lane * 16: no bank conflicts).  The
// weight records of the resident layout are already in that order; an
// activation fragment is 16 rows x 8 halfs per lane group.  Each wave loads
// a quarter of the activation fragments and its own weight tiles, waits for
// its loads of the step about to be computed (vmcnt), and one barrier per
// step publishes the stage and frees the oldest one for the next load.
// Q8_0 only: one resident record per 64-k step (the 4-bit records span two).
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// Lane l's 16 (or 4) bytes land at lds_wave_base + l * 16 (l * 4).
__device__ __forceinline__ void load_lds16(const void* src, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds((global_void_t*)(const_cast<void*>(src)), (lds_void_t*)(lds_wave_base), 16, 0, 0);
}
__device__ __forceinline__ void load_lds4(const void* src, void* lds_wave_base) {
    __builtin_amdgcn_global_load_lds((global_void_t*)(const_cast<void*>(src)), (lds_void_t*)(lds_wave_base), 4, 0, 0);
}

// s_waitcnt for vmcnt <= n only (expcnt and lgkmcnt at their maxima).
template <unsigned n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n < 64u, "vmcnt is six bits");
    __builtin_amdgcn_s_waitcnt((n & 0xfu) | ((n >> 4) << 14) | (0x7u << 4) | (0xfu << 8));
}

template <int TM, int TN>
constexpr unsigned lds_stage_bytes() {
    return 2u * TM * 1024u + 4u * TN * 1024u + 4u * TN * 256u;
}

template <int FMT, int TM, int TN, int NS>
__global__ __launch_bounds__(kThreads, ((NS * lds_stage_bytes<TM, TN>()) <= 80u * 1024u ? 2 : 1)) void prefill_lds_kernel(GemmArgs a) {
    static_assert(FMT == kQ8_0, "one resident record per 64-k step");
    constexpr unsigned kStage = lds_stage_bytes<TM, TN>();
    constexpr unsigned kCodes = 2u * TM * 1024u;            // offset of the weight codes in a stage
    constexpr unsigned kScales = kCodes + 4u * TN * 1024u;  // offset of the weight scales
    constexpr unsigned kLoads = 2u * TM / 4u + 2u * TN;     // load instructions per wave per stage
    static_assert((2u * TM) % 4u == 0u, "activation fragments split over the four waves");
    static_assert(NS >= 2 && NS <= 4, "two to four stages");
    // One LDS object per stage, addressed with compile-time stage numbers:
    // the compiler's wait-count pass then sees that a stage's direct loads
    // and another stage's reads touch different objects (one array indexed
    // at run time makes it wait for every load in flight before any read).
    __shared__ __attribute__((aligned(1024))) unsigned char stage0[kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage1[kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage2[NS > 2 ? kStage : 16];
    __shared__ __attribute__((aligned(1024))) unsigned char stage3[NS > 3 ? kStage : 16];
    const auto stage = [&](unsigned st) __attribute__((always_inline)) -> unsigned char* {
        return st == 0u ? stage0 : st == 1u ? stage1 : st == 2u ? stage2 : stage3;
    };

    const std::uint32_t lane = threadIdx.x & 63u;
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    GemmTile g;
    if (!gemm_tile<TM, TN>(a, wave, g)) return;

    float4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t) acc[i][t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    // Per-lane global sources of step 0; a step advances them by 64 halfs
    // (activations) or one tile (weights).  Padded weight rows (rt >= nt)
    // read the last real tile: their outputs are never stored.
    const _Float16* xsrc[2 * TM / 4];
#pragma unroll
    for (unsigned j = 0; j < 2u * TM / 4u; ++j) {
        const unsigned f = wave + 4u * j, i = f >> 1, b = f & 1u;
        xsrc[j] = a.xh + static_cast<std::uint64_t>(g.m0 + i * 16u + (lane & 15u)) * a.ldx + 32u * b + 8u * (lane >> 4);
    }
    std::uint64_t wtile[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t) {
        const std::uint32_t rt = min(g.rt0 + static_cast<std::uint32_t>(t), a.nt - 1u);
        wtile[t] = static_cast<std::uint64_t>(rt) * a.kt;
    }
    const auto issue = [&](std::uint32_t s, std::uint32_t st) __attribute__((always_inline)) {
        unsigned char* base = stage(st);
#pragma unroll
        for (unsigned j = 0; j < 2u * TM / 4u; ++j) {
            load_lds16(xsrc[j] + static_cast<std::uint64_t>(s) * kStepK, base + (wave + 4u * j) * 1024u);
        }
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const std::uint64_t tile = wtile[t] + s;
            load_lds16(static_cast<const u32x4*>(a.codes) + tile * 64u + lane,
                         base + kCodes + (wave * TN + static_cast<unsigned>(t)) * 1024u);
            load_lds4(static_cast<const std::uint32_t*>(a.scales) + tile * 16u + (lane & 15u),
                        base + kScales + (wave * TN + static_cast<unsigned>(t)) * 256u);
        }
    };
    const auto compute = [&](std::uint32_t s, std::uint32_t st) __attribute__((always_inline)) {
        const unsigned char* base = stage(st);
        // Every LDS read of the step is issued before the first MFMA, so the
        // wave waits for LDS once per step rather than once per fragment pair.
        StepCodes<FMT> w_in[TN];
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const unsigned slot = wave * TN + static_cast<unsigned>(t);
            w_in[t].c = *reinterpret_cast<const u32x4*>(base + kCodes + slot * 1024u + lane * 16u);
            w_in[t].d = *reinterpret_cast<const std::uint32_t*>(base + kScales + slot * 256u + lane * 4u);
        }
        half8v xf[2][TM];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                xf[b][i] = *reinterpret_cast<const half8v*>(base + (static_cast<unsigned>(i) * 2u + b) * 1024u + lane * 16u);
            }
        __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the arithmetic
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            half8v w[TN];
#pragma unroll
            for (int t = 0; t < TN; ++t) w[t] = dequant_block<FMT>(w_in[t], s, b, a.w_scale);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int t = 0; t < TN; ++t) acc[i][t] = mfma16x16x32(w[t], xf[b][i], acc[i][t]);
        }
    };

    const std::uint32_t steps = g.s_end - g.s_begin;
#pragma unroll
    for (unsigned q = 0; q + 1u < NS; ++q) {
        if (q < steps) issue(g.s_begin + q, q);
    }
    // Step q of the split computes stage q mod NS (ST, a constant).
    const auto step = [&](std::uint32_t q, auto st_tag) __attribute__((always_inline)) {
        constexpr unsigned ST = decltype(st_tag)::value;
        // Stage ST is complete once at most the later stages' loads are in
        // flight; near the end fewer follow it, so wait for everything.
        if (q + NS - 2u < steps) {
            wait_vmcnt<kLoads * (NS - 2u)>();
        } else {
            wait_vmcnt<0u>();
        }
        // Every wave's reads of the previous stage are complete before the
        // barrier, after which that stage takes new loads; a bare s_barrier
        // (a fence would also wait for the loads still in flight).
        __builtin_amdgcn_s_waitcnt(0xc07fu);   // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        if (q + NS - 1u < steps) issue(g.s_begin + q + NS - 1u, (ST + NS - 1u) % NS);
        compute(g.s_begin + q, ST);
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
    store_tile<TM, TN>(a, acc, g.m0, g.rt0, g.split, lane);
}

// ---- 2c. GEMM: activations through an LDS ring, weights in registers ----
//
// prefill_lds_kernel's activation pipeline (direct global -> LDS loads of
// lane-ordered fragments, a ring of NS stages) with every wave's weight
// records loaded straight into registers one step ahead, as
// prefill_gemm_kernel loads them.  A wave's weights are read by that wave
// alone, so passing them through LDS only adds LDS traffic (their write and
// read back) beside the activation fragments that all four waves read; here
// a stage holds activations only (2 * TM KiB), and any storage format runs.
//
// Per step q a wave issues, in this order, the weights of step q + 1 (into
// the register set not being computed) and then the activation fragments of
// step q + NS - 1.  At the top of step q the fragments of step q must have
// landed: with two stages everything issued is waited for; with three, the
// last kA loads (the fragments of step q + 1) may stay in flight -- the
// weights of step q were issued before them, so they have landed too.
template <int FMT, int TM, int TN, int NS>
__global__ __launch_bounds__(kThreads, 2) void prefill_hyb_kernel(GemmArgs a) {
    constexpr unsigned kStage = 2u * TM * 1024u;
    constexpr unsigned kA = 2u * TM / 4u;   // activation fragment loads per wave per stage
    static_assert((2u * TM) % 4u == 0u, "activation fragments split over the four waves");
    static_assert(NS == 2 || NS == 3, "two or three stages");
    __shared__ __attribute__((aligned(1024))) unsigned char stage0[kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage1[kStage];
    __shared__ __attribute__((aligned(1024))) unsigned char stage2[NS > 2 ? kStage : 16];
    const auto stage = [&](unsigned st) __attribute__((always_inline)) -> unsigned char* {
        return st == 0u ? stage0 : st == 1u ? stage1 : stage2;
    };

    const std::uint32_t lane = threadIdx.x & 63u;
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    GemmTile g;
    if (!gemm_tile<TM, TN>(a, wave, g)) return;

    float4v acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t) acc[i][t] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    const _Float16* xsrc[kA];
#pragma unroll
    for (unsigned j = 0; j < kA; ++j) {
        const unsigned f = wave + 4u * j, i = f >> 1, b = f & 1u;
        xsrc[j] = a.xh + static_cast<std::uint64_t>(g.m0 + i * 16u + (lane & 15u)) * a.ldx + 32u * b + 8u * (lane >> 4);
    }
    const auto issue_x = [&](std::uint32_t s, std::uint32_t st) __attribute__((always_inline)) {
        unsigned char* base = stage(st);
#pragma unroll
        for (unsigned j = 0; j < kA; ++j) {
            load_lds16(xsrc[j] + static_cast<std::uint64_t>(s) * kStepK, base + (wave + 4u * j) * 1024u);
        }
    };
    const auto load_w = [&](StepCodes<FMT>(&dst)[TN], std::uint32_t s) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < TN; ++t) {
            const std::uint32_t rt = g.rt0 + static_cast<std::uint32_t>(t);
            if constexpr (dense_storage(FMT)) {
                load_dense_step<FMT>(a.codes, a.n, a.kt, rt, s, lane, dst[t]);
            } else {
                load_step<FMT>(a.codes, a.scales, rt, a.kt, s, lane, rt < a.nt, dst[t]);
            }
        }
    };
    const auto compute = [&](std::uint32_t s, std::uint32_t st, const StepCodes<FMT>(&w_in)[TN])
        __attribute__((always_inline)) {
        const unsigned char* base = stage(st);
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            half8v xf[TM];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                xf[i] = *reinterpret_cast<const half8v*>(base + (static_cast<unsigned>(i) * 2u + b) * 1024u + lane * 16u);
            }
            half8v w[TN];
#pragma unroll
            for (int t = 0; t < TN; ++t) w[t] = dequant_block<FMT>(w_in[t], s, b, a.w_scale);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int t = 0; t < TN; ++t) acc[i][t] = mfma16x16x32(w[t], xf[i], acc[i][t]);
        }
    };

    const std::uint32_t steps = g.s_end - g.s_begin;
    StepCodes<FMT> wa[TN], wb[TN];
    if (steps > 0u) load_w(wa, g.s_begin);
#pragma unroll
    for (unsigned q = 0; q + 1u < NS; ++q) {
        if (q < steps) issue_x(g.s_begin + q, q);
    }
    // Step q computes stage q mod NS (ST, a constant) with weight set `cur`
    // and loads the next step's weights into `nxt`.
    const auto step = [&](std::uint32_t q, auto st_tag, StepCodes<FMT>(&cur)[TN], StepCodes<FMT>(&nxt)[TN])
        __attribute__((always_inline)) {
        constexpr unsigned ST = decltype(st_tag)::value;
        if (NS == 3 && q + 1u < steps) {
            wait_vmcnt<kA>();
        } else {
            wait_vmcnt<0u>();
        }
        // Every wave's reads of the stage about to be refilled are complete
        // before the barrier (lgkmcnt(0)), after which it takes new loads.
        __builtin_amdgcn_s_waitcnt(0xc07fu);
        __builtin_amdgcn_s_barrier();
        if (q + 1u < steps) load_w(nxt, g.s_begin + q + 1u);
        if (q + NS - 1u < steps) issue_x(g.s_begin + q + NS - 1u, (ST + NS - 1u) % NS);
        compute(g.s_begin + q, ST, cur);
    };
    // The ring position and the weight set both alternate; a period of
    // 2 * NS steps keeps both compile-time.
    for (std::uint32_t q = 0; q < steps; q += 2u * NS) {
        step(q, std::integral_constant<unsigned, 0>{}, wa, wb);
        if (q + 1u < steps) step(q + 1u, std::integral_constant<unsigned, 1 % NS>{}, wb, wa);
        if (q + 2u < steps) step(q + 2u, std::integral_constant<unsigned, 2 % NS>{}, wa, wb);
        if (q + 3u < steps) step(q + 3u, std::integral_constant<unsigned, 3 % NS>{}, wb, wa);
        if constexpr (NS == 3) {
            if (q + 4u < steps) step(q + 4u, std::integral_constant<unsigned, 4 % NS>{}, wa, wb);
            if (q + 5u < steps) step(q + 5u, std::integral_constant<unsigned, 5 % NS>{}, wb, wa);
        }
    }
    store_tile<TM, TN>(a, acc, g.m0, g.rt0, g.split, lane);
}

// ---- 3. split reduction ------------------------------------------------

__global__ __launch_bounds__(kThreads) void prefill_reduce_kernel(const float* __restrict__ partials,
                                                                  std::uint32_t splits, std::uint32_t m,
                                                                  std::uint64_t n, const float* __restrict__ bias,
                                                                  float* __restrict__ y) {
    const std::uint64_t total = static_cast<std::uint64_t>(m) * n;
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(kThreads) + threadIdx.x; i < total;
         i += static_cast<std::uint64_t>(gridDim.x) * kThreads) {
        float v = 0.0f;
        for (std::uint32_t s = 0; s < splits; ++s) v += partials[s * total + i];
        if (bias) v += bias[i % n];
        y[i] = v;
    }
}

// The same sum four columns at a time (n % 4 == 0, 16-byte aligned rows),
// in 32-bit index arithmetic: total4 = m * n / 4 < 2^32.
__global__ __launch_bounds__(kThreads) void split_reduce4_kernel(const float4v* __restrict__ partials,
                                                                 std::uint32_t splits, std::uint32_t total4,
                                                                 std::uint32_t n4, const float4v* __restrict__ bias,
                                                                 float4v* __restrict__ y) {
    for (std::uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < total4; i += gridDim.x * kThreads) {
        float4v v = {0.0f, 0.0f, 0.0f, 0.0f};
        for (std::uint32_t s = 0; s < splits; ++s) v += partials[static_cast<std::uint64_t>(s) * total4 + i];
        if (bias) v += bias[i % n4];
        y[i] = v;
    }
}

// Partials [splits][m][ncols] of columns col0 .. col0 + ncols - 1 summed in
// split order into y [m][ldy] (+ bias): the remainder launch's K split.
// Four columns at a time (ncols, col0 and ldy multiples of 4).
__global__ __launch_bounds__(kThreads) void split_reduce_cols4_kernel(const float4v* __restrict__ partials,
                                                                      std::uint32_t splits, std::uint32_t m,
                                                                      std::uint32_t ncols4, std::uint64_t ldy4,
                                                                      std::uint64_t col0_4,
                                                                      const float4v* __restrict__ bias,
                                                                      float4v* __restrict__ y) {
    const std::uint32_t total4 = m * ncols4;
    for (std::uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < total4; i += gridDim.x * kThreads) {
        const std::uint32_t row = i / ncols4, c = i - row * ncols4;
        float4v v = {0.0f, 0.0f, 0.0f, 0.0f};
        for (std::uint32_t s = 0; s < splits; ++s) v += partials[static_cast<std::uint64_t>(s) * total4 + i];
        if (bias) v += bias[col0_4 + c];
        y[static_cast<std::uint64_t>(row) * ldy4 + col0_4 + c] = v;
    }
}

// The same sum one column at a time (any alignment, 64-bit indices).
__global__ __launch_bounds__(kThreads) void split_reduce_cols_kernel(const float* __restrict__ partials,
                                                                     std::uint32_t splits, std::uint32_t m,
                                                                     std::uint64_t ncols, std::uint64_t ldy,
                                                                     std::uint64_t col0, const float* __restrict__ bias,
                                                                     float* __restrict__ y) {
    const std::uint64_t total = static_cast<std::uint64_t>(m) * ncols;
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(kThreads) + threadIdx.x; i < total;
         i += static_cast<std::uint64_t>(gridDim.x) * kThreads) {
        const std::uint64_t row = i / ncols, c = i - row * ncols;
        float v = 0.0f;
        for (std::uint32_t s = 0; s < splits; ++s) v += partials[s * total + i];
        if (bias) v += bias[col0 + c];
        y[row * ldy + col0 + c] = v;
    }
}

// ---- weight exponent ---------------------------------------------------

// Largest |dequantized weight| bound over all blocks, as float bits (>= 0).
__global__ __launch_bounds__(kThreads) void prefill_bound_kernel(int type, const void* scales, std::uint64_t entries,
                                                                 std::uint32_t* bound_bits) {
    float local = 0.0f;
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(kThreads) + threadIdx.x; i < entries;
         i += static_cast<std::uint64_t>(gridDim.x) * kThreads) {
        float b;
        if (type == kQ4_K) {
            const uint4 h = static_cast<const uint4*>(scales)[i];
            const float d = fabsf(f16_bits_to_f32(h.x & 0xffffu));
            const float dmin = fabsf(f16_bits_to_f32(h.x >> 16));
            b = fmaxf(d * 945.0f, dmin * 63.0f);  // (d*63)*15 and dmin*63
        } else {
            const float d = fabsf(f16_bits_to_f32(static_cast<const std::uint16_t*>(scales)[i]));
            b = d * (type == kQ8_0 ? 128.0f : 8.0f);
        }
        local = (b > local || b != b) ? b : local;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(local, off);
        local = (o > local || o != o) ? o : local;
    }
    if ((threadIdx.x & 63u) == 0) atomicMax(bound_bits, __float_as_uint(local) & 0x7fffffffu);
}

// Largest |weight| bound of dense storage, as float bits: BF16 the values
// themselves (`count` of them), Q6_K |d| * 32 * 128 over the d plane
// (`count` super-blocks).
__global__ __launch_bounds__(kThreads) void dense_bound_kernel(int storage, const void* w, std::uint64_t count,
                                                               std::uint32_t* bound_bits) {
    float local = 0.0f;
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(kThreads) + threadIdx.x; i < count;
         i += static_cast<std::uint64_t>(gridDim.x) * kThreads) {
        const std::uint16_t bits = static_cast<const std::uint16_t*>(w)[i];
        const float b = storage == kBF16 ? fabsf(__uint_as_float(static_cast<std::uint32_t>(bits) << 16))
                                         : fabsf(f16_bits_to_f32(bits)) * 4096.0f;
        local = (b > local || b != b) ? b : local;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(local, off);
        local = (o > local || o != o) ? o : local;
    }
    if ((threadIdx.x & 63u) == 0) atomicMax(bound_bits, __float_as_uint(local) & 0x7fffffffu);
}

template <int TM, int TN>
hipError_t launch_lds(const GemmArgs& args, std::uint32_t stages, std::uint32_t blocks, hipStream_t stream) {
    const dim3 grid(blocks), block(kThreads);
    if (stages == 2u) hipLaunchKernelGGL((prefill_lds_kernel<kQ8_0, TM, TN, 2>), grid, block, 0, stream, args);
    else if (stages == 3u) hipLaunchKernelGGL((prefill_lds_kernel<kQ8_0, TM, TN, 3>), grid, block, 0, stream, args);
    else hipLaunchKernelGGL((prefill_lds_kernel<kQ8_0, TM, TN, 4>), grid, block, 0, stream, args);
    return hipGetLastError();
}

template <int FMT, int TM, int TN>
hipError_t launch_hyb(const GemmArgs& args, std::uint32_t stages, std::uint32_t blocks, hipStream_t stream) {
    const dim3 grid(blocks), block(kThreads);
    if (stages == 2u) hipLaunchKernelGGL((prefill_hyb_kernel<FMT, TM, TN, 2>), grid, block, 0, stream, args);
    else hipLaunchKernelGGL((prefill_hyb_kernel<FMT, TM, TN, 3>), grid, block, 0, stream, args);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_gemm_fmt(const GemmArgs& args, const PrefillShape& shape, std::uint32_t blocks, hipStream_t stream) {
    const dim3 grid(blocks), block(kThreads);
    const std::uint32_t tm = shape.tile_m, tn = shape.tile_n, pf = shape.prefetch;
    if (shape.hybrid >= 2u) {
        if (tm == 8 && tn == 4) return launch_hyb<FMT, 8, 4>(args, shape.hybrid, blocks, stream);
        if (tm == 8 && tn == 2) return launch_hyb<FMT, 8, 2>(args, shape.hybrid, blocks, stream);
        if (tm == 4 && tn == 2) return launch_hyb<FMT, 4, 2>(args, shape.hybrid, blocks, stream);
    }
    if constexpr (FMT == kQ8_0) {
        if (shape.lds_stages >= 2u) {
            return (tm == 8 && tn == 4) ? launch_lds<8, 4>(args, shape.lds_stages, blocks, stream)
                                        : launch_lds<4, 2>(args, shape.lds_stages, blocks, stream);
        }
    }
    if (tm == 8 && tn == 4) {
        if (pf == 2) hipLaunchKernelGGL((prefill_gemm_kernel<FMT, 8, 4, 2>), grid, block, 0, stream, args);
        else hipLaunchKernelGGL((prefill_gemm_kernel<FMT, 8, 4, 1>), grid, block, 0, stream, args);
    } else if (tm == 8 && tn == 2) {
        hipLaunchKernelGGL((prefill_gemm_kernel<FMT, 8, 2, 2>), grid, block, 0, stream, args);
    } else if (tm == 4 && tn == 4) {
        hipLaunchKernelGGL((prefill_gemm_kernel<FMT, 4, 4, 2>), grid, block, 0, stream, args);
    } else {
        hipLaunchKernelGGL((prefill_gemm_kernel<FMT, 4, 2, 2>), grid, block, 0, stream, args);
    }
    return hipGetLastError();
}

} // namespace

PrefillShape plan_prefill(const TilePlanes& p, std::uint32_t m, const PrefillTuning& tuning) {
    PrefillShape s;
    // Register tile per wave: TM x TN MFMA tiles (16 x 16 each).  Measured on
    // the Qwen2-7B shapes at M = 512 (TFLOP/s, Q8_0 / Q4_0 / Q4_K):
    //  * long K (down, K = 18944): 8x4, one step of prefetch, 8 K splits
    //    (623 / 649 / 571; 8x2 with 4 splits 612 / 632 / 562);
    //  * wide grids (gate|up, 2368 row tiles): Q8_0 8x4 with one step of
    //    prefetch (694; 8x2 663), the 4-bit formats 8x2 (805 / 708; 8x4
    //    703 / 550) -- their codes are half the bytes, so the shorter
    //    register tile keeps more waves resident for the same loads;
    //  * narrow grids (q|k|v, o): 4x2 with a 2-way K split (381 / 376 / 316
    //    on q|k|v; 4x4 335 / 328 / 263).
    //  * Q4_K on the hybrid kernel (activations through LDS, weights in
    //    registers; measured at M = 512: gate|up 8x4 234 -> 190 us, down
    //    126 -> 117, o 4x2 45 -> 42, q|k|v 54 -> 52), the 8x4 tile for wide
    //    grids too.  Q8_0 and Q4_0 measured even on it (within 3 %).
    const bool long_k = p.k >= 8192u;
    const bool wide = p.nt >= 1024u;
    const bool hyb_auto = p.type == kQ4_K;
    if (long_k || (wide && (p.type == kQ8_0 || hyb_auto))) {
        s.tile_m = 8u;
        s.tile_n = 4u;
        s.prefetch = 1u;
    } else if (wide) {
        s.tile_m = 8u;
        s.tile_n = 2u;
        s.prefetch = 2u;
    } else {
        s.tile_m = 4u;
        s.tile_n = 2u;
        s.prefetch = 2u;
    }
    if (tuning.tile_m == 4 || tuning.tile_m == 8) s.tile_m = tuning.tile_m;
    if (tuning.tile_n == 2 || tuning.tile_n == 4) s.tile_n = tuning.tile_n;
    if (tuning.prefetch == 1 || tuning.prefetch == 2) s.prefetch = tuning.prefetch;
    if (s.tile_m != 8 || s.tile_n != 4) s.prefetch = 2;
    const std::uint32_t bm = 16u * s.tile_m;
    s.m_tiles = static_cast<std::uint32_t>(ceil_div(m, bm));
    s.groups = static_cast<std::uint32_t>(ceil_div(p.nt, 4u * s.tile_n));
    s.steps = static_cast<std::uint32_t>(p.kp / kStepK);
    std::uint32_t splits = tuning.k_splits;
    if (splits == 0u) {
        // Split K while the doubled grid stays within 2.5 workgroups per CU,
        // keeping at least 16 steps per split: q|k|v (288 tiles) and o (224)
        // split 2 ways, down (56) 8 ways (measured: q|k|v 4 ways 4 % and o
        // 4 ways 1 % off their best; down 16 ways 16 % slower).
        const std::uint64_t tiles = static_cast<std::uint64_t>(s.m_tiles) * s.groups;
        splits = 1u;
        while (tiles * splits * 2u <= 640u && s.steps / (splits * 2u) >= 16u) splits *= 2u;
    }
    // A grid of 8x4 tiles (two workgroups per CU) that ends in a round less
    // than half full -- Qwen2-7B gate|up at M = 512: 592 workgroups on 512
    // slots, the last 80 costing as long as the first 512 -- keeps whole
    // rounds on the 8x4 tile and runs the remaining rows as a second launch
    // on the 4x2 tile (measured: 205 -> 166 us).
    if (s.tile_m == 8u && s.tile_n == 4u && splits == 1u) {
        const std::uint64_t slots = 2ull * (tuning.cus ? tuning.cus : 256u);
        const std::uint64_t grid = static_cast<std::uint64_t>(s.m_tiles) * s.groups;
        if (grid > slots && grid % slots != 0u && (grid % slots) * 2u < slots && slots % s.m_tiles == 0u) {
            const std::uint32_t main_groups = static_cast<std::uint32_t>(grid / slots * slots / s.m_tiles);
            const std::uint64_t rest_tiles = p.nt - static_cast<std::uint64_t>(main_groups) * 4u * s.tile_n;
            s.groups = main_groups;
            s.rem_groups = static_cast<std::uint32_t>(ceil_div(rest_tiles, 8u));
            s.rem_m_tiles = static_cast<std::uint32_t>(ceil_div(m, 64u));
            // The 4x2 remainder splits K until its grid reaches about two
            // workgroups per CU, at least 8 steps per split, the partials'
            // columns whole float4 runs.  Measured on gate|up at M = 512
            // (320 workgroups unsplit; warmed, same process): Q8_0 170.8 us
            // unsplit, 164.8 at 2 splits, 166.6 at 3, 173.5 at 4; Q4_K
            // 192.8 / 183.8 / 186.5 / 193.0.
            const std::uint64_t rem_blocks = static_cast<std::uint64_t>(s.rem_groups) * s.rem_m_tiles;
            const std::uint64_t rem_cols = p.n - static_cast<std::uint64_t>(main_groups) * 4u * s.tile_n * 16u;
            std::uint64_t rs = ceil_div(2ull * (tuning.cus ? tuning.cus : 256u), rem_blocks);
            rs = std::min<std::uint64_t>(rs, s.steps / 8u);
            if (tuning.rem_splits) rs = std::min<std::uint64_t>(tuning.rem_splits, s.steps);
            if (rs > 1u && rem_cols % 4u == 0u) {
                s.rem_steps_per_split = static_cast<std::uint32_t>(ceil_div(s.steps, rs));
                s.rem_splits = static_cast<std::uint32_t>(ceil_div(s.steps, s.rem_steps_per_split));
            }
        }
    }
    // The LDS pipeline runs the Q8_0 8x4 and 4x2 tiles only.  Automatic: two
    // stages for the 8x4 tile (measured at M = 512: gate|up 716 vs 700
    // TFLOP/s, down 690 vs 637; the 4x2 remainder 48 vs 55 us); the 4x2 tile
    // on its own takes registers above 256 row tiles (q|k|v, 288: 41.4 us
    // against 43.5 on LDS) and the LDS pipeline up to them (o, 224: 34.1
    // against 35.9).
    const bool lds_tile = (s.tile_m == 8u && s.tile_n == 4u) || (s.tile_m == 4u && s.tile_n == 2u);
    const bool hyb_tile = lds_tile || (s.tile_m == 8u && s.tile_n == 2u);
    if ((tuning.lds_stages == 0x12u || tuning.lds_stages == 0x13u) && hyb_tile) {
        s.hybrid = tuning.lds_stages - 0x10u;
    } else if (tuning.lds_stages == 0u && hyb_auto && hyb_tile) {
        s.hybrid = 2u;
    } else if (p.type == kQ8_0 && lds_tile) {
        if (tuning.lds_stages >= 2u && tuning.lds_stages <= 4u) {
            s.lds_stages = tuning.lds_stages;
        } else if (tuning.lds_stages == 0u && (s.tile_m == 8u || p.nt <= 256u)) {
            s.lds_stages = 2u;
        }
    }
    splits = splits < 1u ? 1u : (splits > s.steps ? s.steps : splits);
    s.steps_per_split = static_cast<std::uint32_t>(ceil_div(s.steps, splits));
    s.splits = static_cast<std::uint32_t>(ceil_div(s.steps, s.steps_per_split));
    return s;
}

std::uint64_t prefill_ldx(std::uint64_t k) { return ceil_div(k, 256u) * 256u; }
std::uint32_t prefill_rows_padded(std::uint32_t m) { return static_cast<std::uint32_t>(ceil_div(m, 256u) * 256u); }

std::uint64_t prefill_workspace_bytes(std::uint64_t k, std::uint32_t m, const PrefillShape& shape, std::uint64_t n) {
    const std::uint64_t mp = prefill_rows_padded(m);
    std::uint64_t bytes = ceil_div(mp * prefill_ldx(k) * 2u, 256u) * 256u + ceil_div(mp * 4u, 256u) * 256u;
    if (shape.splits > 1u) bytes += static_cast<std::uint64_t>(shape.splits) * m * n * 4u;
    if (shape.rem_groups && shape.rem_splits > 1u) {
        const std::uint64_t col0 = static_cast<std::uint64_t>(shape.groups) * 4u * shape.tile_n * 16u;
        bytes += static_cast<std::uint64_t>(shape.rem_splits) * m * (n - col0) * 4u;
    }
    return bytes;
}

hipError_t launch_prefill_linear(const TilePlanes& p, const float* x, const float* bias, float* y, std::uint32_t m,
                                 const PrefillShape& shape, void* workspace, hipStream_t stream, bool converted,
                                 const SplitEpilogue* epilogue) {
    const std::uint64_t mp = prefill_rows_padded(m);
    const std::uint64_t ldx = prefill_ldx(p.k);
    auto* base = static_cast<std::uint8_t*>(workspace);
    auto* xh = reinterpret_cast<_Float16*>(base);
    base += ceil_div(mp * ldx * 2u, 256u) * 256u;
    auto* row_inv = reinterpret_cast<float*>(base);
    base += ceil_div(mp * 4u, 256u) * 256u;
    auto* partials = reinterpret_cast<float*>(base);

    // `converted`: the operand of these rows is already in the workspace.
    hipError_t err = converted ? hipSuccess : launch_prefill_activations(x, m, p.k, ldx, mp, xh, row_inv, stream);
    if (err != hipSuccess) return err;

    GemmArgs a{};
    a.codes = p.codes;
    a.scales = p.scales;
    a.nt = p.nt;
    a.kt = p.kt;
    a.n = p.n;
    a.xh = xh;
    a.ldx = ldx;
    a.row_inv = row_inv;
    a.w_scale = p.prefill_scale;
    a.w_unscale = p.prefill_unscale;
    a.m = m;
    a.m_tiles = shape.m_tiles;
    a.groups = shape.groups;
    a.steps = shape.steps;
    a.steps_per_split = shape.steps_per_split;
    const bool split = shape.splits > 1u;
    a.partial = split ? 1u : 0u;
    a.bias = split ? nullptr : bias;
    a.out = split ? partials : y;
    a.ldo = p.n;
    a.col0 = 0u;
    a.blocks = shape.m_tiles * shape.groups * shape.splits;
    a.rt_base = 0u;
    const auto launch = [&](const GemmArgs& args, const PrefillShape& sh) {
        const std::uint32_t blocks = (args.blocks + 7u) / 8u * 8u;  // whole rounds of the eight XCDs
        switch (p.type) {
        case kQ8_0: return launch_gemm_fmt<kQ8_0>(args, sh, blocks, stream);
        case kQ4_0: return launch_gemm_fmt<kQ4_0>(args, sh, blocks, stream);
        case kQ4_K: return launch_gemm_fmt<kQ4_K>(args, sh, blocks, stream);
        case kF16: return launch_gemm_fmt<kF16>(args, sh, blocks, stream);
        case kBF16: return launch_gemm_fmt<kBF16>(args, sh, blocks, stream);
        case kQ6_K: return launch_gemm_fmt<kQ6_K>(args, sh, blocks, stream);
        default: return hipErrorInvalidValue;
        }
    };
    err = launch(a, shape);
    if (err == hipSuccess && shape.rem_groups) {
        // The rows past the 8x4 launch's whole rounds, on the 4x2 tile.
        PrefillShape rem = shape;
        rem.tile_m = 4u;
        rem.tile_n = 2u;
        rem.prefetch = 2u;
        rem.m_tiles = shape.rem_m_tiles;
        rem.groups = shape.rem_groups;
        GemmArgs r = a;
        r.rt_base = shape.groups * 4u * shape.tile_n;
        r.m_tiles = rem.m_tiles;
        r.groups = rem.groups;
        const bool rem_split = shape.rem_splits > 1u;
        const std::uint64_t col0 = static_cast<std::uint64_t>(r.rt_base) * 16u;
        if (rem_split) {
            r.steps_per_split = shape.rem_steps_per_split;
            r.partial = 1u;
            r.bias = nullptr;
            r.out = partials;
            r.ldo = p.n - col0;
            r.col0 = col0;
        }
        r.blocks = rem.m_tiles * rem.groups * shape.rem_splits;
        err = launch(r, rem);
        if (err == hipSuccess && rem_split) {
            const std::uint64_t ncols = p.n - col0;
            const std::uint64_t total4 = static_cast<std::uint64_t>(m) * ncols / 4u;
            const auto aligned = [](const void* q) { return reinterpret_cast<std::uintptr_t>(q) % 16u == 0u; };
            if (ncols % 4u == 0u && p.n % 4u == 0u && total4 < (1ull << 32) && aligned(partials) && aligned(y) &&
                (!bias || aligned(bias))) {
                const std::uint64_t grid = ceil_div(total4, kThreads);
                hipLaunchKernelGGL(split_reduce_cols4_kernel, dim3(static_cast<unsigned>(grid < 1024u ? grid : 1024u)),
                                   dim3(kThreads), 0, stream, reinterpret_cast<const float4v*>(partials),
                                   shape.rem_splits, m, static_cast<std::uint32_t>(ncols / 4u), p.n / 4u, col0 / 4u,
                                   reinterpret_cast<const float4v*>(bias), reinterpret_cast<float4v*>(y));
            } else {
                const std::uint64_t grid = ceil_div(static_cast<std::uint64_t>(m) * ncols, kThreads);
                hipLaunchKernelGGL(split_reduce_cols_kernel, dim3(static_cast<unsigned>(grid < 4096u ? grid : 4096u)),
                                   dim3(kThreads), 0, stream, partials, shape.rem_splits, m, ncols, p.n, col0, bias, y);
            }
            err = hipGetLastError();
        }
    }
    if (err != hipSuccess || !split) return err;
    if (epilogue) return launch_split_epilogue(partials, shape.splits, m, p.n, bias, *epilogue, stream);
    return launch_split_reduce(partials, shape.splits, m, p.n, bias, y, stream);
}

std::uint64_t prefill_partials_offset(std::uint64_t k, std::uint32_t m) {
    const std::uint64_t mp = prefill_rows_padded(m);
    return ceil_div(mp * prefill_ldx(k) * 2u, 256u) * 256u + ceil_div(mp * 4u, 256u) * 256u;
}

hipError_t launch_split_reduce(const float* partials, std::uint32_t splits, std::uint32_t m, std::uint64_t n,
                               const float* bias, float* y, hipStream_t stream) {
    const std::uint64_t total = static_cast<std::uint64_t>(m) * n;
    const auto aligned = [](const void* p) { return reinterpret_cast<std::uintptr_t>(p) % 16u == 0u; };
    if (n % 4u == 0u && total / 4u < (1ull << 32) && aligned(partials) && aligned(y) && (!bias || aligned(bias))) {
        const std::uint64_t total4 = total / 4u;
        const std::uint64_t grid = ceil_div(total4, kThreads);
        hipLaunchKernelGGL(split_reduce4_kernel, dim3(static_cast<unsigned>(grid < 1024u ? grid : 1024u)),
                           dim3(kThreads), 0, stream, reinterpret_cast<const float4v*>(partials), splits,
                           static_cast<std::uint32_t>(total4), static_cast<std::uint32_t>(n / 4u),
                           reinterpret_cast<const float4v*>(bias), reinterpret_cast<float4v*>(y));
        return hipGetLastError();
    }
    const std::uint64_t grid = ceil_div(total, kThreads);
    hipLaunchKernelGGL(prefill_reduce_kernel, dim3(static_cast<unsigned>(grid < 8192u ? grid : 8192u)), dim3(kThreads),
                       0, stream, partials, splits, m, n, bias, y);
    return hipGetLastError();
}

namespace {
// e = smallest integer with bound * 2^-e <= 2^15 (scale 1 for a zero or
// non-finite bound).
void set_prefill_exponent(TilePlanes& p, float bound) {
    p.prefill_scale = 1.0f;
    p.prefill_unscale = 1.0f;
    if (bound > 0.0f && bound < 3.0e38f) {
        int e = 0;
        (void)std::frexp(bound, &e);          // bound = f * 2^e, f in [0.5, 1)
        e -= 15;                              // bound * 2^-e < 2^15
        e = e < -100 ? -100 : (e > 100 ? 100 : e);
        p.prefill_scale = std::ldexp(1.0f, -e);
        p.prefill_unscale = std::ldexp(1.0f, e);
    }
}
} // namespace

hipError_t compute_dense_prefill_scale(TilePlanes& p, std::uint32_t* bound_scratch, hipStream_t stream) {
    p.prefill_scale = 1.0f;
    p.prefill_unscale = 1.0f;
    if (p.type == kF16) return hipSuccess;   // the rows are the f16 operands themselves
    const std::uint64_t count = p.type == kBF16 ? p.k * p.n : p.k * p.n / 256u;
    const void* src = p.type == kBF16 ? p.codes
                                      : static_cast<const void*>(static_cast<const unsigned char*>(p.codes) + count * 208u);
    hipError_t err = hipMemsetAsync(bound_scratch, 0, sizeof(std::uint32_t), stream);
    if (err != hipSuccess) return err;
    const std::uint64_t grid = ceil_div(count, kThreads);
    hipLaunchKernelGGL(dense_bound_kernel, dim3(static_cast<unsigned>(grid < 4096u ? grid : 4096u)), dim3(kThreads), 0,
                       stream, p.type, src, count, bound_scratch);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    std::uint32_t bits = 0;
    err = hipMemcpyAsync(&bits, bound_scratch, sizeof(bits), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) return err;
    float bound;
    std::memcpy(&bound, &bits, sizeof(bound));
    set_prefill_exponent(p, bound);
    return hipSuccess;
}

hipError_t compute_prefill_scale(TilePlanes& p, std::uint32_t* bound_scratch, hipStream_t stream) {
    const auto geo = geometry_of(p.type);
    const std::uint64_t tiles = static_cast<std::uint64_t>(p.nt) * p.kt;
    // Scale entries: f16 per block (Q8_0, Q4_0), one 16-byte header per super-block (Q4_K).
    const std::uint64_t entries = p.type == kQ4_K ? tiles * 16u : tiles * (geo.scale_tile_bytes / 2u);
    hipError_t err = hipMemsetAsync(bound_scratch, 0, sizeof(std::uint32_t), stream);
    if (err != hipSuccess) return err;
    const std::uint64_t grid = ceil_div(entries, kThreads);
    hipLaunchKernelGGL(prefill_bound_kernel, dim3(static_cast<unsigned>(grid < 4096u ? grid : 4096u)), dim3(kThreads),
                       0, stream, p.type, p.scales, entries, bound_scratch);
    err = hipGetLastError();
    if (err != hipSuccess) return err;
    std::uint32_t bits = 0;
    err = hipMemcpyAsync(&bits, bound_scratch, sizeof(bits), hipMemcpyDeviceToHost, stream);
    if (err == hipSuccess) err = hipStreamSynchronize(stream);
    if (err != hipSuccess) return err;
    float bound;
    std::memcpy(&bound, &bits, sizeof(bound));
    set_prefill_exponent(p, bound);
    return hipSuccess;
}

} // namespace air_hip

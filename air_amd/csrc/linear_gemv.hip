// linear_gemv.hip -- the M = 1 decode linear (matrix-vector product).
//
// Replaces specialized_matvec_kernel (src/cuda/cuda_backend.cu:585-606) for
// single-sequence decode.  Same arithmetic contract as the other decode
// kernels: exact integer codes as the f16 B operand of
// v_mfma_f32_16x16x32_f16, the activation split into f16 hi + lo with a
// power-of-two scale per 32-element block, f32 block-scale epilogue.
//
// "Block-diagonal" A operand.  With one activation row, a 16x32 A operand
// would carry 15 rows of zeros.  Instead A row r holds the activation block
// b0 + r, so one split serves a whole chunk of 16 consecutive blocks; the
// MFMA of weight block b0 + r then has its useful output in D row r (lane
// group r/4, element r%4), and only that slot accumulates.  Per lane, the
// activation costs 8 floats per 16 blocks, which leaves the registers for
// prefetching: every wave issues the loads of a whole chunk (8 KiB of Q8_0
// codes per row tile) before computing the previous one.
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"

namespace air_hip {
namespace {

constexpr std::uint32_t kChunkBlocks = 16;

__device__ __forceinline__ float half_bits_to_float(std::uint32_t bits16) {
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(bits16)));
}

__device__ __forceinline__ float lane_value(float v, int src) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), src));
}

template <int FMT> struct GemvFormat;
template <> struct GemvFormat<kQ8_0> {
    static constexpr int kBlocksPerTile = 2;
    static constexpr int kCodeVecs = 1;        // uint4 per lane per tile
    using Scale = std::uint32_t;
};
template <> struct GemvFormat<kQ4_0> {
    static constexpr int kBlocksPerTile = 4;
    static constexpr int kCodeVecs = 1;
    using Scale = uint2;
};
template <> struct GemvFormat<kQ4_K> {
    static constexpr int kBlocksPerTile = 8;
    static constexpr int kCodeVecs = 2;
    using Scale = uint4;
};

// One chunk (16 blocks) of R row tiles plus the lane's activations.
template <int FMT, int R>
struct Chunk {
    static constexpr int kTiles = kChunkBlocks / GemvFormat<FMT>::kBlocksPerTile;
    uint4 c[kTiles][R][GemvFormat<FMT>::kCodeVecs];
    typename GemvFormat<FMT>::Scale sc[kTiles][R];
    float4 x[2];
};

template <int FMT, int R>
__device__ __forceinline__ void load_chunk(Chunk<FMT, R>& ch, const void* __restrict__ codes_,
                                           const void* __restrict__ scales_, std::uint32_t rt0, std::uint32_t NT,
                                           std::uint32_t KT, std::uint32_t chunk, std::uint32_t lane,
                                           const float* __restrict__ x, std::uint64_t nblocks) {
    using F = GemvFormat<FMT>;
    using Scale = typename F::Scale;
    constexpr int T = Chunk<FMT, R>::kTiles;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        // Tile (rt0 + r, chunk * T) as a wave-uniform base; lanes add their
        // own 16-byte (codes) or scale-record offset.
        const std::uint64_t tile0 = static_cast<std::uint64_t>(rt0 + r) * KT + static_cast<std::uint64_t>(chunk) * T;
        const u32x4* cbase = static_cast<const u32x4*>(codes_) + tile0 * F::kCodeVecs * 64u;
        const Scale* sbase = static_cast<const Scale*>(scales_) + tile0 * 16u;
        const bool row_live = (rt0 + r) < NT;
#pragma unroll
        for (int j = 0; j < T; ++j) {
            const bool live = row_live && chunk * T + j < KT;
#pragma unroll
            for (int v = 0; v < F::kCodeVecs; ++v) {
                // Weight codes are read once per pass: non-temporal loads keep
                // them from displacing the activations and scales in the caches.
                u32x4 word = {0u, 0u, 0u, 0u};
                if (live) word = __builtin_nontemporal_load(cbase + (j * F::kCodeVecs + v) * 64u + lane);
                ch.c[j][r][v] = make_uint4(word.x, word.y, word.z, word.w);
            }
            ch.sc[j][r] = live ? sbase[j * 16u + (lane & 15u)] : Scale{};
        }
    }
    // A row r = lane % 16 holds block chunk*16 + r, elements 8*(lane/16)..+7.
    const std::uint64_t kb = static_cast<std::uint64_t>(chunk) * kChunkBlocks + (lane & 15u);
    if (kb < nblocks) {
        const float4* src = reinterpret_cast<const float4*>(x + kb * 32u + 8u * (lane >> 4));
        ch.x[0] = src[0];
        ch.x[1] = src[1];
    } else {
        ch.x[0] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        ch.x[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
}

// Weight block j of a tile as the f16 B operand (exact integers).
template <int FMT, int R>
__device__ __forceinline__ half8v tile_block_codes(const Chunk<FMT, R>& ch, int t, int r, int j) {
    if constexpr (FMT == kQ8_0) {
        const uint4 c = ch.c[t][r][0];
        half2v p0, p1, p2, p3;
        q8_dword_to_half(j == 0 ? c.x : c.z, p0, p1);
        q8_dword_to_half(j == 0 ? c.y : c.w, p2, p3);
        half8v out;
        out[0] = p0[0]; out[1] = p0[1]; out[2] = p1[0]; out[3] = p1[1];
        out[4] = p2[0]; out[5] = p2[1]; out[6] = p3[0]; out[7] = p3[1];
        return out;
    } else if constexpr (FMT == kQ4_0) {
        const uint4 c = ch.c[t][r][0];
        return nibble_dword_to_half8<8>(j == 0 ? c.x : j == 1 ? c.y : j == 2 ? c.z : c.w);
    } else {
        const uint4 c = ch.c[t][r][j >> 2];
        const int q = j & 3;
        return nibble_dword_to_half8<0>(q == 0 ? c.x : q == 1 ? c.y : q == 2 ? c.z : c.w);
    }
}

template <int FMT, int R>
__device__ __forceinline__ void compute_chunk(const Chunk<FMT, R>& ch, std::uint32_t lane, float4v (&acc)[R]) {
    using F = GemvFormat<FMT>;
    constexpr int T = Chunk<FMT, R>::kTiles;
    const float v[8] = {ch.x[0].x, ch.x[0].y, ch.x[0].z, ch.x[0].w, ch.x[1].x, ch.x[1].y, ch.x[1].z, ch.x[1].w};
    float amax = fmaxf(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))),
                       fmaxf(fmaxf(fabsf(v[4]), fabsf(v[5])), fmaxf(fabsf(v[6]), fabsf(v[7]))));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    float s, inv;
    block_scale(amax, s, inv);
    half8v hi, lo;
    split8(v, s, hi, lo);
    float xsum = 0.0f;
    if constexpr (FMT == kQ4_K) {
        xsum = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
        xsum += __shfl_xor(xsum, 16);
        xsum += __shfl_xor(xsum, 32);
    }
    const std::uint32_t group = lane >> 4;

#pragma unroll
    for (int t = 0; t < T; ++t) {
        // Q4_K: the tile is one super-block; its 8 sub-block scales per row.
        float q4k_d[R], q4k_m[R];
        std::uint32_t q4k_packed[R][3];
        if constexpr (FMT == kQ4_K) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                q4k_d[r] = half_bits_to_float(ch.sc[t][r].x & 0xffffu);
                q4k_m[r] = half_bits_to_float(ch.sc[t][r].x >> 16);
                q4k_packed[r][0] = ch.sc[t][r].y;
                q4k_packed[r][1] = ch.sc[t][r].z;
                q4k_packed[r][2] = ch.sc[t][r].w;
            }
        }
#pragma unroll
        for (int j = 0; j < F::kBlocksPerTile; ++j) {
            const int row = t * F::kBlocksPerTile + j;   // A / D row of this block
            const int i = row & 3;
            const bool mine = group == static_cast<std::uint32_t>(row >> 2);
            const float inv_r = lane_value(inv, row);
            float sum_r = 0.0f;
            if constexpr (FMT == kQ4_K) sum_r = lane_value(xsum, row);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const half8v w = tile_block_codes<FMT, R>(ch, t, r, j);
                float4v p = mfma16x16x32(hi, w, float4v{0.0f, 0.0f, 0.0f, 0.0f});
                p = mfma16x16x32(lo, w, p);
                float updated;
                if constexpr (FMT == kQ8_0) {
                    const float d = half_bits_to_float((ch.sc[t][r] >> (16 * j)) & 0xffffu);
                    updated = fmaf(d * inv_r, p[i], acc[r][i]);
                } else if constexpr (FMT == kQ4_0) {
                    const std::uint32_t sw = j < 2 ? ch.sc[t][r].x : ch.sc[t][r].y;
                    const float d = half_bits_to_float((sw >> (16 * (j & 1))) & 0xffffu);
                    updated = fmaf(d * inv_r, p[i], acc[r][i]);
                } else {
                    std::uint32_t s6 = 0, m6 = 0;
                    q4k_scale_min(q4k_packed[r], static_cast<std::uint32_t>(j), s6, m6);
                    const float dj = q4k_d[r] * static_cast<float>(s6);
                    const float mj = q4k_m[r] * static_cast<float>(m6);
                    updated = fmaf(-mj, sum_r, fmaf(dj * inv_r, p[i], acc[r][i]));
                }
                acc[r][i] = mine ? updated : acc[r][i];
            }
        }
    }
}

constexpr int gemv_max_waves(int FMT, int R) { return FMT >= 0 && R >= 4 ? 4 : 8; }

// Workgroup = W waves on the same R row tiles; the chunks of K are split
// across the waves.  P = 2: each wave double-buffers whole chunks.  P = 1:
// one chunk buffer, loaded and consumed in turn -- the lower register count
// lets twice as many waves share a CU, which hides the load latency by
// occupancy instead.
template <int FMT, int R, int P>
__global__ void __launch_bounds__(64 * gemv_max_waves(FMT, R))
decode_gemv_kernel(const void* __restrict__ codes_, const void* __restrict__ scales_,
                   const float* __restrict__ x, const float* __restrict__ bias, float* __restrict__ y,
                   std::uint64_t K, std::uint64_t N, std::uint32_t NT, std::uint32_t KT) {
    extern __shared__ float wave_sums[];
    using Ch = Chunk<FMT, R>;
    const std::uint32_t lane = threadIdx.x & 63u;
    // Wave-uniform: chunk indices, tile addresses and liveness stay scalar.
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const std::uint32_t W = blockDim.x >> 6;
    const std::uint32_t rt0 = blockIdx.x * R;
    const std::uint64_t nblocks = K / 32u;
    const std::uint32_t chunks = static_cast<std::uint32_t>(ceil_div(KT, static_cast<std::uint64_t>(Ch::kTiles)));
    const std::uint32_t c_begin = static_cast<std::uint32_t>((static_cast<std::uint64_t>(chunks) * wave) / W);
    const std::uint32_t c_end = static_cast<std::uint32_t>((static_cast<std::uint64_t>(chunks) * (wave + 1u)) / W);

    float4v acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    if constexpr (P == 1) {
        for (std::uint32_t c = c_begin; c < c_end; ++c) {
            Ch a;
            load_chunk<FMT, R>(a, codes_, scales_, rt0, NT, KT, c, lane, x, nblocks);
            compute_chunk<FMT, R>(a, lane, acc);
        }
    } else {
        Ch a, b;
        if (c_begin < c_end) load_chunk<FMT, R>(a, codes_, scales_, rt0, NT, KT, c_begin, lane, x, nblocks);
        for (std::uint32_t c = c_begin; c < c_end; c += 2u) {
            if (c + 1u < c_end) load_chunk<FMT, R>(b, codes_, scales_, rt0, NT, KT, c + 1u, lane, x, nblocks);
            compute_chunk<FMT, R>(a, lane, acc);
            if (c + 1u >= c_end) break;
            if (c + 2u < c_end) load_chunk<FMT, R>(a, codes_, scales_, rt0, NT, KT, c + 2u, lane, x, nblocks);
            compute_chunk<FMT, R>(b, lane, acc);
        }
    }

    // Row n = 16*tile + lane%16: add the four D slots and the four lane groups.
    float total[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float t = (acc[r][0] + acc[r][1]) + (acc[r][2] + acc[r][3]);
        t += __shfl_xor(t, 16);
        t += __shfl_xor(t, 32);
        total[r] = t;
    }
    if (W > 1u) {
        if (wave > 0u && lane < 16u) {
#pragma unroll
            for (int r = 0; r < R; ++r) wave_sums[((wave - 1u) * R + r) * 16u + lane] = total[r];
        }
        __syncthreads();
        if (wave == 0u && lane < 16u) {
            for (std::uint32_t w = 1; w < W; ++w) {
#pragma unroll
                for (int r = 0; r < R; ++r) total[r] += wave_sums[((w - 1u) * R + r) * 16u + lane];
            }
        }
    }
    if (wave != 0u || lane >= 16u) return;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const std::uint64_t n = static_cast<std::uint64_t>(rt0 + r) * 16u + lane;
        if ((rt0 + r) < NT && n < N) y[n] = total[r] + (bias ? bias[n] : 0.0f);
    }
}

template <int FMT, int R, int P>
hipError_t launch_gemv_variant(const TilePlanes& p, const float* x, const float* bias, float* y,
                               std::uint32_t W, hipStream_t stream) {
    if (W == 0u || W > static_cast<std::uint32_t>(gemv_max_waves(FMT, R))) return hipErrorInvalidConfiguration;
    const dim3 grid(static_cast<unsigned>(ceil_div(p.nt, R)), 1, 1);
    const std::size_t lds = static_cast<std::size_t>(W - 1u) * R * 16u * sizeof(float);
    decode_gemv_kernel<FMT, R, P><<<grid, 64u * W, lds, stream>>>(p.codes, p.scales, x, bias, y, p.k, p.n, p.nt,
                                                                   p.kt);
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_gemv_fmt(const TilePlanes& p, const float* x, const float* bias, float* y, std::uint32_t R,
                           std::uint32_t W, std::uint32_t P, hipStream_t s) {
    if (R == 1u) {
        return P == 1u ? launch_gemv_variant<FMT, 1, 1>(p, x, bias, y, W, s)
                       : launch_gemv_variant<FMT, 1, 2>(p, x, bias, y, W, s);
    }
    if (R == 2u) {
        return P == 1u ? launch_gemv_variant<FMT, 2, 1>(p, x, bias, y, W, s)
                       : launch_gemv_variant<FMT, 2, 2>(p, x, bias, y, W, s);
    }
    return P == 1u ? launch_gemv_variant<FMT, 4, 1>(p, x, bias, y, W, s)
                   : launch_gemv_variant<FMT, 4, 2>(p, x, bias, y, W, s);
}

} // namespace

GemvShape plan_decode_gemv(const TilePlanes& p, const DecodeTuning& tuning) {
    GemvShape g{};
    const std::uint32_t tiles_per_chunk = kChunkBlocks / (geometry_of(p.type).tile_k / 32u);
    const std::uint32_t chunks = static_cast<std::uint32_t>(ceil_div(p.kt, tiles_per_chunk));
    // One row tile per wave (measured best for every Qwen2 shape).  Few row
    // groups (< 2048, e.g. q|k|v, o, down): split the chunks of K over the
    // waves of a workgroup until the grid holds about 8192 waves, each wave
    // double-buffering its chunks.  Many row groups (gate|up, lm_head): four
    // single-buffered waves per workgroup -- the register count halves and
    // twice as many waves per CU keep the loads in flight (measured 2-5 %
    // faster than double buffering on those shapes).
    g.rows_per_wave = 1u;
    if (tuning.rows_per_wave == 1u || tuning.rows_per_wave == 2u || tuning.rows_per_wave == 4u) {
        g.rows_per_wave = tuning.rows_per_wave;
    }
    const std::uint32_t cap = static_cast<std::uint32_t>(g.rows_per_wave >= 4u ? 4 : 8);
    const std::uint64_t groups = ceil_div(p.nt, g.rows_per_wave);
    const bool wide = groups >= 2048u;
    std::uint64_t w = wide ? 4u : ceil_div(8192u, groups);
    if (w > cap) w = cap;
    if (w > chunks) w = chunks;
    g.waves_per_group = w == 0u ? 1u : static_cast<std::uint32_t>(w);
    if (tuning.waves_per_group != 0u) g.waves_per_group = tuning.waves_per_group < cap ? tuning.waves_per_group : cap;
    // Chunks in flight per wave: one for wide grids and when no wave owns
    // more than one chunk, else two.
    g.depth = (wide || ceil_div(chunks, g.waves_per_group) <= 1u) ? 1u : 2u;
    return g;
}

hipError_t launch_decode_gemv(const TilePlanes& p, const float* x, const float* bias, float* y,
                              const GemvShape& g, hipStream_t stream) {
    switch (p.type) {
    case kQ8_0: return launch_gemv_fmt<kQ8_0>(p, x, bias, y, g.rows_per_wave, g.waves_per_group, g.depth, stream);
    case kQ4_0: return launch_gemv_fmt<kQ4_0>(p, x, bias, y, g.rows_per_wave, g.waves_per_group, g.depth, stream);
    case kQ4_K: return launch_gemv_fmt<kQ4_K>(p, x, bias, y, g.rows_per_wave, g.waves_per_group, g.depth, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace air_hip

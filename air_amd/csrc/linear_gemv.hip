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

// Which D rows a chunk's blocks land in.  The MFMA of a tile's block has its
// useful output in one D row (= A row), and D row r lives in lane group r / 4,
// slot r % 4; the lane group owning a block applies its scale.  The rows are
// laid out so that each lane group owns whole tiles whose scale records it
// can load itself, one coalesced load per four tiles:
//   Q8_0 (8 tiles of 2 blocks): tile t, block j -> row 4 (t % 4) + 2 (t / 4)
//        + j, so group g owns tiles g and g + 4.  A unit of half a chunk (U =
//        2, tiles 4h .. 4h + 3 of the chunk, its own A operand) puts unit tile
//        t in rows 4 t + j: group g owns tile g in slots 0 and 1;
//   Q4_0 (4 tiles of 4 blocks): tile t, block j -> row 4 t + j (group t);
//   Q4_K (2 tiles of 8 blocks): tile t, block j -> row 8 t + j (groups 2t,
//        2t + 1 each own four blocks of the tile).
// A row r of unit h therefore holds chunk block block_of_row(r, h), and is
// zero unless row_of_unit(r) (Q8_0 half-chunk units use slots 0 and 1 only).
template <int FMT, int U>
__device__ __forceinline__ std::uint32_t block_of_row(std::uint32_t r, std::uint32_t h) {
    if constexpr (FMT == kQ8_0 && U == 1) return 2u * (r >> 2) + 8u * ((r & 3u) >> 1) + (r & 1u);
    if constexpr (FMT == kQ8_0) return 8u * h + 2u * (r >> 2) + (r & 1u);
    return r;
}
template <int FMT, int U>
__device__ __forceinline__ bool row_of_unit(std::uint32_t r) {
    return FMT != kQ8_0 || U == 1 || (r & 3u) < 2u;
}
// Tiles of a unit whose scale records a lane loads, and the i-th of them
// (unit-relative) for lane group g.
template <int FMT, int T>
constexpr int own_tiles() { return FMT == kQ8_0 ? T / 4 : 1; }
template <int FMT>
__device__ __forceinline__ std::uint32_t own_tile(std::uint32_t g, int i) {
    if constexpr (FMT == kQ8_0) return g + 4u * static_cast<std::uint32_t>(i);
    if constexpr (FMT == kQ4_0) return g;
    return g >> 1;
}

// One work unit of R row tiles plus the lane's activations: a chunk (16
// blocks) split into U units of 16/U blocks each (U = 2 for Q8_0 only).  The
// activation operand spans the whole chunk; a unit's tiles use the rows of
// its own blocks.  sc holds the scale records of the lane's own tiles.
// NORM: the activations are RMS-normalised in the kernel, and nw holds the
// norm weights of the lane's x.
template <int FMT, int R, int U, bool NORM>
struct Chunk {
    static constexpr int kTiles = kChunkBlocks / GemvFormat<FMT>::kBlocksPerTile / U;
    static constexpr int kOwn = own_tiles<FMT, kTiles>();
    uint4 c[kTiles][R][GemvFormat<FMT>::kCodeVecs];
    typename GemvFormat<FMT>::Scale sc[kOwn][R];
    float4 x[2];
    float4v nw[NORM ? 2 : 1];    // native vectors: struct copies would go to scratch
};

template <int FMT, int R, int U, bool NORM>
__device__ __forceinline__ void load_chunk(Chunk<FMT, R, U, NORM>& ch, const void* __restrict__ codes_,
                                           const void* __restrict__ scales_, std::uint32_t rt0, std::uint32_t NT,
                                           std::uint32_t KT, std::uint32_t unit, std::uint32_t lane,
                                           const float* __restrict__ x, const float* __restrict__ norm_w,
                                           std::uint64_t nblocks) {
    // Issue order = return order: the activations first (the split they
    // feed can start while the codes stream), then the scale records,
    // then the codes tile by tile.
    using F = GemvFormat<FMT>;
    using Scale = typename F::Scale;
    constexpr int T = Chunk<FMT, R, U, NORM>::kTiles;
    constexpr int kOwn = Chunk<FMT, R, U, NORM>::kOwn;
    const std::uint32_t chunk = unit / U;
    const std::uint32_t kt0 = unit * T;   // first k tile of the unit
    const std::uint32_t group = lane >> 4;
    if (rt0 + R <= NT && kt0 + T <= KT) {
        // Every tile live (all but the last unit of a ragged K): no fill.
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const std::uint64_t tile0 = static_cast<std::uint64_t>(rt0 + r) * KT + kt0;
            const u32x4* cbase = static_cast<const u32x4*>(codes_) + tile0 * F::kCodeVecs * 64u;
            const Scale* sbase = static_cast<const Scale*>(scales_) + tile0 * 16u;
            // The lane's own tiles' records: consecutive lanes, consecutive
            // records (Q8_0: 256 contiguous bytes per load).
#pragma unroll
            for (int i = 0; i < kOwn; ++i) ch.sc[i][r] = sbase[own_tile<FMT>(group, i) * 16u + (lane & 15u)];
#pragma unroll
            for (int j = 0; j < T; ++j) {
#pragma unroll
                for (int v = 0; v < F::kCodeVecs; ++v) {
                    const u32x4 word = __builtin_nontemporal_load(cbase + (j * F::kCodeVecs + v) * 64u + lane);
                    ch.c[j][r][v] = make_uint4(word.x, word.y, word.z, word.w);
                }
            }
        }
    } else {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        // Tile (rt0 + r, kt0) as a wave-uniform base; lanes add their own
        // 16-byte (codes) or scale-record offset.
        const std::uint64_t tile0 = static_cast<std::uint64_t>(rt0 + r) * KT + kt0;
        const u32x4* cbase = static_cast<const u32x4*>(codes_) + tile0 * F::kCodeVecs * 64u;
        const Scale* sbase = static_cast<const Scale*>(scales_) + tile0 * 16u;
        const bool row_live = (rt0 + r) < NT;
#pragma unroll
        for (int i = 0; i < kOwn; ++i) {
            const std::uint32_t t = own_tile<FMT>(group, i);
            const bool live = row_live && kt0 + t < KT;
            ch.sc[i][r] = live ? sbase[t * 16u + (lane & 15u)] : Scale{};
        }
#pragma unroll
        for (int j = 0; j < T; ++j) {
            const bool live = row_live && kt0 + j < KT;
#pragma unroll
            for (int v = 0; v < F::kCodeVecs; ++v) {
                // Weight codes are read once per pass: non-temporal loads keep
                // them from displacing the activations and scales in the caches.
                u32x4 word = {0u, 0u, 0u, 0u};
                if (live) word = __builtin_nontemporal_load(cbase + (j * F::kCodeVecs + v) * 64u + lane);
                ch.c[j][r][v] = make_uint4(word.x, word.y, word.z, word.w);
            }
        }
    }
    }
    // A row r = lane % 16 holds chunk block block_of_row(r, h), elements
    // 8*(lane/16)..+7; rows the unit does not use stay zero.
    const std::uint32_t arow = lane & 15u;
    const std::uint64_t kb = static_cast<std::uint64_t>(chunk) * kChunkBlocks + block_of_row<FMT, U>(arow, unit % U);
    const bool row_used = row_of_unit<FMT, U>(arow);
    if (kb < nblocks && row_used) {
        const float4* src = reinterpret_cast<const float4*>(x + kb * 32u + 8u * (lane >> 4));
        ch.x[0] = src[0];
        ch.x[1] = src[1];
        if constexpr (NORM) {
            const float4v* wsrc = reinterpret_cast<const float4v*>(norm_w + kb * 32u + 8u * (lane >> 4));
            ch.nw[0] = wsrc[0];
            ch.nw[1] = wsrc[1];
        }
    } else {
        ch.x[0] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        ch.x[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if constexpr (NORM) {
            ch.nw[0] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
            ch.nw[1] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
}

// Weight block j of a tile as the f16 B operand (exact integers).
template <int FMT, int R, int U, bool NORM>
__device__ __forceinline__ half8v tile_block_codes(const Chunk<FMT, R, U, NORM>& ch, int t, int r, int j) {
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

// The RMS norm's per-element step, (x * scale) * w, without contraction (the
// norm kernel's arithmetic).
__device__ __forceinline__ float norm_apply(float x, float scale, float w) {
#pragma clang fp contract(off)
    const float xs = x * scale;
    return xs * w;
}

template <int FMT, int R, int U, bool NORM>
__device__ __forceinline__ void compute_chunk(const Chunk<FMT, R, U, NORM>& ch, std::uint32_t unit,
                                              std::uint32_t lane, float norm_scale, float4v (&acc)[R]) {
    using F = GemvFormat<FMT>;
    constexpr int T = Chunk<FMT, R, U, NORM>::kTiles;
    // Q4_K's first A / D row of the unit (U = 1 for the 4-bit formats: 0).
    const std::uint32_t row0 = (unit % U) * (kChunkBlocks / U);
    float v[8] = {ch.x[0].x, ch.x[0].y, ch.x[0].z, ch.x[0].w, ch.x[1].x, ch.x[1].y, ch.x[1].z, ch.x[1].w};
    if constexpr (NORM) {
        const float w[8] = {ch.nw[0][0], ch.nw[0][1], ch.nw[0][2], ch.nw[0][3],
                            ch.nw[1][0], ch.nw[1][1], ch.nw[1][2], ch.nw[1][3]};
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = norm_apply(v[e], norm_scale, w[e]);
    }
    // One power-of-two scale for the whole unit (all 64 lanes).  The f16
    // hi + lo split keeps ~21 significant bits of every element, however far
    // below the unit's maximum it lies, so the scale only guards the range.
    float amax = fmaxf(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))),
                       fmaxf(fmaxf(fabsf(v[4]), fabsf(v[5])), fmaxf(fabsf(v[6]), fabsf(v[7]))));
    amax = wave_max(amax);
    float s, inv;
    block_scale(amax, s, inv);
    half8v hi, lo;
    split8(v, s, hi, lo);
    // Q4_K: scaled block sums for the dmin term from one MFMA pair against an
    // all-ones B: D row r = sum of block r, in every column -- the very lanes
    // and slot where block r's products land.
    float4v xs{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (FMT == kQ4_K) {
        half8v ones;
#pragma unroll
        for (int e = 0; e < 8; ++e) ones[e] = static_cast<_Float16>(1.0f);
        xs = mfma16x16x32(hi, ones, xs);
        xs = mfma16x16x32(lo, ones, xs);
    }
    const std::uint32_t group = lane >> 4;

    // Sums in the scaled domain, multiplied by inv once at the end.  Q8_0 /
    // Q4_0: the blocks of one tile own one lane group of D, so the tile's
    // scale record is masked once per tile: lanes of other groups add
    // 0 x (a finite product).
    float4v cacc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) cacc[r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (FMT == kQ4_K) {
        // A lane's four D slots hold blocks 4 * group + i - row0 of the unit
        // (i = 0..3): sub-blocks 4h + i of one tile.  Each block's MFMA result
        // is selected into the slots of the lane group that owns it, and
        // only the lane's own four (scale, min) pairs are decoded, once per
        // unit -- the same value as scaling every block with a scale masked
        // to zero outside its lane group (those terms add exact zeros).
        const int first = static_cast<int>(4u * group) - static_cast<int>(row0);
        const bool lane_owns = first >= 0 && first < static_cast<int>(kChunkBlocks / U);
        const bool upper = (first & 4) != 0;   // sub-blocks 4-7 of the tile
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float4v sel{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int t = 0; t < T; ++t) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int rel = t * 8 + j;
                    const half8v w = tile_block_codes<FMT, R, U, NORM>(ch, t, r, j);
                    float4v p = mfma16x16x32(hi, w, float4v{0.0f, 0.0f, 0.0f, 0.0f});
                    p = mfma16x16x32(lo, w, p);
                    const std::uint32_t owner = (row0 + static_cast<std::uint32_t>(rel)) >> 2;
                    sel[rel & 3] = group == owner ? p[rel & 3] : sel[rel & 3];
                }
            }
            // The record of the lane's own tile (first / 8, loaded by
            // load_chunk): f16 (d, dmin), then the 12 packed 6-bit scale / min
            // bytes (src/reference/tensor_reader.cpp:153-165).
            const uint4 rec = ch.sc[0][r];
            const std::uint32_t packed[3] = {rec.y, rec.z, rec.w};
            std::uint32_t scales = 0, mins = 0;
            q4k_scale_min_x4(packed, upper, scales, mins);
            const float d = lane_owns ? half_bits_to_float(rec.x & 0xffffu) : 0.0f;
            const float dmin = lane_owns ? half_bits_to_float(rec.x >> 16) : 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float dj = d * static_cast<float>((scales >> (8 * i)) & 0xffu);
                const float mj = dmin * static_cast<float>((mins >> (8 * i)) & 0xffu);
                cacc[r][i] = fmaf(-mj, xs[i], fmaf(dj, sel[i], cacc[r][i]));
            }
        }
    }
#pragma unroll
    for (int t = 0; t < (FMT == kQ4_K ? 0 : T); ++t) {
        // Owner lane group and the D slot of block j: Q8_0 tile t of a whole
        // chunk is owned by group t % 4 in slots 2 (t / 4) + j, tile t of a
        // half chunk by group t in slots j; Q4_0 tile t by group t in slots j.
        const std::uint32_t owner = FMT == kQ8_0 ? static_cast<std::uint32_t>(t & 3) : static_cast<std::uint32_t>(t);
        const bool own = group == owner;
        typename F::Scale sc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (FMT == kQ8_0) {
                sc[r] = own ? ch.sc[t >> 2][r] : 0u;
            } else if constexpr (FMT == kQ4_0) {
                sc[r] = own ? ch.sc[0][r] : make_uint2(0u, 0u);
            }
        }
        const int slot0 = FMT == kQ8_0 && U == 1 ? 2 * (t >> 2) : 0;
#pragma unroll
        for (int j = 0; j < F::kBlocksPerTile; ++j) {
            const int i = slot0 + j;                                // D slot of this block
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const half8v w = tile_block_codes<FMT, R, U, NORM>(ch, t, r, j);
                float4v p = mfma16x16x32(hi, w, float4v{0.0f, 0.0f, 0.0f, 0.0f});
                p = mfma16x16x32(lo, w, p);
                if constexpr (FMT == kQ8_0) {
                    const float d = half_bits_to_float((sc[r] >> (16 * j)) & 0xffffu);
                    cacc[r][i] = fmaf(d, p[i], cacc[r][i]);
                } else {
                    const std::uint32_t sw = j < 2 ? sc[r].x : sc[r].y;
                    const float d = half_bits_to_float((sw >> (16 * (j & 1))) & 0xffffu);
                    cacc[r][i] = fmaf(d, p[i], cacc[r][i]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[r][i] = fmaf(inv, cacc[r][i], acc[r][i]);
    }
}

// Waves per workgroup: single-buffered one-tile waves fit 16 per CU.
constexpr int gemv_max_waves(int R, int P) { return R >= 4 ? 4 : (R == 1 && P == 1 ? 16 : 8); }

// The SwiGLU of the step, silu(g) * u with silu(g) = g / (1 + e^-g), without
// contraction (the separate silu_mul kernel's arithmetic).
__device__ __forceinline__ float swiglu(float g, float u) {
#pragma clang fp contract(off)
    const float s = g / (1.0f + expf(-g));
    return s * u;
}

__device__ __forceinline__ double square_sum4(double acc, float4 v) {
#pragma clang fp contract(off)
    acc += static_cast<double>(v.x) * v.x;
    acc += static_cast<double>(v.y) * v.y;
    acc += static_cast<double>(v.z) * v.z;
    acc += static_cast<double>(v.w) * v.w;
    return acc;
}

// Workgroup = W waves on the same R row tiles; the chunks of K are split
// across the waves.  P = 2: each wave double-buffers whole chunks.  P = 1:
// one chunk buffer, loaded and consumed in turn -- the lower register count
// lets twice as many waves share a CU, which hides the load latency by
// occupancy instead.
//
// Fused step work around the linear (R = 1 only):
//   NORM     x is RMS-normalised first: scale = 1 / sqrt(mean(x^2) + eps)
//            from a double sum of squares over the whole row (every
//            workgroup reduces it, each wave a slice), then x * scale * w;
//   EPI = 0  y = W x + b;  1  y += W x + b (the residual stream);
//   EPI = 2  SwiGLU over a fused gate|up matrix (N = 2F): the workgroup
//            owns gate tile t (waves [0, W/2)) and up tile t + NT/2 (waves
//            [W/2, W)) and writes y[n] = silu(g[n] + b[n]) * (u[n] + b[F + n]).
//
// Pair split (pair_slots != null; R = 1, EPI 0 or 1): two workgroups share a
// row tile, workgroup 2t + h taking half h of its work units, so a narrow
// grid (224 row tiles on 256 CUs) spreads over twice the workgroups.  Each
// half deposits its row sums with one 64-bit atomic exchange per row of
// (float bits << 32 | 1 + h) into pair_slots[n]; the half that finds its
// partner's word there adds the two, writes y and puts the slot back to
// zero.  Value and flag travel in the same atomic word, so no fence is
// needed, and IEEE addition is commutative, so y is the same whichever half
// arrives second.  The slots start at zero and every launch leaves them so;
// launches on one slot array must not overlap.
template <int FMT, int R, int P, int U, bool NORM, int EPI>
__global__ void __launch_bounds__(64 * gemv_max_waves(R, P))
decode_gemv_kernel(const void* __restrict__ codes_, const void* __restrict__ scales_,
                   const float* __restrict__ x, const float* __restrict__ bias, float* __restrict__ y,
                   std::uint64_t K, std::uint64_t N, std::uint32_t NT, std::uint32_t KT,
                   const float* __restrict__ norm_w, double eps, std::uint64_t* __restrict__ pair_slots) {
    extern __shared__ float wave_sums[];
    using Ch = Chunk<FMT, R, U, NORM>;
    const std::uint32_t lane = threadIdx.x & 63u;
    // Wave-uniform: chunk indices, tile addresses and liveness stay scalar.
    const std::uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const std::uint32_t W = blockDim.x >> 6;
    const std::uint32_t group_waves = EPI == 2 ? W / 2u : W;       // waves per row tile
    const bool up_half = EPI == 2 && wave >= group_waves;
    const std::uint32_t gw = up_half ? wave - group_waves : wave;
    const bool pair = EPI != 2 && R == 1 && pair_slots != nullptr;
    const std::uint32_t half = pair ? (blockIdx.x & 1u) : 0u;
    const std::uint32_t group = pair ? (blockIdx.x >> 1) : blockIdx.x;
    const std::uint32_t rt0 = EPI == 2 ? group + (up_half ? NT / 2u : 0u) : group * R;
    const std::uint64_t nblocks = K / 32u;
    // Work units of Ch::kTiles k tiles (U per 16-block chunk), split over the
    // waves of the row tile (of both workgroups of a pair).
    const std::uint32_t chunks = static_cast<std::uint32_t>(ceil_div(KT, static_cast<std::uint64_t>(Ch::kTiles) * U));
    const std::uint64_t units = static_cast<std::uint64_t>(chunks) * U;
    const std::uint32_t tile_waves = pair ? 2u * group_waves : group_waves;
    const std::uint32_t vw = half * group_waves + gw;
    const std::uint32_t c_begin = static_cast<std::uint32_t>((units * vw) / tile_waves);
    const std::uint32_t c_end = static_cast<std::uint32_t>((units * (vw + 1u)) / tile_waves);

    float4v acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = float4v{0.0f, 0.0f, 0.0f, 0.0f};

    Ch a, b;

    float norm_scale = 1.0f;
    if constexpr (NORM) {
        __shared__ double norm_red[16];
        double ss = 0.0;
        for (std::uint64_t i = threadIdx.x; i < K / 4u; i += blockDim.x) {
            ss = square_sum4(ss, reinterpret_cast<const float4*>(x)[i]);
        }
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
        if (lane == 0u) norm_red[wave] = ss;
        __syncthreads();
        double total = 0.0;
        for (std::uint32_t w = 0; w < W; ++w) total += norm_red[w];
        norm_scale = static_cast<float>(1.0 / sqrt(total / static_cast<double>(K) + eps));
    }

    if constexpr (P == 1) {
        for (std::uint32_t c = c_begin; c < c_end; ++c) {
            load_chunk<FMT, R, U, NORM>(a, codes_, scales_, rt0, NT, KT, c, lane, x, norm_w, nblocks);
            compute_chunk<FMT, R, U, NORM>(a, c, lane, norm_scale, acc);
        }
    } else {
        if (c_begin < c_end) {
            load_chunk<FMT, R, U, NORM>(a, codes_, scales_, rt0, NT, KT, c_begin, lane, x, norm_w, nblocks);
        }
        for (std::uint32_t c = c_begin; c < c_end; c += 2u) {
            if (c + 1u < c_end) {
                load_chunk<FMT, R, U, NORM>(b, codes_, scales_, rt0, NT, KT, c + 1u, lane, x, norm_w, nblocks);
            }
            compute_chunk<FMT, R, U, NORM>(a, c, lane, norm_scale, acc);
            if (c + 1u >= c_end) break;
            if (c + 2u < c_end) {
                load_chunk<FMT, R, U, NORM>(a, codes_, scales_, rt0, NT, KT, c + 2u, lane, x, norm_w, nblocks);
            }
            compute_chunk<FMT, R, U, NORM>(b, c + 1u, lane, norm_scale, acc);
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
    float up_total = 0.0f;   // EPI 2: the up tile's sum
    if (W > 1u) {
        if (wave > 0u && lane < 16u) {
#pragma unroll
            for (int r = 0; r < R; ++r) wave_sums[((wave - 1u) * R + r) * 16u + lane] = total[r];
        }
        __syncthreads();
        if (wave == 0u && lane < 16u) {
            if constexpr (EPI == 2) {
                for (std::uint32_t w = 1; w < group_waves; ++w) total[0] += wave_sums[(w - 1u) * 16u + lane];
                up_total = wave_sums[(group_waves - 1u) * 16u + lane];
                for (std::uint32_t w = group_waves + 1u; w < W; ++w) up_total += wave_sums[(w - 1u) * 16u + lane];
            } else {
                for (std::uint32_t w = 1; w < W; ++w) {
#pragma unroll
                    for (int r = 0; r < R; ++r) total[r] += wave_sums[((w - 1u) * R + r) * 16u + lane];
                }
            }
        }
    }
    if (wave != 0u || lane >= 16u) return;
    if constexpr (EPI == 2) {
        const std::uint64_t F = N / 2u;
        const std::uint64_t n = static_cast<std::uint64_t>(group) * 16u + lane;
        if (n < F) {
            const float g = total[0] + (bias ? bias[n] : 0.0f);
            const float u = up_total + (bias ? bias[F + n] : 0.0f);
            y[n] = swiglu(g, u);
        }
    } else {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const std::uint64_t n = static_cast<std::uint64_t>(rt0 + r) * 16u + lane;
            if ((rt0 + r) >= NT || n >= N) continue;
            float sum = total[r];
            if (pair) {
                const std::uint64_t mine =
                    (static_cast<std::uint64_t>(__float_as_uint(sum)) << 32) | static_cast<std::uint64_t>(1u + half);
                const std::uint64_t other =
                    __hip_atomic_exchange(pair_slots + n, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (other == 0u) continue;   // the partner finishes the row
                __hip_atomic_store(pair_slots + n, std::uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                sum = sum + __uint_as_float(static_cast<std::uint32_t>(other >> 32));
            }
            const float out = sum + (bias ? bias[n] : 0.0f);
            if constexpr (EPI == 1) {
                y[n] = y[n] + out;
            } else {
                y[n] = out;
            }
        }
    }
}

template <int FMT, int R, int P, int U, bool NORM, int EPI>
hipError_t launch_gemv_variant(const TilePlanes& p, const float* x, const float* bias, float* y,
                               std::uint32_t W, const GemvFusion& f, std::uint64_t* pair_slots, hipStream_t stream) {
    if (W == 0u || W > static_cast<std::uint32_t>(gemv_max_waves(R, P))) return hipErrorInvalidConfiguration;
    if (EPI == 2 && (W % 2u != 0u || p.nt % 2u != 0u)) return hipErrorInvalidConfiguration;
    if (pair_slots && (EPI == 2 || R != 1 || p.n > kGemvPairSlots)) return hipErrorInvalidConfiguration;
    const unsigned groups = EPI == 2 ? p.nt / 2u : static_cast<unsigned>(ceil_div(p.nt, R));
    const std::size_t lds = static_cast<std::size_t>(W - 1u) * R * 16u * sizeof(float);
    decode_gemv_kernel<FMT, R, P, U, NORM, EPI><<<dim3(pair_slots ? 2u * groups : groups), 64u * W, lds, stream>>>(
        p.codes, p.scales, x, bias, y, p.k, p.n, p.nt, p.kt, f.norm_weight, f.eps, pair_slots);
    return hipGetLastError();
}

// One row tile per wave (the fused step variants).
template <int FMT, bool NORM, int EPI>
hipError_t launch_gemv_r1(const TilePlanes& p, const float* x, const float* bias, float* y, const GemvShape& g,
                          const GemvFusion& f, std::uint64_t* pairs, hipStream_t s) {
    const std::uint32_t W = g.waves_per_group, P = g.depth;
    if (g.units_per_chunk == 2u) {
        return P == 1u ? launch_gemv_variant<FMT, 1, 1, 2, NORM, EPI>(p, x, bias, y, W, f, pairs, s)
                       : launch_gemv_variant<FMT, 1, 2, 2, NORM, EPI>(p, x, bias, y, W, f, pairs, s);
    }
    return P == 1u ? launch_gemv_variant<FMT, 1, 1, 1, NORM, EPI>(p, x, bias, y, W, f, pairs, s)
                   : launch_gemv_variant<FMT, 1, 2, 1, NORM, EPI>(p, x, bias, y, W, f, pairs, s);
}

template <int FMT>
hipError_t launch_gemv_fmt(const TilePlanes& p, const float* x, const float* bias, float* y, const GemvShape& g,
                           const GemvFusion& f, std::uint64_t* pair_slots, hipStream_t s) {
    const bool norm = f.norm_weight != nullptr;
    std::uint64_t* pairs = g.pair_split ? pair_slots : nullptr;
    if (g.pair_split && !pairs) return hipErrorInvalidValue;
    if (norm || f.epilogue != 0) {
        if (g.rows_per_wave != 1u) return hipErrorInvalidConfiguration;
        if (!norm && f.epilogue == 1) return launch_gemv_r1<FMT, false, 1>(p, x, bias, y, g, f, pairs, s);
        if (!norm && f.epilogue == 2) return launch_gemv_r1<FMT, false, 2>(p, x, bias, y, g, f, pairs, s);
        if (norm && f.epilogue == 0) return launch_gemv_r1<FMT, true, 0>(p, x, bias, y, g, f, pairs, s);
        if (norm && f.epilogue == 2) return launch_gemv_r1<FMT, true, 2>(p, x, bias, y, g, f, pairs, s);
        return hipErrorInvalidValue;
    }
    const std::uint32_t R = g.rows_per_wave, W = g.waves_per_group, P = g.depth;
    if (R == 1u) return launch_gemv_r1<FMT, false, 0>(p, x, bias, y, g, f, pairs, s);
    if (R == 2u) {
        return P == 1u ? launch_gemv_variant<FMT, 2, 1, 1, false, 0>(p, x, bias, y, W, f, pairs, s)
                       : launch_gemv_variant<FMT, 2, 2, 1, false, 0>(p, x, bias, y, W, f, pairs, s);
    }
    return P == 1u ? launch_gemv_variant<FMT, 4, 1, 1, false, 0>(p, x, bias, y, W, f, pairs, s)
                   : launch_gemv_variant<FMT, 4, 2, 1, false, 0>(p, x, bias, y, W, f, pairs, s);
}

} // namespace

GemvShape plan_decode_gemv(const TilePlanes& p, const DecodeTuning& tuning) {
    GemvShape g{};
    const std::uint32_t tiles_per_chunk = kChunkBlocks / (geometry_of(p.type).tile_k / 32u);
    const std::uint32_t chunks = static_cast<std::uint32_t>(ceil_div(p.kt, tiles_per_chunk));
    // One row tile per wave (measured best for every Qwen2 shape), then by
    // grid width and K (Qwen2-7B Q8_0, HIP-graph replay):
    //  * very wide grids (>= 4096 row groups, lm_head): four single-buffered
    //    waves per workgroup -- half the registers of double buffering, so
    //    twice the waves per CU keep the loads in flight;
    //  * Q8_0 with short K (<= 8 chunks: q|k|v, o, gate|up): each chunk is
    //    split into two units of half its tiles, so more, shorter waves share
    //    a row tile (one unit per wave up to 16 waves, 8 single-buffered waves
    //    on wide grids) -- 4-7 % faster on those shapes.  The 4-bit formats
    //    are bound by instruction issue, and a unit split doubles the
    //    activation-split work per weight byte (measured 4-5 % slower);
    //  * otherwise (down; the 4-bit formats): the chunks split over the
    //    waves until the grid holds about 8192 waves, up to 16 single-
    //    buffered ones (down) or double-buffered when a wave owns several.
    g.rows_per_wave = 1u;
    if (tuning.rows_per_wave == 1u || tuning.rows_per_wave == 2u || tuning.rows_per_wave == 4u) {
        g.rows_per_wave = tuning.rows_per_wave;
    }
    const std::uint64_t groups = ceil_div(p.nt, g.rows_per_wave);
    const bool huge = groups >= 4096u;
    const bool wide = groups >= 2048u;
    const bool short_k = chunks <= 8u;
    g.units_per_chunk = (p.type == kQ8_0 && g.rows_per_wave == 1u && short_k && !huge) ? 2u : 1u;
    // Half-chunk units exist for Q8_0 only (a 4-bit chunk's tiles do not
    // split in two): the override asks for them there alone.
    if (g.rows_per_wave == 1u && (tuning.units_per_chunk == 1u || (tuning.units_per_chunk == 2u && p.type == kQ8_0))) {
        g.units_per_chunk = tuning.units_per_chunk;
    }
    const std::uint64_t units = static_cast<std::uint64_t>(chunks) * g.units_per_chunk;
    std::uint64_t w;
    if (huge) {
        w = 4u;
    } else if (g.units_per_chunk == 2u) {
        w = wide ? 8u : units;
    } else {
        w = ceil_div(8192u, groups);
    }
    if (tuning.waves_per_group != 0u) w = tuning.waves_per_group;
    if (w > units) w = units;
    if (w == 0u) w = 1u;
    // Units in flight per wave: one for wide grids and when no wave owns
    // more than one unit, else two; the buffer count bounds the waves.
    const auto depth_for = [&](std::uint64_t waves) -> std::uint32_t {
        if (tuning.depth == 1u || tuning.depth == 2u) return tuning.depth;   // a forced depth bounds the waves
        return (wide || ceil_div(units, waves) <= 1u) ? 1u : 2u;
    };
    const std::uint64_t wanted = w;
    std::uint32_t depth = depth_for(w);
    for (int pass = 0; pass < 2; ++pass) {
        const std::uint64_t cap = static_cast<std::uint64_t>(gemv_max_waves(static_cast<int>(g.rows_per_wave),
                                                                            static_cast<int>(depth)));
        if (w > cap) w = cap;
        depth = depth_for(w);
    }
    // Long K on a narrow grid (down: 224 row tiles, 37 chunks each) runs
    // single-buffered waves.  A workgroup ends with its wave of most chunks,
    // so the count is chosen for balance (warmed graph replay of 12 distinct
    // copies of down, us per launch):
    //  * Q8_0: eight waves (5 or 4 chunks each) 14.75-14.86, thirteen 15.03,
    //    sixteen 15.31-15.67 (eight double-buffered 15.50); the M = 1 step
    //    1.536 -> 1.520 ms;
    //  * the 4-bit formats: from twelve to sixteen waves, the count whose
    //    chunks spread most evenly -- thirteen for 37 chunks (2.85 of at most
    //    3 each): Q4_0 11.68-11.87 against sixteen's 12.09-12.22 and eight's
    //    12.78-12.83, Q4_K 12.42-12.61 against 12.68-12.76.
    if (tuning.waves_per_group == 0u && !wide && g.units_per_chunk == 1u && g.rows_per_wave == 1u && wanted > 8u) {
        w = wanted > 16u ? 16u : wanted;
        if (p.type == kQ8_0) {
            w = 8u;
        } else if (w == 16u && units > 16u) {
            std::uint64_t best = 16u;
            for (std::uint64_t c = 16u; c >= 12u; --c) {
                // balance = units / (c * ceil(units / c)); compare cross-multiplied
                if (c * ceil_div(units, c) < best * ceil_div(units, best)) best = c;
            }
            w = best;
        }
        depth = 1u;
    }
    // A grid just past one workgroup per CU (q|k|v: 288 row tiles on 256
    // CUs) ends in a round of few workgroups: split each tile's units over a
    // pair of workgroups with half the waves each.  Measured (Q8_0, 288-304
    // row tiles): K = 3584 (14 units) 7.00 -> 6.71 us, K = 2048 (8) 5.37 ->
    // 5.29; K = 1536 (6) even; K = 896 (4) 4.17 -> 4.37, two waves a side.
    const bool pair_fits = g.rows_per_wave == 1u && p.n <= kGemvPairSlots && units >= 2u;
    bool pair = pair_fits && groups > 256u && groups <= 320u && units >= 8u;
    if (tuning.pair_split == 1u) pair = false;
    if (tuning.pair_split == 2u) pair = pair_fits;
    if (pair && tuning.waves_per_group == 0u) {
        w = (w + 1u) / 2u;
        depth = depth_for(2u * w);
    }
    if (tuning.depth == 1u || tuning.depth == 2u) depth = tuning.depth;
    {
        const std::uint64_t cap = static_cast<std::uint64_t>(gemv_max_waves(static_cast<int>(g.rows_per_wave),
                                                                            static_cast<int>(depth)));
        if (w > cap) w = cap;
    }
    g.waves_per_group = static_cast<std::uint32_t>(w);
    g.depth = depth;
    g.pair_split = pair ? 1u : 0u;
    return g;
}

GemvShape plan_decode_gemv_fused(const TilePlanes& p, const DecodeTuning& tuning, int epilogue) {
    // The SwiGLU workgroup holds a gate tile and its up tile: no pair split.
    DecodeTuning t = tuning;
    if (epilogue == 2) t.pair_split = 1u;
    GemvShape g = plan_decode_gemv(p, t);
    g.rows_per_wave = 1u;
    if (g.units_per_chunk == 2u && p.type != kQ8_0) g.units_per_chunk = 1u;
    if (epilogue == 2) {
        // A gate tile and its up tile per workgroup: twice the waves of the
        // plain plan, single-buffered past eight.
        std::uint32_t w = 2u * g.waves_per_group;
        if (w > 16u) w = 16u;
        if (w > 8u) g.depth = 1u;
        g.waves_per_group = w < 2u ? 2u : w;
    }
    return g;
}

hipError_t launch_decode_gemv(const TilePlanes& p, const float* x, const float* bias, float* y,
                              const GemvShape& g, std::uint64_t* pair_slots, hipStream_t stream) {
    return launch_decode_gemv_fused(p, x, bias, y, g, GemvFusion{}, pair_slots, stream);
}

hipError_t launch_decode_gemv_fused(const TilePlanes& p, const float* x, const float* bias, float* y,
                                    const GemvShape& g, const GemvFusion& f, std::uint64_t* pair_slots,
                                    hipStream_t stream) {
    switch (p.type) {
    case kQ8_0: return launch_gemv_fmt<kQ8_0>(p, x, bias, y, g, f, pair_slots, stream);
    case kQ4_0: return launch_gemv_fmt<kQ4_0>(p, x, bias, y, g, f, pair_slots, stream);
    case kQ4_K: return launch_gemv_fmt<kQ4_K>(p, x, bias, y, g, f, pair_slots, stream);
    default: return hipErrorInvalidValue;
    }
}

} // namespace air_hip

// linear_dense.hip -- linears over matrices held as dense rows.
//
// The encodings with no resident tile format here (F32, F16, BF16 and Q6_K;
// decode_element, src/cuda/cuda_backend.cu:241-344, decodes them per
// element inside every GEMV) are held as rows w[n][k] in their own bytes:
// F32, F16 and BF16 as the GGUF rows, Q6_K as its 256-weight super-blocks
// split into 208-byte records (the codes and 6-bit sub-block scales, 16-byte
// aligned) and a plane of the blocks' f16 scales d after them: the file's
// 210 bytes per 256 weights, no more.  The kernels decode four consecutive
// weights at a time to f32 exactly as the reference decodes each element
// (Q6_K: (d * scale) * q), so a Q6_K linear streams the file's bytes.  A real
// Qwen2.5 Q4_K_M file carries Q6_K tensors (lm_head, half the ffn_down /
// attn_v) and F16 / BF16 files carry every linear this way.  Plain f32 FMA
// with f32 accumulation, one launch per linear, no workspace:
//   rows 1..64: dense_rows_kernel, four output columns per workgroup for up
//               to 16 rows of x (K split over its four waves); the weights
//               are read once per 16 rows;
//   more rows:  dense_gemm_kernel, 64 x 64 output tiles staged through LDS.
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"

namespace air_hip {
namespace {

constexpr unsigned kDenseThreads = 256;
constexpr unsigned kDenseCols = 4;       // output columns per wave (rows kernel)
constexpr unsigned kDenseMaxRows = 16;   // rows of x per workgroup of the rows kernel
constexpr unsigned kDenseRowsKernelMax = 64;   // wider x: the tiled GEMM
constexpr unsigned kGemmTile = 64;
constexpr unsigned kGemmK = 32;

// Q6_K super-block record: 192 bytes of codes, then the 16 int8 sub-block
// scales; block b's f16 d is entry b of the plane that follows all
// `nblocks` records.  The codes are the canonical block's ql / qh bytes
// regrouped by the lane that reads them: element e = 128 h + 32 j + 16 s + i
// (half h, quadrant j, half-quadrant s, i < 16) has its low nibble (nibble
// j / 2) in canonical ql byte 64 h + 32 (j % 2) + 16 s + i and its high pair
// (bits 2j, 2j + 1) in qh byte 32 h + 16 s + i (src/reference/tensor_reader.cpp:197-242);
// with g = i / 4, lane group g's 48 bytes hold those 4-byte runs at
//     b = 12 (2 h + s) + {0: ql of j % 2 = 0, 4: ql of j % 2 = 1, 8: qh},
// and its byte b lies at q6k_code_offset(g, b) = 48 g + b: a lane group
// reads its whole super-block (its four elements of each of the 16
// sub-blocks) in three 16-byte loads.
constexpr std::uint32_t kQ6kRecord = 208;

// Byte offset in a record of the 4-byte run of element e's low nibbles
// (qh = false) or high pairs (qh = true); e a multiple of 4.
__device__ __forceinline__ std::uint32_t q6k_run(std::uint32_t e, bool qh) {
    const std::uint32_t h = e >> 7, j = (e >> 5) & 3u, s = (e >> 4) & 1u, g = (e >> 2) & 3u;
    return q6k_code_offset(g, 12u * (2u * h + s) + (qh ? 8u : 4u * (j & 1u)));
}

typedef _Float16 half4v __attribute__((ext_vector_type(4)));

// Four Q6_K codes (low nibbles in the low half of `nib`'s bytes, high pairs
// in bits 4-5 of `hib`'s bytes) as exact f16 values q - 32: 1024 + q under
// the exponent byte 0x64, minus 1056.
__device__ __forceinline__ half4v q6_codes4(std::uint32_t nib, std::uint32_t hib) {
    const std::uint32_t u = (nib & 0x0f0f0f0fu) | (hib & 0x30303030u);
    const half2v bias = {(_Float16)1056.0f, (_Float16)1056.0f};
    const half2v lo = bits_as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias;
    const half2v hi = bits_as_half2(__builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias;
    return half4v{lo[0], lo[1], hi[0], hi[1]};
}

__device__ __forceinline__ const std::uint16_t* q6k_d_plane(const void* w, std::uint64_t nblocks) {
    return reinterpret_cast<const std::uint16_t*>(static_cast<const unsigned char*>(w) + nblocks * kQ6kRecord);
}

// Four consecutive weights w[idx .. idx + 3] (idx a multiple of 4) of a
// dense matrix stored as WT (f32, f16 / bf16 bits, or Q6_K records of a
// matrix of nblocks super-blocks), as exact f32.  Q6_K: a row is whole
// super-blocks (k a multiple of 256), so element idx lies in record idx /
// 256 at position e = idx % 256 (quadrant j = e / 32 % 4); four weights
// share a 4-byte run of low nibbles (nibble j / 2), one of high pairs (bits
// 2j, 2j + 1) and the sub-block scale e / 16; each is (d * sc) * (q - 32),
// the reference's decode (src/reference/tensor_reader.cpp:197-242).
template <int WT>
__device__ __forceinline__ float4 load_w4(const void* __restrict__ w, std::uint64_t idx, std::uint64_t nblocks) {
    if constexpr (WT == kQ6_K) {
        const unsigned char* rec = static_cast<const unsigned char*>(w) + (idx >> 8) * kQ6kRecord;
        const std::uint32_t e = static_cast<std::uint32_t>(idx & 255u);
        const std::uint32_t j = (e >> 5) & 3u;
        const std::uint32_t ql = *reinterpret_cast<const std::uint32_t*>(rec + q6k_run(e, false));
        const std::uint32_t qh = *reinterpret_cast<const std::uint32_t*>(rec + q6k_run(e, true));
        const float d = f16_bits_to_f32(q6k_d_plane(w, nblocks)[idx >> 8]);
        // Sub-block e / 16 = 8 h + 2 j + s.
        const int sc = static_cast<int>(static_cast<std::int8_t>(rec[192u + (e >> 4)]));
        const float ds = d * static_cast<float>(sc);
        const std::uint32_t nib = (j >> 1) ? (ql >> 4) & 0x0f0f0f0fu : ql & 0x0f0f0f0fu;
        const std::uint32_t hb = (qh >> (2u * j)) & 0x03030303u;
        const std::uint32_t q = nib | (hb << 4);
        const auto val = [&](std::uint32_t b) {
            return ds * static_cast<float>(static_cast<int>((q >> (8u * b)) & 0xffu) - 32);
        };
        return make_float4(val(0), val(1), val(2), val(3));
    } else if constexpr (WT == kF32) {
        return *reinterpret_cast<const float4*>(static_cast<const float*>(w) + idx);
    } else {
        const uint2 v = *reinterpret_cast<const uint2*>(static_cast<const std::uint16_t*>(w) + idx);
        if constexpr (WT == kF16) {
            const auto h = [](std::uint32_t b) {
                return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(b)));
            };
            return make_float4(h(v.x & 0xffffu), h(v.x >> 16), h(v.y & 0xffffu), h(v.y >> 16));
        } else {
            return make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u),
                               __uint_as_float(v.y << 16), __uint_as_float(v.y & 0xffff0000u));
        }
    }
}

// One workgroup per kDenseCols output columns and MB rows of x; its four
// waves split K (wave w takes the 256-element steps w, w + 4, ...), each
// lane strides its wave's steps by float4, and the four partial sums meet in
// LDS in a fixed order.
template <unsigned MB, int WT>
__global__ __launch_bounds__(kDenseThreads) void dense_rows_kernel(const void* __restrict__ w,
                                                                   const float* __restrict__ x,
                                                                   const float* __restrict__ bias,
                                                                   float* __restrict__ y, std::uint32_t m,
                                                                   std::uint64_t k, std::uint64_t n) {
    constexpr unsigned kWaves = kDenseThreads / 64u;
    __shared__ float red[kWaves][MB][kDenseCols];
    const std::uint64_t nblocks = k * n / 256u;   // Q6_K super-blocks (the d plane's offset)
    const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const std::uint64_t n0 = static_cast<std::uint64_t>(blockIdx.x) * kDenseCols;
    const std::uint32_t r0 = blockIdx.y * MB;
    const std::uint32_t rows = m - r0 < MB ? m - r0 : MB;
    x += static_cast<std::uint64_t>(r0) * k;
    y += static_cast<std::uint64_t>(r0) * n;
    std::uint64_t wr[kDenseCols];   // element index of each column's row
#pragma unroll
    for (unsigned c = 0; c < kDenseCols; ++c) {
        const std::uint64_t col = n0 + c < n ? n0 + c : n - 1u;   // clamped; not stored
        wr[c] = col * k;
    }
    float acc[MB][kDenseCols];
#pragma unroll
    for (unsigned i = 0; i < MB; ++i)
#pragma unroll
        for (unsigned c = 0; c < kDenseCols; ++c) acc[i][c] = 0.0f;
    for (std::uint64_t kk = 4u * (lane + 64u * wave); kk < k; kk += 4u * kDenseThreads) {
        float4 wv[kDenseCols];
#pragma unroll
        for (unsigned c = 0; c < kDenseCols; ++c) wv[c] = load_w4<WT>(w, wr[c] + kk, nblocks);
#pragma unroll
        for (unsigned i = 0; i < MB; ++i) {
            if (i < rows) {
                const float4 xv = *reinterpret_cast<const float4*>(x + i * k + kk);
#pragma unroll
                for (unsigned c = 0; c < kDenseCols; ++c) {
                    acc[i][c] = fmaf(wv[c].x, xv.x, acc[i][c]);
                    acc[i][c] = fmaf(wv[c].y, xv.y, acc[i][c]);
                    acc[i][c] = fmaf(wv[c].z, xv.z, acc[i][c]);
                    acc[i][c] = fmaf(wv[c].w, xv.w, acc[i][c]);
                }
            }
        }
    }
#pragma unroll
    for (unsigned i = 0; i < MB; ++i) {
#pragma unroll
        for (unsigned c = 0; c < kDenseCols; ++c) {
            float v = acc[i][c];
            for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
            if (lane == 0u) red[wave][i][c] = v;
        }
    }
    __syncthreads();
    if (threadIdx.x < MB * kDenseCols) {
        const unsigned i = threadIdx.x / kDenseCols, c = threadIdx.x % kDenseCols;
        if (i < rows && n0 + c < n) {
            float v = red[0][i][c];
#pragma unroll
            for (unsigned q = 1; q < kWaves; ++q) v += red[q][i][c];
            y[static_cast<std::uint64_t>(i) * n + n0 + c] = bias ? v + bias[n0 + c] : v;
        }
    }
}

template <int WT>
__global__ __launch_bounds__(kDenseThreads) void dense_gemm_kernel(const void* __restrict__ w,
                                                                   const float* __restrict__ x,
                                                                   const float* __restrict__ bias,
                                                                   float* __restrict__ y, std::uint32_t m,
                                                                   std::uint64_t k, std::uint64_t n) {
    // k-major tiles (4 floats of padding keep float4 reads aligned).
    __shared__ float xs[kGemmK][kGemmTile + 4];
    __shared__ float ws[kGemmK][kGemmTile + 4];
    const std::uint64_t nblocks = k * n / 256u;   // Q6_K super-blocks (the d plane's offset)
    const unsigned t = threadIdx.x, tx = t & 15u, ty = t >> 4;
    const std::uint64_t n0 = static_cast<std::uint64_t>(blockIdx.x) * kGemmTile;
    const std::uint64_t m0 = static_cast<std::uint64_t>(blockIdx.y) * kGemmTile;
    float acc[4][4];
#pragma unroll
    for (unsigned i = 0; i < 4; ++i)
#pragma unroll
        for (unsigned j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (std::uint64_t k0 = 0; k0 < k; k0 += kGemmK) {
        // 64 rows x 32 k of each operand: 512 float4, two per thread.
#pragma unroll
        for (unsigned h = 0; h < 2; ++h) {
            const unsigned idx = t + kDenseThreads * h, row = idx >> 3, kq = (idx & 7u) * 4u;
            float4 xv = make_float4(0.f, 0.f, 0.f, 0.f), wv = make_float4(0.f, 0.f, 0.f, 0.f);
            if (m0 + row < m) xv = *reinterpret_cast<const float4*>(x + (m0 + row) * k + k0 + kq);
            if (n0 + row < n) wv = load_w4<WT>(w, (n0 + row) * k + k0 + kq, nblocks);
            xs[kq + 0][row] = xv.x;
            xs[kq + 1][row] = xv.y;
            xs[kq + 2][row] = xv.z;
            xs[kq + 3][row] = xv.w;
            ws[kq + 0][row] = wv.x;
            ws[kq + 1][row] = wv.y;
            ws[kq + 2][row] = wv.z;
            ws[kq + 3][row] = wv.w;
        }
        __syncthreads();
#pragma unroll 8
        for (unsigned kk = 0; kk < kGemmK; ++kk) {
            const float4 a = *reinterpret_cast<const float4*>(&xs[kk][4u * ty]);
            const float4 b = *reinterpret_cast<const float4*>(&ws[kk][4u * tx]);
            const float av[4] = {a.x, a.y, a.z, a.w};
            const float bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (unsigned i = 0; i < 4; ++i)
#pragma unroll
                for (unsigned j = 0; j < 4; ++j) acc[i][j] = fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (unsigned i = 0; i < 4; ++i) {
        const std::uint64_t row = m0 + 4u * ty + i;
#pragma unroll
        for (unsigned j = 0; j < 4; ++j) {
            const std::uint64_t col = n0 + 4u * tx + j;
            if (row < m && col < n) y[row * n + col] = bias ? acc[i][j] + bias[col] : acc[i][j];
        }
    }
}

// Embedding rows: out[i] = w[rows[i]] decoded exactly (f16 bits through
// f16_bits_to_f32, the canonical decode's conversion).
template <int WT>
__global__ __launch_bounds__(kDenseThreads) void dense_rows_gather_kernel(const void* __restrict__ w,
                                                                          std::uint64_t k, std::uint64_t n,
                                                                          const std::int32_t* __restrict__ rows,
                                                                          std::uint32_t count,
                                                                          float* __restrict__ out) {
    const std::uint32_t i = blockIdx.y;
    if (i >= count) return;
    const std::int32_t row = rows[i];
    if (row < 0 || static_cast<std::uint64_t>(row) >= n) return;
    const std::uint64_t base = static_cast<std::uint64_t>(row) * k;
    float* dst = out + static_cast<std::uint64_t>(i) * k;
    for (std::uint64_t c = blockIdx.x * static_cast<std::uint64_t>(kDenseThreads) + threadIdx.x; c < k;
         c += static_cast<std::uint64_t>(gridDim.x) * kDenseThreads) {
        if constexpr (WT == kQ6_K) {
            const float4 v = load_w4<kQ6_K>(w, base + (c & ~std::uint64_t{3}), k * n / 256u);
            const std::uint64_t lane4 = c & 3u;
            dst[c] = lane4 == 0u ? v.x : lane4 == 1u ? v.y : lane4 == 2u ? v.z : v.w;
        } else if constexpr (WT == kF32) {
            dst[c] = static_cast<const float*>(w)[base + c];
        } else if constexpr (WT == kF16) {
            dst[c] = f16_bits_to_f32(static_cast<const std::uint16_t*>(w)[base + c]);
        } else {
            dst[c] = __uint_as_float(static_cast<std::uint32_t>(static_cast<const std::uint16_t*>(w)[base + c]) << 16);
        }
    }
}

// One row of x through Q6_K records (M = 1) on the matrix cores.  A
// workgroup owns one 16-row tile; its W waves split the row's super-blocks.
// Per super-block the 16 sub-blocks of 16 weights form a block-diagonal
// problem (the M = 1 GEMV's trick, linear_gemv.hip): A row r holds the
// activations of sub-block r (lane l: row l % 16, elements 4 (l / 16)..+3),
// split into f16 hi + lo under one power-of-two scale per super-block; the
// 16x16x16 MFMAs of sub-block j take the exact f16 codes q - 32 of the 16
// rows (lane l: row l % 16, the same four elements, from the lane group's
// contiguous 48 bytes of the record) against A with only row j live, so
// they accumulate and D row j (lane group j / 4, slot j % 4) ends with the
// sub-block's products, which take its own scale sc (exact in f32; the lane
// group's four scales are one dword of the record).  Per super-block, the
// scaled slots times d * (inverse activation scale); the waves' row sums
// meet in LDS in wave order.
// U super-blocks per work unit (their loads issued together), P units in
// flight per wave (2: the next unit loads while the current computes).
template <int U, int P>
__global__ __launch_bounds__(1024) void q6k_gemv_kernel(const unsigned char* __restrict__ w,
                                                        const float* __restrict__ x, const float* __restrict__ bias,
                                                        float* __restrict__ y, std::uint64_t k, std::uint64_t n) {
    __shared__ float red[16][16];
    const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6, W = blockDim.x >> 6;
    const unsigned g = lane >> 4;
    const std::uint64_t sbs = k / 256u;
    const std::uint64_t row = static_cast<std::uint64_t>(blockIdx.x) * 16u + (lane & 15u);
    const bool live = row < n;
    const std::uint64_t rrow = live ? row : n - 1u;   // padded rows read the last real row, not stored
    const std::uint16_t* dplane = q6k_d_plane(w, sbs * n);
    const std::uint64_t units = (sbs + U - 1u) / U;
    const std::uint64_t u0 = units * wave / W, u1 = units * (wave + 1u) / W;
    // Loads of one super-block (plain vector variables: a struct of them
    // would live in scratch memory).
    const auto load = [&](std::uint64_t sb, u32x4& c0, u32x4& c1, u32x4& c2, std::uint32_t& scw, std::uint32_t& dbits,
                          float4v& xv) __attribute__((always_inline)) {
        const std::uint64_t blk = rrow * sbs + sb;
        const unsigned char* rec = w + blk * kQ6kRecord;
        const u32x4* cp = reinterpret_cast<const u32x4*>(rec + 48u * g);
        c0 = cp[0];   // group bytes 0..15; plain loads: the four groups' loads
        c1 = cp[1];   // of one instruction interleave with the next ones' in
        c2 = cp[2];   // the same lines, which L2 then serves
        scw = *reinterpret_cast<const std::uint32_t*>(rec + 192u + 4u * g);
        dbits = dplane[blk];
        xv = *reinterpret_cast<const float4v*>(x + sb * 256u + 16u * (lane & 15u) + 4u * g);
    };
    float4v acc = {0.0f, 0.0f, 0.0f, 0.0f};
    const auto compute = [&](const u32x4& c0, const u32x4& c1, const u32x4& c2, std::uint32_t scw, std::uint32_t dbits,
                             const float4v& xv) __attribute__((always_inline)) {
        const float amax = wave_max(fmaxf(fmaxf(fabsf(xv[0]), fabsf(xv[1])), fmaxf(fabsf(xv[2]), fabsf(xv[3]))));
        float s, inv;
        block_scale(amax, s, inv);
        const float e8[8] = {xv[0], xv[1], xv[2], xv[3], 0.0f, 0.0f, 0.0f, 0.0f};
        half8v h8, l8;
        split8(e8, s, h8, l8);
        const half4v hi = {h8[0], h8[1], h8[2], h8[3]};
        const half4v lo = {l8[0], l8[1], l8[2], l8[3]};
        // Sub-block jb's MFMAs take A with only row jb live (the other rows
        // zero), so D row jb collects exactly its products and the MFMAs
        // accumulate: four accumulators, jb % 4, keep four chains in flight.
        const half4v zero4 = {(_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f, (_Float16)0.0f};
        const unsigned arow = lane & 15u;
        float4v dacc0 = {0.0f, 0.0f, 0.0f, 0.0f}, dacc1 = dacc0, dacc2 = dacc0, dacc3 = dacc0;
#pragma unroll
        for (int jb = 0; jb < 16; ++jb) {
            // Sub-block jb = 8 h + 2 j + s: group word 3 (2 h + s) + part.
            const int h = jb >> 3, j = (jb >> 1) & 3, sh = jb & 1;
            const int wl = 3 * (2 * h + sh) + (j & 1), wh = 3 * (2 * h + sh) + 2;
            const u32x4& vl = wl < 4 ? c0 : wl < 8 ? c1 : c2;
            const u32x4& vh = wh < 4 ? c0 : wh < 8 ? c1 : c2;
            const std::uint32_t ql = vl[wl & 3];
            const std::uint32_t qh = vh[wh & 3];
            const std::uint32_t nib = (j >> 1) ? (ql >> 4) : ql;
            const std::uint32_t hib = 2 * j <= 4 ? (qh << (4 - 2 * j)) : (qh >> (2 * j - 4));
            const half4v wq = q6_codes4(nib, hib);
            const bool row_live = arow == static_cast<unsigned>(jb);
            const half4v ah = row_live ? hi : zero4;
            const half4v al = row_live ? lo : zero4;
            float4v& dacc = (jb & 3) == 0 ? dacc0 : (jb & 3) == 1 ? dacc1 : (jb & 3) == 2 ? dacc2 : dacc3;
            dacc = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, wq, dacc, 0, 0, 0);
            dacc = __builtin_amdgcn_mfma_f32_16x16x16f16(al, wq, dacc, 0, 0, 0);
        }
        // Lane group g holds D rows 4 g + i: sub-block 4 g + i, in slot i of
        // accumulator i; its scale is byte i of the group's scale dword.
        const auto scale = [&](int i) {
            return static_cast<float>(static_cast<std::int8_t>((scw >> (8 * i)) & 0xffu));
        };
        const float4v cacc = {scale(0) * dacc0[0], scale(1) * dacc1[1], scale(2) * dacc2[2], scale(3) * dacc3[3]};
        const float dv = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(dbits))) * inv;
        acc += dv * cacc;
    };
    // A unit's super-blocks past the row's end load nothing and add nothing.
    u32x4 ac0[U], ac1[U], ac2[U], bc0[U], bc1[U], bc2[U];
    std::uint32_t asc[U], ad[U], bsc[U], bd[U];
    float4v ax[U], bx[U];
    const auto load_unit = [&](std::uint64_t u, u32x4 (&c0)[U], u32x4 (&c1)[U], u32x4 (&c2)[U], std::uint32_t (&sc)[U],
                               std::uint32_t (&d)[U], float4v (&xv)[U]) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            const std::uint64_t sb = u * U + i;
            if (sb < sbs) load(sb, c0[i], c1[i], c2[i], sc[i], d[i], xv[i]);
        }
    };
    const auto compute_unit = [&](std::uint64_t u, const u32x4 (&c0)[U], const u32x4 (&c1)[U], const u32x4 (&c2)[U],
                                  const std::uint32_t (&sc)[U], const std::uint32_t (&d)[U], const float4v (&xv)[U])
        __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < U; ++i) {
            if (u * U + i < sbs) compute(c0[i], c1[i], c2[i], sc[i], d[i], xv[i]);
        }
    };
    if constexpr (P == 1) {
        for (std::uint64_t u = u0; u < u1; ++u) {
            load_unit(u, ac0, ac1, ac2, asc, ad, ax);
            compute_unit(u, ac0, ac1, ac2, asc, ad, ax);
        }
    } else {
        if (u0 < u1) load_unit(u0, ac0, ac1, ac2, asc, ad, ax);
        for (std::uint64_t u = u0; u < u1; u += 2u) {
            if (u + 1u < u1) load_unit(u + 1u, bc0, bc1, bc2, bsc, bd, bx);
            compute_unit(u, ac0, ac1, ac2, asc, ad, ax);
            if (u + 1u >= u1) break;
            if (u + 2u < u1) load_unit(u + 2u, ac0, ac1, ac2, asc, ad, ax);
            compute_unit(u + 1u, bc0, bc1, bc2, bsc, bd, bx);
        }
    }
    // Row l % 16's sum: the four slots, then the four lane groups.
    float t = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    t += __shfl_xor(t, 16);
    t += __shfl_xor(t, 32);
    if (lane < 16u) red[wave][lane] = t;
    __syncthreads();
    if (wave == 0u && lane < 16u && live) {
        float v = red[0][lane];
        for (unsigned q = 1; q < W; ++q) v += red[q][lane];
        y[row] = bias ? v + bias[row] : v;
    }
}

// The whole matrix as f32 [n][k] (resident decode), four weights per thread.
template <int WT>
__global__ __launch_bounds__(kDenseThreads) void dense_dequantize_kernel(const void* __restrict__ w,
                                                                         std::uint64_t quads, float* __restrict__ out) {
    for (std::uint64_t q = blockIdx.x * static_cast<std::uint64_t>(kDenseThreads) + threadIdx.x; q < quads;
         q += static_cast<std::uint64_t>(gridDim.x) * kDenseThreads) {
        reinterpret_cast<float4*>(out)[q] = load_w4<WT>(w, 4u * q, quads / 64u);
    }
}

// Canonical Q6_K blocks (210 bytes: [ql 128][qh 64][scales 16][d 2]) ->
// 208-byte records (the codes in lane-group order, then the scales) and the
// d plane after them; thread t writes output word t of the records, or one
// d entry.
__global__ __launch_bounds__(kDenseThreads) void q6k_records_kernel(const unsigned char* __restrict__ src,
                                                                    std::uint64_t blocks,
                                                                    std::uint32_t* __restrict__ dst) {
    constexpr std::uint32_t kWords = kQ6kRecord / 4u;
    std::uint16_t* dplane = reinterpret_cast<std::uint16_t*>(reinterpret_cast<unsigned char*>(dst) + blocks * kQ6kRecord);
    for (std::uint64_t t = blockIdx.x * static_cast<std::uint64_t>(kDenseThreads) + threadIdx.x;
         t < blocks * (kWords + 1u); t += static_cast<std::uint64_t>(gridDim.x) * kDenseThreads) {
        if (t < blocks * kWords) {
            const std::uint64_t b = t / kWords;
            const std::uint32_t word = static_cast<std::uint32_t>(t % kWords);
            std::uint32_t from;   // canonical byte offset of the word's 4-byte run
            if (word < 48u) {
                // Record byte 4 word = q6k_code_offset(g, b): group word b / 4
                // = 3 (2 h + s) + part, part 0 / 1 the low nibbles of
                // quadrants with j % 2 = part, part 2 the high pairs.
                const std::uint32_t g = word / 12u, gw = word % 12u;
                const std::uint32_t run = gw / 3u, part = gw % 3u;
                const std::uint32_t h = run >> 1, s = run & 1u;
                from = part < 2u ? 64u * h + 32u * part + 16u * s + 4u * g : 128u + 32u * h + 16u * s + 4u * g;
            } else {
                from = 192u + 4u * (word - 48u);   // the scales as they are
            }
            const unsigned char* bytes = src + b * 210u + from;
            dst[t] = static_cast<std::uint32_t>(bytes[0]) | (static_cast<std::uint32_t>(bytes[1]) << 8) |
                     (static_cast<std::uint32_t>(bytes[2]) << 16) | (static_cast<std::uint32_t>(bytes[3]) << 24);
        } else {
            const std::uint64_t b = t - blocks * kWords;
            const unsigned char* bytes = src + b * 210u + 208u;
            dplane[b] = static_cast<std::uint16_t>(bytes[0] | (bytes[1] << 8));
        }
    }
}

} // namespace

// Launch of the Q6_K GEMV (one 16-row tile per workgroup).  Measured on the
// Qwen2-7B shapes (graphs over copies larger than the Infinity Cache): waves
// until the grid holds about 8192, at least two and at most 16 (one per
// super-block); one super-block per work unit; one unit in flight for long
// rows (down, 74 super-blocks: 22.3 us, flat within 0.5 us over 4..16 waves
// and both depths), two for short ones (o 6.5 us, lm_head 127 us; the FMA
// GEMV it replaced took 22.9, 6.9 and 192).
std::uint32_t q6k_gemv_waves(std::uint64_t k, std::uint64_t n, std::uint32_t waves) {
    const std::uint64_t sbs = k / 256u, tiles = ceil_div(n, 16u);
    std::uint64_t w = waves != 0u ? waves : ceil_div(8192u, tiles);
    if (waves == 0u && w < 2u) w = 2u;
    if (w > 16u) w = 16u;
    if (w > sbs) w = sbs;
    return static_cast<std::uint32_t>(w < 1u ? 1u : w);
}

Q6kGemvPlan plan_q6k_gemv(std::uint64_t k, std::uint64_t n, const DenseMfmaShape& tuning) {
    Q6kGemvPlan g;
    g.waves = q6k_gemv_waves(k, n, tuning.waves);
    g.units = tuning.tile_n == 2u ? 2u : 1u;
    g.depth = tuning.depth == 4u ? 1u : tuning.depth == 2u ? 2u : (k / 256u >= 32u ? 1u : 2u);
    return g;
}

std::uint64_t dense_resident_bytes(int storage, std::uint64_t k, std::uint64_t n) {
    switch (storage) {
    case kF32: return k * n * 4u;
    case kF16: case kBF16: return k * n * 2u;
    case kQ6_K: return k % 256u == 0u ? k * n / 256u * (kQ6kRecord + 2u) : 0u;
    default: return 0u;
    }
}

hipError_t launch_q6k_records(const void* canonical, std::uint64_t blocks, void* records, hipStream_t stream) {
    const std::uint64_t words = blocks * (kQ6kRecord / 4u + 1u);
    const unsigned grid = static_cast<unsigned>(std::min<std::uint64_t>(ceil_div(words, kDenseThreads), 65535u));
    hipLaunchKernelGGL(q6k_records_kernel, dim3(grid), dim3(kDenseThreads), 0, stream,
                       static_cast<const unsigned char*>(canonical), blocks, static_cast<std::uint32_t*>(records));
    return hipGetLastError();
}

hipError_t launch_dense_dequantize(const void* w, int storage, std::uint64_t k, std::uint64_t n, float* out,
                                   hipStream_t stream) {
    if (k % 4u != 0u) return hipErrorInvalidValue;
    const std::uint64_t quads = k * n / 4u;
    const unsigned grid = static_cast<unsigned>(std::min<std::uint64_t>(ceil_div(quads, kDenseThreads), 65535u));
    switch (storage) {
    case kF32: hipLaunchKernelGGL(dense_dequantize_kernel<kF32>, dim3(grid), dim3(kDenseThreads), 0, stream, w, quads, out); break;
    case kF16: hipLaunchKernelGGL(dense_dequantize_kernel<kF16>, dim3(grid), dim3(kDenseThreads), 0, stream, w, quads, out); break;
    case kBF16: hipLaunchKernelGGL(dense_dequantize_kernel<kBF16>, dim3(grid), dim3(kDenseThreads), 0, stream, w, quads, out); break;
    case kQ6_K: hipLaunchKernelGGL(dense_dequantize_kernel<kQ6_K>, dim3(grid), dim3(kDenseThreads), 0, stream, w, quads, out); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int WT>
hipError_t launch_dense_typed(const void* w, std::uint64_t k, std::uint64_t n, const float* x, const float* bias,
                              float* y, std::uint32_t m, hipStream_t stream, const DenseTuning& tuning) {
    if (WT == kQ6_K && m == 1u && tuning.path != 2u) {
        const std::uint64_t tiles = ceil_div(n, 16u);
        if (tiles > 0x7fffffffu) return hipErrorInvalidValue;
        const Q6kGemvPlan g = plan_q6k_gemv(k, n, tuning.shape);
        const auto* wb = static_cast<const unsigned char*>(w);
        const dim3 grid(static_cast<unsigned>(tiles)), block(64u * g.waves);
        if (g.units == 2u) {
            if (g.depth == 2u) hipLaunchKernelGGL((q6k_gemv_kernel<2, 2>), grid, block, 0, stream, wb, x, bias, y, k, n);
            else hipLaunchKernelGGL((q6k_gemv_kernel<2, 1>), grid, block, 0, stream, wb, x, bias, y, k, n);
        } else {
            if (g.depth == 2u) hipLaunchKernelGGL((q6k_gemv_kernel<1, 2>), grid, block, 0, stream, wb, x, bias, y, k, n);
            else hipLaunchKernelGGL((q6k_gemv_kernel<1, 1>), grid, block, 0, stream, wb, x, bias, y, k, n);
        }
        return hipGetLastError();
    }
    if (m <= kDenseRowsKernelMax) {
        const dim3 grid(static_cast<unsigned>(ceil_div(n, kDenseCols)), static_cast<unsigned>(ceil_div(m, kDenseMaxRows)));
        if (m == 1u) {
            hipLaunchKernelGGL((dense_rows_kernel<1, WT>), grid, dim3(kDenseThreads), 0, stream, w, x, bias, y, m, k, n);
        } else if (m <= 4u) {
            hipLaunchKernelGGL((dense_rows_kernel<4, WT>), grid, dim3(kDenseThreads), 0, stream, w, x, bias, y, m, k, n);
        } else {
            hipLaunchKernelGGL((dense_rows_kernel<kDenseMaxRows, WT>), grid, dim3(kDenseThreads), 0, stream, w, x, bias,
                               y, m, k, n);
        }
    } else {
        const dim3 grid(static_cast<unsigned>(ceil_div(n, kGemmTile)), static_cast<unsigned>(ceil_div(m, kGemmTile)));
        hipLaunchKernelGGL(dense_gemm_kernel<WT>, grid, dim3(kDenseThreads), 0, stream, w, x, bias, y, m, k, n);
    }
    return hipGetLastError();
}

bool dense_mfma_route(int storage, std::uint64_t k, std::uint64_t n, std::uint32_t m, const DenseTuning& tuning) {
    (void)n;
    if (tuning.path == 2u || !dense_mfma_supported(storage, k)) return false;
    if (tuning.path == 1u) return true;
    // Measured on the Qwen2-7B shapes: the matrix cores win from two rows to
    // 64 (F16 down M = 16 120 -> 57 us, gate|up M = 32 514 -> 107; Q6_K down
    // M = 32 272 -> 129); a single row streams faster through the FMA GEMV
    // (F16 down 29 against 39 us, Q6_K 23 against 74), and at M = 512 the
    // launches per 64 rows re-read the weights (gate|up 1964 against 2284
    // us, Q6_K down 1589 against 2045).
    return m >= 2u && m <= 64u;
}

hipError_t launch_dense_linear(const void* w, int storage, std::uint64_t k, std::uint64_t n, const float* x,
                               const float* bias, float* y, std::uint32_t m, hipStream_t stream,
                               const DenseTuning& tuning) {
    if (m == 0u || k == 0u || n == 0u || k % kGemmK != 0u) return hipErrorInvalidValue;
    if (dense_mfma_route(storage, k, n, m, tuning)) {
        return launch_dense_mfma(w, storage, k, n, x, bias, y, m, tuning.shape, stream);
    }
    switch (storage) {
    case kF32: return launch_dense_typed<kF32>(w, k, n, x, bias, y, m, stream, tuning);
    case kF16: return launch_dense_typed<kF16>(w, k, n, x, bias, y, m, stream, tuning);
    case kBF16: return launch_dense_typed<kBF16>(w, k, n, x, bias, y, m, stream, tuning);
    case kQ6_K: return k % 256u == 0u ? launch_dense_typed<kQ6_K>(w, k, n, x, bias, y, m, stream, tuning) : hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dense_rows(const void* w, int storage, std::uint64_t k, std::uint64_t n, const std::int32_t* rows,
                             std::uint32_t count, float* out, hipStream_t stream) {
    if (count == 0u) return hipSuccess;
    const unsigned gx = static_cast<unsigned>(std::min<std::uint64_t>(ceil_div(k, kDenseThreads), 64u));
    const dim3 grid(gx, count);
    switch (storage) {
    case kF32:
        hipLaunchKernelGGL(dense_rows_gather_kernel<kF32>, grid, dim3(kDenseThreads), 0, stream, w, k, n, rows, count, out);
        break;
    case kF16:
        hipLaunchKernelGGL(dense_rows_gather_kernel<kF16>, grid, dim3(kDenseThreads), 0, stream, w, k, n, rows, count, out);
        break;
    case kBF16:
        hipLaunchKernelGGL(dense_rows_gather_kernel<kBF16>, grid, dim3(kDenseThreads), 0, stream, w, k, n, rows, count,
                           out);
        break;
    case kQ6_K:
        hipLaunchKernelGGL(dense_rows_gather_kernel<kQ6_K>, grid, dim3(kDenseThreads), 0, stream, w, k, n, rows, count,
                           out);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace air_hip

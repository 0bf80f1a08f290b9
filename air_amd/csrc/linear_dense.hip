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

// Q6_K super-block record: [ql:128][qh:64][scales:16 x int8]; block b's f16
// d is entry b of the plane that follows all `nblocks` records.
constexpr std::uint32_t kQ6kRecord = 208;

__device__ __forceinline__ const std::uint16_t* q6k_d_plane(const void* w, std::uint64_t nblocks) {
    return reinterpret_cast<const std::uint16_t*>(static_cast<const unsigned char*>(w) + nblocks * kQ6kRecord);
}

// Four consecutive weights w[idx .. idx + 3] (idx a multiple of 4) of a
// dense matrix stored as WT (f32, f16 / bf16 bits, or Q6_K records of a
// matrix of nblocks super-blocks), as exact f32.  Q6_K: a row is whole
// super-blocks (k a multiple of 256), so
// element idx lies in record idx / 256 at position e = idx % 256: half
// h = e / 128, quadrant j and offset i within it; its low nibble is nibble
// j >> 1 of ql[64 h + 32 (j & 1) + i], its high bits are bits 2j, 2j + 1 of
// qh[32 h + i], its scale is scales[8 h + i / 16 + 2 j]; four weights share
// the quadrant and the scale (src/reference/tensor_reader.cpp:197-242).
template <int WT>
__device__ __forceinline__ float4 load_w4(const void* __restrict__ w, std::uint64_t idx, std::uint64_t nblocks) {
    if constexpr (WT == kQ6_K) {
        const unsigned char* rec = static_cast<const unsigned char*>(w) + (idx >> 8) * kQ6kRecord;
        const std::uint32_t e = static_cast<std::uint32_t>(idx & 255u);
        const std::uint32_t h = e >> 7, j = (e >> 5) & 3u, i = e & 31u;
        const std::uint32_t ql = *reinterpret_cast<const std::uint32_t*>(rec + 64u * h + 32u * (j & 1u) + i);
        const std::uint32_t qh = *reinterpret_cast<const std::uint32_t*>(rec + 128u + 32u * h + i);
        const std::uint32_t scw = *reinterpret_cast<const std::uint32_t*>(rec + 192u + 8u * h + 4u * (j >> 1));
        const float d = f16_bits_to_f32(q6k_d_plane(w, nblocks)[idx >> 8]);
        // scales[8h + i/16 + 2j]: byte (i/16 + 2j) - 4 (j >> 1) of the word.
        const int sc = static_cast<int>(static_cast<std::int8_t>((scw >> (8u * ((i >> 4) + 2u * (j & 1u)))) & 0xffu));
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

// One row of x through Q6_K records (M = 1).  A lane takes one 16-weight
// group of a super-block -- group g = 8 h + 2 j + g1 holds elements
// 128 h + 32 j + 16 g1 .. + 15, its low nibbles in 16 bytes of ql (nibble
// j >> 1), its high bits in 16 bytes of qh (bits 2j, 2j + 1), one 6-bit
// sub-block scale -- for the workgroup's C consecutive output columns, so
// its 16 activations are loaded once per super-block and C columns.
// Sixteen lanes cover a super-block, a wave four, the workgroup's kWaves
// waves 4 kWaves per step.  Software-pipelined: a wave holds the loads of its
// next step (activations and every column's codes) in flight while it
// computes the current one.  Each weight is fma(d * sc, q, -32 * d * sc),
// which rounds once and so equals the reference's (d * sc) * (q - 32), then
// enters an f32 FMA with x; lane and wave partials meet in a fixed order.
template <unsigned C, unsigned kWaves>
__global__ __launch_bounds__(64 * kWaves) void q6k_gemv_pipe_kernel(const unsigned char* __restrict__ w,
                                                                    const float* __restrict__ x,
                                                                    const float* __restrict__ bias,
                                                                    float* __restrict__ y, std::uint64_t k,
                                                                    std::uint64_t n) {
    __shared__ float red[kWaves][C];
    const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const std::uint64_t sbs = k / 256u;
    const std::uint16_t* dplane = q6k_d_plane(w, sbs * n);
    const std::uint64_t c0 = static_cast<std::uint64_t>(blockIdx.x) * C;
    const std::uint32_t g = lane & 15u, h = g >> 3, j = (g >> 1) & 3u, g1 = g & 1u;
    const std::uint32_t e0 = 128u * h + 32u * j + 16u * g1;
    const std::uint32_t ql_off = 64u * h + 32u * (j & 1u) + 16u * g1;
    const std::uint32_t qh_off = 128u + 32u * h + 16u * g1;
    const std::uint32_t sc_off = 192u + 8u * h + 2u * j + g1;
    struct Step {
        float4 x[4];
        u32x4 ql[C], qh[C];
        std::uint32_t sc[C], d[C];
    };
    const auto load = [&](Step& st, std::uint64_t sb) __attribute__((always_inline)) {
        const float4* xp = reinterpret_cast<const float4*>(x + sb * 256u + e0);
#pragma unroll
        for (unsigned i = 0; i < 4; ++i) st.x[i] = xp[i];
#pragma unroll
        for (unsigned c = 0; c < C; ++c) {
            const std::uint64_t col = c0 + c < n ? c0 + c : n - 1u;   // clamped; not stored
            const std::uint64_t blk = col * sbs + sb;
            const unsigned char* rec = w + blk * kQ6kRecord;
            st.ql[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rec + ql_off));
            st.qh[c] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(rec + qh_off));
            st.sc[c] = rec[sc_off];
            st.d[c] = dplane[blk];
        }
    };
    float acc[C];
#pragma unroll
    for (unsigned c = 0; c < C; ++c) acc[c] = 0.0f;
    const auto compute = [&](const Step& st) __attribute__((always_inline)) {
        const float xv[16] = {st.x[0].x, st.x[0].y, st.x[0].z, st.x[0].w, st.x[1].x, st.x[1].y, st.x[1].z, st.x[1].w,
                              st.x[2].x, st.x[2].y, st.x[2].z, st.x[2].w, st.x[3].x, st.x[3].y, st.x[3].z, st.x[3].w};
#pragma unroll
        for (unsigned c = 0; c < C; ++c) {
            const float d = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<std::uint16_t>(st.d[c])));
            const float ds = d * static_cast<float>(static_cast<int>(static_cast<std::int8_t>(st.sc[c])));
            const float bias32 = -32.0f * ds;
#pragma unroll
            for (unsigned t = 0; t < 4; ++t) {
                const std::uint32_t lo = st.ql[c][t], hi = st.qh[c][t];
                const std::uint32_t nib = (j >> 1) ? (lo >> 4) & 0x0f0f0f0fu : lo & 0x0f0f0f0fu;
                const std::uint32_t q = nib | (((hi >> (2u * j)) & 0x03030303u) << 4);
#pragma unroll
                for (unsigned b = 0; b < 4; ++b) {
                    const float wq = fmaf(ds, static_cast<float>((q >> (8u * b)) & 0xffu), bias32);
                    acc[c] = fmaf(wq, xv[4u * t + b], acc[c]);
                }
            }
        }
    };
    const std::uint64_t stride = 4u * kWaves;
    std::uint64_t sb = 4u * wave + (lane >> 4);
    // Lanes past the last super-block stay in the loop (uniform trip count
    // per wave is not needed: each lane's loads are its own) but load nothing.
    Step a, b;
    if (sb < sbs) load(a, sb);
    while (sb < sbs) {
        const std::uint64_t next = sb + stride;
        if (next < sbs) load(b, next);
        compute(a);
        if (next >= sbs) break;
        const std::uint64_t after = next + stride;
        if (after < sbs) load(a, after);
        compute(b);
        sb = after;
    }
#pragma unroll
    for (unsigned c = 0; c < C; ++c) {
        float v = acc[c];
        for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
        if (lane == 0u) red[wave][c] = v;
    }
    __syncthreads();
    if (threadIdx.x < C && c0 + threadIdx.x < n) {
        float v = red[0][threadIdx.x];
#pragma unroll
        for (unsigned q = 1; q < kWaves; ++q) v += red[q][threadIdx.x];
        y[c0 + threadIdx.x] = bias ? v + bias[c0 + threadIdx.x] : v;
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

// Canonical Q6_K blocks (210 bytes: [ql][qh][scales][d]) -> 208-byte
// records and the d plane after them; thread t writes output word t of the
// records, or one d entry.
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
            const unsigned char* bytes = src + b * 210u + 4u * word;
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

// Launch shape of the Q6_K GEMV (a sweep may set it; zeros = the measured
// default).
static Q6kGemvShape g_q6k_shape{};
void set_q6k_gemv_shape(const Q6kGemvShape& shape) { g_q6k_shape = shape; }
Q6kGemvShape q6k_gemv_shape(std::uint64_t k, std::uint64_t n) {
    if (g_q6k_shape.columns != 0u) return g_q6k_shape;
    (void)n;
    // Measured on the Qwen2-7B shapes (graphs of distinct matrices, so no
    // matrix is served from the Infinity Cache): long K (down, 74
    // super-blocks per row) 4 columns per workgroup, 21.9 us (2.5 TB/s of its
    // own bytes; without the pipeline 26.5 us at its best shape, f32 rows
    // 42 us); short K (o, lm_head: one step per wave) 2 columns, 6.9 and
    // 167 us.  Eight columns, or more waves splitting K, were slower.
    return k >= 8192u ? Q6kGemvShape{4u, 4u} : Q6kGemvShape{2u, 4u};
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
                              float* y, std::uint32_t m, hipStream_t stream) {
    if (WT == kQ6_K && m == 1u) {
        const auto* wb = static_cast<const unsigned char*>(w);
        const Q6kGemvShape shape = q6k_gemv_shape(k, n);
        const dim3 grid(static_cast<unsigned>(ceil_div(n, shape.columns)));
#define AIR_Q6K_GEMV(C, W)                                                                                          \
        if (shape.columns == C && shape.waves == W) {                                                               \
            hipLaunchKernelGGL((q6k_gemv_pipe_kernel<C, W>), grid, dim3(64 * W), 0, stream, wb, x, bias, y, k, n);  \
            return hipGetLastError();                                                                               \
        }
        AIR_Q6K_GEMV(2, 4) AIR_Q6K_GEMV(4, 4)
#undef AIR_Q6K_GEMV
        return hipErrorInvalidConfiguration;
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
    case kF32: return launch_dense_typed<kF32>(w, k, n, x, bias, y, m, stream);
    case kF16: return launch_dense_typed<kF16>(w, k, n, x, bias, y, m, stream);
    case kBF16: return launch_dense_typed<kBF16>(w, k, n, x, bias, y, m, stream);
    case kQ6_K: return k % 256u == 0u ? launch_dense_typed<kQ6_K>(w, k, n, x, bias, y, m, stream) : hipErrorInvalidValue;
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

// linear_dense.hip -- linears over matrices held as dense f32 rows.
//
// The encodings with no resident tile format here (F32, F16, BF16 and Q6_K;
// decode_element, src/cuda/cuda_backend.cu:241-344, decodes them per
// element inside every GEMV) are held as dense rows w[n][k]: F32, F16 and
// BF16 as their own GGUF rows (converted exactly to f32 as they are loaded),
// Q6_K decoded once at prepare time, bit for bit, into f32 rows.  A real Qwen2.5 Q4_K_M file carries Q6_K tensors
// (lm_head, half the ffn_down / attn_v) and F16 / BF16 files carry every
// linear this way.  These kernels are the coverage route for them: plain f32
// FMA with f32 accumulation, weights read at 4 (F32, Q6_K) or 2 (F16, BF16)
// bytes per element, one launch per linear, no workspace.
//   rows 1..64: dense_rows_kernel, four output columns per workgroup for up
//               to 16 rows of x (K split over its four waves); the weights
//               are read once per 16 rows (M = 1 at 7B shapes: 5-6 TB/s of
//               f32 weights);
//   more rows:  dense_gemm_kernel, 64 x 64 output tiles staged through LDS
//               (45 TFLOP/s at 512 rows).
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

// Four consecutive weights w[idx .. idx + 3] (idx a multiple of 4) of a
// dense matrix stored as WT (f32, or f16 / bf16 bits), as exact f32.
template <int WT>
__device__ __forceinline__ float4 load_w4(const void* __restrict__ w, std::uint64_t idx) {
    if constexpr (WT == kF32) {
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
        for (unsigned c = 0; c < kDenseCols; ++c) wv[c] = load_w4<WT>(w, wr[c] + kk);
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
            if (n0 + row < n) wv = load_w4<WT>(w, (n0 + row) * k + k0 + kq);
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
        if constexpr (WT == kF32) {
            dst[c] = static_cast<const float*>(w)[base + c];
        } else if constexpr (WT == kF16) {
            dst[c] = f16_bits_to_f32(static_cast<const std::uint16_t*>(w)[base + c]);
        } else {
            dst[c] = __uint_as_float(static_cast<std::uint32_t>(static_cast<const std::uint16_t*>(w)[base + c]) << 16);
        }
    }
}

} // namespace

template <int WT>
hipError_t launch_dense_typed(const void* w, std::uint64_t k, std::uint64_t n, const float* x, const float* bias,
                              float* y, std::uint32_t m, hipStream_t stream) {
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

hipError_t launch_dense_linear(const void* w, int storage, std::uint64_t k, std::uint64_t n, const float* x,
                               const float* bias, float* y, std::uint32_t m, hipStream_t stream) {
    if (m == 0u || k == 0u || n == 0u || k % kGemmK != 0u) return hipErrorInvalidValue;
    switch (storage) {
    case kF32: return launch_dense_typed<kF32>(w, k, n, x, bias, y, m, stream);
    case kF16: return launch_dense_typed<kF16>(w, k, n, x, bias, y, m, stream);
    case kBF16: return launch_dense_typed<kBF16>(w, k, n, x, bias, y, m, stream);
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
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace air_hip

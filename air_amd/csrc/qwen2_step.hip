// qwen2_step.hip -- the Qwen2 step around the linears: embedding rows,
// RMSNorm, RoPE, paged KV append, attention, SiLU * up, residual add, greedy
// argmax.
//
// Each kernel follows the reference executor's arithmetic (src/reference/
// reference_executor.cpp:17-138, 325-428) operation by operation where that
// is cheap on the GPU, so a HIP step differs from the reference only through
// the linears (relative error ~1e-6):
//   * RMSNorm: double sum of squares, scale = float(1 / sqrt(mean + eps)),
//     out = (x * scale) * w in float;
//   * RoPE: cos / sin come from a host table built with the reference's
//     double formulas; the rotation is two float products and one float
//     add / subtract, never fused;
//   * attention: double scores (sequential dot over the head dimension),
//     double softmax with the denominator summed in token order, float
//     probabilities, float accumulation of p * v in token order, never fused;
//   * greedy: the first maximum (std::max_element, src/runtime/sampling.cpp:13-16).
//
// The KV cache is paged: a page holds `page_tokens` tokens of every layer's K
// and V ([layer][2][page_tokens][kv_width] f32); a row's sequence is named by
// its page table (int32 page indices).
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"
#include "air_hip_kv.hpp"

namespace air_hip {
namespace {

constexpr unsigned kThreads = 256;

// ---- embedding rows --------------------------------------------------------

// out[i][k] = W[rows[i]][k] decoded bit-exactly from the resident tiles.
__global__ __launch_bounds__(kThreads) void matrix_rows_kernel(int type, const void* codes_, const void* scales_,
                                                               std::uint64_t K, std::uint64_t N, std::uint32_t KT,
                                                               const std::int32_t* __restrict__ rows,
                                                               std::uint32_t m, float* __restrict__ out) {
#pragma clang fp contract(off)
    const std::uint32_t i = blockIdx.y;
    if (i >= m) return;
    const std::int32_t row = rows[i];
    if (row < 0 || static_cast<std::uint64_t>(row) >= N) return;
    const std::uint32_t rt = static_cast<std::uint32_t>(row) >> 4, r = static_cast<std::uint32_t>(row) & 15u;
    float* dst = out + static_cast<std::uint64_t>(i) * K;
    for (std::uint64_t k = blockIdx.x * static_cast<std::uint64_t>(kThreads) + threadIdx.x; k < K;
         k += static_cast<std::uint64_t>(gridDim.x) * kThreads) {
        float value = 0.0f;
        if (type == kQ8_0) {
            const std::uint32_t kt = static_cast<std::uint32_t>(k / 64u), kk = static_cast<std::uint32_t>(k % 64u);
            const std::uint32_t hb = kk / 32u, within = kk % 32u, g = within / 8u, e = within % 8u;
            const std::uint64_t tile = static_cast<std::uint64_t>(rt) * KT + kt;
            const std::uint8_t* rec = static_cast<const std::uint8_t*>(codes_) + (tile * 64u + 16u * g + r) * 16u;
            const int q = static_cast<int>(rec[8u * hb + e]) - 128;
            const std::uint32_t sc = static_cast<const std::uint32_t*>(scales_)[tile * 16u + r];
            value = f16_bits_to_f32((sc >> (16u * hb)) & 0xffffu) * static_cast<float>(q);
        } else if (type == kQ4_0) {
            const std::uint32_t kt = static_cast<std::uint32_t>(k / 128u), kk = static_cast<std::uint32_t>(k % 128u);
            const std::uint32_t j = kk / 32u, within = kk % 32u, g = within / 8u, e = within % 8u;
            const std::uint64_t tile = static_cast<std::uint64_t>(rt) * KT + kt;
            const std::uint32_t w = static_cast<const std::uint32_t*>(codes_)[(tile * 64u + 16u * g + r) * 4u + j];
            const int q = static_cast<int>((w >> kNibblePos[e]) & 0x0fu) - 8;
            const std::uint32_t sw = static_cast<const std::uint32_t*>(scales_)[(tile * 16u + r) * 2u + j / 2u];
            value = f16_bits_to_f32((sw >> (16u * (j & 1u))) & 0xffffu) * static_cast<float>(q);
        } else {
            const std::uint32_t kt = static_cast<std::uint32_t>(k / 256u), kk = static_cast<std::uint32_t>(k % 256u);
            const std::uint32_t j = kk / 32u, within = kk % 32u, g = within / 8u, e = within % 8u;
            const std::uint64_t tile = static_cast<std::uint64_t>(rt) * KT + kt;
            const std::uint32_t w = static_cast<const std::uint32_t*>(
                codes_)[(((tile * 2u + j / 4u) * 64u) + 16u * g + r) * 4u + (j & 3u)];
            const std::uint32_t n = (w >> kNibblePos[e]) & 0x0fu;
            const std::uint32_t* hd = static_cast<const std::uint32_t*>(scales_) + (tile * 16u + r) * 4u;
            const std::uint32_t packed[3] = {hd[1], hd[2], hd[3]};
            std::uint32_t s6 = 0, m6 = 0;
            q4k_scale_min(packed, j, s6, m6);
            const float d = f16_bits_to_f32(hd[0] & 0xffffu);
            const float dmin = f16_bits_to_f32(hd[0] >> 16);
            value = (d * static_cast<float>(s6)) * static_cast<float>(n) - dmin * static_cast<float>(m6);
        }
        dst[k] = value;
    }
}

// ---- RMSNorm ---------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const float* x, const float* __restrict__ w,
                                                            float* out, std::uint64_t n, double eps) {
#pragma clang fp contract(off)
    __shared__ double red[kThreads / 64];
    const float* row = x + static_cast<std::uint64_t>(blockIdx.x) * n;
    float* dst = out + static_cast<std::uint64_t>(blockIdx.x) * n;
    double sum = 0.0;
    for (std::uint64_t i = threadIdx.x; i < n; i += kThreads) sum += static_cast<double>(row[i]) * row[i];
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = sum;
    __syncthreads();
    const double total = (red[0] + red[1]) + (red[2] + red[3]);
    const double mean = total / static_cast<double>(n);
    const float scale = static_cast<float>(1.0 / sqrt(mean + eps));
    for (std::uint64_t i = threadIdx.x; i < n; i += kThreads) dst[i] = row[i] * scale * w[i];
}

// ---- RoPE ------------------------------------------------------------------

// One thread per (row, head, pair); q heads then k heads of each fused row.
__global__ __launch_bounds__(kThreads) void rope_kernel(float* __restrict__ qkv, std::uint64_t stride, std::uint32_t m,
                                                        const std::int32_t* __restrict__ positions,
                                                        std::uint32_t q_heads, std::uint32_t kv_heads,
                                                        std::uint32_t head_dim, std::uint32_t rope_dims,
                                                        const float2* __restrict__ table,
                                                        std::uint64_t table_positions) {
#pragma clang fp contract(off)
    const std::uint32_t half = rope_dims / 2u;
    const std::uint32_t heads = q_heads + kv_heads;
    const std::uint64_t total = static_cast<std::uint64_t>(m) * heads * half;
    for (std::uint64_t idx = blockIdx.x * static_cast<std::uint64_t>(kThreads) + threadIdx.x; idx < total;
         idx += static_cast<std::uint64_t>(gridDim.x) * kThreads) {
        const std::uint32_t i = static_cast<std::uint32_t>(idx % half);
        const std::uint32_t h = static_cast<std::uint32_t>((idx / half) % heads);
        const std::uint32_t r = static_cast<std::uint32_t>(idx / (static_cast<std::uint64_t>(half) * heads));
        const std::int32_t pos = positions[r];
        if (pos < 0 || static_cast<std::uint64_t>(pos) >= table_positions) continue;
        float* base = qkv + static_cast<std::uint64_t>(r) * stride + static_cast<std::uint64_t>(h) * head_dim;
        const float2 cs = table[static_cast<std::uint64_t>(pos) * half + i];
        const float first = base[i];
        const float second = base[i + half];
        const float a = first * cs.x;
        const float b = second * cs.y;
        const float c = first * cs.y;
        const float d = second * cs.x;
        base[i] = a - b;
        base[i + half] = c + d;
    }
}

// ---- paged KV ----------------------------------------------------------------

// Copies each row's k and v (after RoPE) from its fused q|k|v output into its page slot.
__global__ __launch_bounds__(kThreads) void kv_append_kernel(KvGeometry g, const float* __restrict__ qkv,
                                                             std::uint64_t stride, std::uint64_t q_width,
                                                             std::uint32_t m, const std::int32_t* __restrict__ positions,
                                                             const std::int32_t* __restrict__ tables,
                                                             std::uint32_t layer) {
    const std::uint32_t r = blockIdx.y;
    if (r >= m) return;
    const std::int32_t* table = tables + static_cast<std::uint64_t>(r) * g.max_pages;
    const std::uint64_t pos = static_cast<std::uint64_t>(positions[r]);
    float* k = kv_slot(g, table, layer, pos, false);
    float* v = kv_slot(g, table, layer, pos, true);
    if (!k || !v) return;
    const float* src = qkv + static_cast<std::uint64_t>(r) * stride + q_width;
    for (std::uint32_t i = blockIdx.x * kThreads + threadIdx.x; i < g.kv_width; i += gridDim.x * kThreads) {
        k[i] = src[i];
        v[i] = src[g.kv_width + i];
    }
}

// RoPE of the q and k heads and the KV append in one pass (one workgroup
// column per row): the same arithmetic as rope_kernel followed by
// kv_append_kernel.  A row whose position lies outside the table is not
// rotated; a row without a valid page slot is rotated but not stored.
// Where rope_kv_append_kernel reads q|k|v: the row itself, or (SPLIT) the
// sum of a K-split linear's partials ([splits][m][stride], split_stride =
// m * stride floats apart) from zero in split order, plus bias -- the split
// reduction's arithmetic, so the result is bit-identical to reducing first.
struct QkvSplit {
    const float* partials;
    std::uint32_t splits;
    std::uint64_t split_stride;
    const float* bias;
};

__device__ __forceinline__ float split_sum1(const float* __restrict__ p, std::uint32_t splits, std::uint64_t stride) {
    float t = 0.0f;
    for (std::uint32_t s = 0; s < splits; s += 8u) {
        float q[8];
#pragma unroll
        for (std::uint32_t e = 0; e < 8u; ++e) q[e] = p[(s + e < splits ? s + e : splits - 1u) * stride];
#pragma unroll
        for (std::uint32_t e = 0; e < 8u; ++e) {
            if (s + e < splits) t += q[e];
        }
    }
    return t;
}

template <bool SPLIT>
__global__ __launch_bounds__(kThreads) void rope_kv_append_kernel(
    KvGeometry g, float* __restrict__ qkv, std::uint64_t stride, std::uint64_t q_width, std::uint32_t m,
    const std::int32_t* __restrict__ positions, const std::int32_t* __restrict__ tables, std::uint32_t layer,
    std::uint32_t q_heads, std::uint32_t kv_heads, std::uint32_t head_dim, std::uint32_t rope_dims,
    const float2* __restrict__ table, std::uint64_t table_positions, QkvSplit src) {
#pragma clang fp contract(off)
    const std::uint32_t r = blockIdx.y;
    if (r >= m) return;
    const std::int32_t pos = positions[r];
    const bool rotate = pos >= 0 && static_cast<std::uint64_t>(pos) < table_positions;
    const std::int32_t* ptable = tables + static_cast<std::uint64_t>(r) * g.max_pages;
    float* kd = kv_slot(g, ptable, layer, static_cast<std::uint64_t>(pos), false);
    float* vd = kv_slot(g, ptable, layer, static_cast<std::uint64_t>(pos), true);
    if (!vd) kd = nullptr;  // both or neither, as the separate append
    float* row = qkv + static_cast<std::uint64_t>(r) * stride;
    const float* prow = SPLIT ? src.partials + static_cast<std::uint64_t>(r) * stride : nullptr;
    // Value of column c of the row's q|k|v.  SPLIT writes every column back
    // to the row (the plain reduction's output), rotated where RoPE applies.
    const auto load = [&](std::uint64_t c) __attribute__((always_inline)) -> float {
        if constexpr (SPLIT) {
            float t = split_sum1(prow + c, src.splits, src.split_stride);
            if (src.bias) t += src.bias[c];
            return t;
        } else {
            return row[c];
        }
    };
    const std::uint32_t half = rope_dims / 2u;
    const std::uint32_t tail = head_dim - rope_dims;             // dims past the rotary part
    const std::uint64_t q_items = static_cast<std::uint64_t>(q_heads) * half;
    const std::uint64_t k_items = static_cast<std::uint64_t>(kv_heads) * (half + tail);
    const std::uint64_t q_tails = SPLIT ? static_cast<std::uint64_t>(q_heads) * tail : 0u;
    const std::uint64_t total = q_items + k_items + q_tails + g.kv_width;  // + the v row
    for (std::uint64_t idx = blockIdx.x * static_cast<std::uint64_t>(kThreads) + threadIdx.x; idx < total;
         idx += static_cast<std::uint64_t>(gridDim.x) * kThreads) {
        if (idx < q_items + k_items) {
            std::uint64_t base;                                    // first column of the head
            std::uint32_t i;
            float* dst = nullptr;                                  // the k head in the pool
            if (idx < q_items) {
                base = (idx / half) * head_dim;
                i = static_cast<std::uint32_t>(idx % half);
            } else {
                const std::uint64_t e = idx - q_items;
                const std::uint32_t h = static_cast<std::uint32_t>(e / (half + tail));
                const std::uint32_t j = static_cast<std::uint32_t>(e % (half + tail));
                base = q_width + static_cast<std::uint64_t>(h) * head_dim;
                if (kd) dst = kd + static_cast<std::uint64_t>(h) * head_dim;
                if (j >= half) {                                  // unrotated tail dim
                    const std::uint32_t t = rope_dims + (j - half);
                    const float v = load(base + t);
                    if (SPLIT) row[base + t] = v;
                    if (dst) dst[t] = v;
                    continue;
                }
                i = j;
            }
            const float first = load(base + i);
            const float second = load(base + i + half);
            float lo = first, hi = second;
            if (rotate) {
                const float2 cs = table[static_cast<std::uint64_t>(pos) * half + i];
                const float a = first * cs.x;
                const float b = second * cs.y;
                const float c = first * cs.y;
                const float d = second * cs.x;
                lo = a - b;
                hi = c + d;
            }
            if (rotate || SPLIT) {
                row[base + i] = lo;
                row[base + i + half] = hi;
            }
            if (dst) {
                dst[i] = lo;
                dst[i + half] = hi;
            }
        } else if (idx < q_items + k_items + q_tails) {           // SPLIT: q tail dims
            const std::uint64_t e = idx - q_items - k_items;
            const std::uint64_t c = (e / tail) * head_dim + rope_dims + e % tail;
            row[c] = load(c);
        } else {
            const std::uint64_t i = idx - q_items - k_items - q_tails;
            const std::uint64_t c = q_width + g.kv_width + i;
            if (SPLIT) {
                const float v = load(c);
                row[c] = v;
                if (vd) vd[i] = v;
            } else if (vd) {
                vd[i] = row[c];
            }
        }
    }
}

// One workgroup per (row, q head): attention over tokens 0..positions[row] of
// the row's sequence, in the reference's arithmetic (see file comment).
// scratch: [m * q_heads][score_stride] doubles.
__global__ __launch_bounds__(kThreads) void attention_kernel(KvGeometry g, const float* __restrict__ qkv,
                                                             std::uint64_t stride, std::uint32_t m,
                                                             const std::int32_t* __restrict__ positions,
                                                             const std::int32_t* __restrict__ tables,
                                                             std::uint32_t layer, std::uint32_t q_heads,
                                                             std::uint32_t kv_heads, std::uint32_t head_dim,
                                                             double* __restrict__ scratch, std::uint64_t score_stride,
                                                             float* __restrict__ out) {
#pragma clang fp contract(off)
    __shared__ float qs[512];
    __shared__ double red[kThreads / 64];
    __shared__ double denom_shared;
    const std::uint32_t r = blockIdx.x / q_heads;
    const std::uint32_t qh = blockIdx.x % q_heads;
    if (r >= m) return;
    const std::uint32_t kvh = static_cast<std::uint32_t>((static_cast<std::uint64_t>(qh) * kv_heads) / q_heads);
    const std::int32_t* table = tables + static_cast<std::uint64_t>(r) * g.max_pages;
    std::uint64_t total = static_cast<std::uint64_t>(positions[r] < 0 ? 0 : positions[r]) + 1u;
    if (total > score_stride) total = score_stride;
    const float* q = qkv + static_cast<std::uint64_t>(r) * stride + static_cast<std::uint64_t>(qh) * head_dim;
    for (std::uint32_t d = threadIdx.x; d < head_dim; d += kThreads) qs[d] = q[d];
    __syncthreads();
    double* scores = scratch + static_cast<std::uint64_t>(blockIdx.x) * score_stride;
    const double scale = 1.0 / sqrt(static_cast<double>(head_dim));
    double local_max = -__builtin_huge_val();
    for (std::uint64_t t = threadIdx.x; t < total; t += kThreads) {
        const float* slot = kv_slot(g, table, layer, t, false);
        double s = 0.0;
        if (slot) {
            const float* key = slot + static_cast<std::uint64_t>(kvh) * head_dim;
            for (std::uint32_t d = 0; d < head_dim; ++d) s += static_cast<double>(qs[d]) * static_cast<double>(key[d]);
        }
        s *= scale;
        scores[t] = s;
        local_max = s > local_max ? s : local_max;
    }
    for (int off = 32; off > 0; off >>= 1) {
        const double o = __shfl_xor(local_max, off);
        local_max = o > local_max ? o : local_max;
    }
    if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = local_max;
    __syncthreads();
    double maximum = red[0];
    for (unsigned w = 1; w < kThreads / 64; ++w) maximum = red[w] > maximum ? red[w] : maximum;
    for (std::uint64_t t = threadIdx.x; t < total; t += kThreads) scores[t] = exp(scores[t] - maximum);
    __syncthreads();
    if (threadIdx.x == 0) {
        double denominator = 0.0;
        for (std::uint64_t t = 0; t < total; ++t) denominator += scores[t];
        denom_shared = denominator;
    }
    __syncthreads();
    const double denominator = denom_shared;
    float* dst = out + static_cast<std::uint64_t>(r) * q_heads * head_dim + static_cast<std::uint64_t>(qh) * head_dim;
    for (std::uint32_t d = threadIdx.x; d < head_dim; d += kThreads) {
        float acc = 0.0f;
        for (std::uint64_t t = 0; t < total; ++t) {
            const float p = static_cast<float>(scores[t] / denominator);
            const float* slot = kv_slot(g, table, layer, t, true);
            const float pv = slot ? p * slot[static_cast<std::uint64_t>(kvh) * head_dim + d] : 0.0f;
            acc = acc + pv;
        }
        dst[d] = acc;
    }
}

// ---- elementwise -------------------------------------------------------------

// out[r][i] = silu(gate[r][i]) * up[r][i] over fused gate|up rows.
__global__ __launch_bounds__(kThreads) void silu_mul_kernel(const float* __restrict__ gate_up, float* __restrict__ out,
                                                            std::uint32_t m, std::uint64_t ffn) {
#pragma clang fp contract(off)
    const std::uint64_t total = static_cast<std::uint64_t>(m) * ffn;
    for (std::uint64_t idx = blockIdx.x * static_cast<std::uint64_t>(kThreads) + threadIdx.x; idx < total;
         idx += static_cast<std::uint64_t>(gridDim.x) * kThreads) {
        const std::uint64_t r = idx / ffn, i = idx % ffn;
        const float g = gate_up[r * 2u * ffn + i];
        const float u = gate_up[r * 2u * ffn + ffn + i];
        const float s = g / (1.0f + expf(-g));
        out[idx] = s * u;
    }
}

__global__ __launch_bounds__(kThreads) void add_kernel(float* __restrict__ x, const float* __restrict__ y,
                                                       std::uint64_t count) {
    for (std::uint64_t i = blockIdx.x * static_cast<std::uint64_t>(kThreads) + threadIdx.x; i < count;
         i += static_cast<std::uint64_t>(gridDim.x) * kThreads) {
        x[i] = x[i] + y[i];
    }
}

// First maximum of each row (std::max_element with operator<): the largest
// value, the lowest index among equal values.  A row holding any non-finite
// value (NaN or +-inf) gives -1 instead of an index: the reference CUDA
// executor flags such a value and fails the step
// (src/cuda/cuda_backend.cu:613-624, 2368).
constexpr unsigned kArgmaxThreads = 256;
constexpr unsigned kArgmaxSlice = 4096;   // logits per workgroup of the first pass

// Merges a candidate (value, index) into the running best.
__device__ __forceinline__ void argmax_merge(float v, std::uint32_t i, float& bv, std::uint32_t& bi) {
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

// One logit: a non-finite value is never selected and marks the row.
__device__ __forceinline__ void argmax_take(float v, std::uint32_t i, float& bv, std::uint32_t& bi, bool& bad) {
    if (!__builtin_isfinite(v)) {
        bad = true;
        return;
    }
    argmax_merge(v, i, bv, bi);
}

// The selection rule does not depend on the visiting order, so a row is cut
// into slices of kArgmaxSlice logits, each reduced by its own workgroup to
// (best value, its index, any non-finite) -- partial (row, slice) -- and a
// second pass merges a row's slices.
struct ArgmaxPartial {
    float value;
    std::uint32_t index;
    std::uint32_t bad;
    std::uint32_t pad;
};

__global__ __launch_bounds__(kArgmaxThreads) void argmax_slice_kernel(const float* __restrict__ logits,
                                                                      std::uint64_t n, std::uint32_t slices,
                                                                      ArgmaxPartial* __restrict__ partials) {
    __shared__ float wave_v[kArgmaxThreads / 64];
    __shared__ std::uint32_t wave_i[kArgmaxThreads / 64];
    __shared__ std::uint32_t wave_bad[kArgmaxThreads / 64];
    const std::uint32_t slice = blockIdx.x, r = blockIdx.y;
    const float* row = logits + static_cast<std::uint64_t>(r) * n;
    const std::uint64_t begin = static_cast<std::uint64_t>(slice) * kArgmaxSlice;
    const std::uint64_t end = begin + kArgmaxSlice < n ? begin + kArgmaxSlice : n;
    float bv = -__builtin_huge_valf();
    std::uint32_t bi = 0xffffffffu;
    bool bad = false;
    const bool vec = (n % 4u == 0) && (reinterpret_cast<std::uintptr_t>(row) % 16u == 0);
    if (vec) {
        // Four float4 per thread, all loads issued before the first compare.
        constexpr unsigned kPer = kArgmaxSlice / 4u / kArgmaxThreads;
        float4 v[kPer];
#pragma unroll
        for (unsigned j = 0; j < kPer; ++j) {
            const std::uint64_t e = begin + 4u * (threadIdx.x + j * kArgmaxThreads);
            v[j] = e < end ? *reinterpret_cast<const float4*>(row + e)
                           : make_float4(-__builtin_huge_valf(), -__builtin_huge_valf(), -__builtin_huge_valf(),
                                         -__builtin_huge_valf());
        }
#pragma unroll
        for (unsigned j = 0; j < kPer; ++j) {
            const std::uint64_t e = begin + 4u * (threadIdx.x + j * kArgmaxThreads);
            if (e >= end) continue;
            const std::uint32_t base = static_cast<std::uint32_t>(e);
            argmax_take(v[j].x, base, bv, bi, bad);
            argmax_take(v[j].y, base + 1u, bv, bi, bad);
            argmax_take(v[j].z, base + 2u, bv, bi, bad);
            argmax_take(v[j].w, base + 3u, bv, bi, bad);
        }
    } else {
        for (std::uint64_t i = begin + threadIdx.x; i < end; i += kArgmaxThreads) {
            argmax_take(row[i], static_cast<std::uint32_t>(i), bv, bi, bad);
        }
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const std::uint32_t oi = __shfl_xor(bi, off);
        argmax_merge(ov, oi, bv, bi);
    }
    const bool wave_has_bad = __any(bad ? 1 : 0) != 0;
    if ((threadIdx.x & 63u) == 0) {
        wave_v[threadIdx.x >> 6] = bv;
        wave_i[threadIdx.x >> 6] = bi;
        wave_bad[threadIdx.x >> 6] = wave_has_bad ? 1u : 0u;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        bv = wave_v[0];
        bi = wave_i[0];
        std::uint32_t any_bad = wave_bad[0];
        for (unsigned w = 1; w < kArgmaxThreads / 64; ++w) {
            argmax_merge(wave_v[w], wave_i[w], bv, bi);
            any_bad |= wave_bad[w];
        }
        partials[static_cast<std::uint64_t>(r) * slices + slice] = ArgmaxPartial{bv, bi, any_bad, 0u};
    }
}

// One wave per row merges its slices' partials.  n >= 1 finite values always
// select an index; an empty selection means every value was non-finite,
// which the flag already records.
__global__ __launch_bounds__(64) void argmax_rows_kernel(const ArgmaxPartial* __restrict__ partials,
                                                         std::uint32_t slices, std::int32_t* __restrict__ out) {
    const std::uint32_t r = blockIdx.x;
    float bv = -__builtin_huge_valf();
    std::uint32_t bi = 0xffffffffu;
    bool bad = false;
    for (std::uint32_t s = threadIdx.x; s < slices; s += 64u) {
        const ArgmaxPartial p = partials[static_cast<std::uint64_t>(r) * slices + s];
        bad = bad || p.bad != 0u;
        argmax_merge(p.value, p.index, bv, bi);
    }
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const std::uint32_t oi = __shfl_xor(bi, off);
        argmax_merge(ov, oi, bv, bi);
    }
    const bool any_bad = __any(bad ? 1 : 0) != 0;
    if (threadIdx.x == 0) out[r] = any_bad ? -1 : static_cast<std::int32_t>(bi);
}

// RMSNorm of rows of n <= 8 * kNormThreads floats (n % 8 == 0), thread t
// holding elements 8t..8t+7 in registers (one coalesced read of the row),
// with the residual add of the reference's add_in_place fused in front when
// `y` is given: x += y, then out = x * float(1 / sqrt(mean(x^2) + eps)) * w.
// Without y, x and out may alias; with y they must not (x receives the sum).
//
// SPLIT: y holds `splits` partial outputs of a K-split linear
// (y[s][row][n], split_stride = m * n floats apart) and the value added is
// their sum from zero in split order plus bias -- the split reduction's
// arithmetic, so the result is bit-identical to reducing first.  The
// partials are loaded eight splits at a time so their latencies overlap.
// w == null stops after the add (no norm, out unused).
//
// LOAD: out is also split for the skinny kernel as split_rows_kernel splits
// a row (one power-of-two scale per row from max|out|, runs of eight through
// emit_split_run), so the next linear needs no split launch; the grid then
// covers the padded rows (zeros), as split_rows_kernel's does.
constexpr unsigned kNormThreads = 1024;

struct NormLoad {
    uint4* xs;
    float* block_sums;
    float* inv_scale;
    std::uint32_t rows;   // live rows; rows rows..mp-1 are padding
    std::uint32_t mp;     // 16 * ceil(rows / 16)
    std::uint32_t nb;     // 32-blocks per split row (kp / 32)
};

__device__ __forceinline__ float4v split_sum4(const float* __restrict__ p, std::uint32_t splits,
                                             std::uint64_t stride) {
    float4v t = {0.0f, 0.0f, 0.0f, 0.0f};
    for (std::uint32_t s = 0; s < splits; s += 8u) {
        float4v q[8];
#pragma unroll
        for (std::uint32_t e = 0; e < 8u; ++e) {
            const std::uint32_t src = s + e < splits ? s + e : splits - 1u;  // in bounds; unused past the end
            q[e] = *reinterpret_cast<const float4v*>(p + src * stride);
        }
#pragma unroll
        for (std::uint32_t e = 0; e < 8u; ++e) {
            if (s + e < splits) t += q[e];
        }
    }
    return t;
}

// PF: out is also converted for the next prefill linear on it, as
// prefill_activations_kernel converts a row (f16 of out * s, s the power of
// two that puts the row's max |out| in [2^14, 2^15), zero past n up to ldx;
// row_inv = 1 / s); the grid covers the padded rows (zeros, row_inv 1).
struct PrefillRows {
    _Float16* xh;
    float* row_inv;
    std::uint32_t rows;   // live rows; rows rows..mp-1 are padding
    std::uint64_t ldx;    // f16 row stride (>= n, a multiple of 8)
};

template <bool SPLIT, bool LOAD, bool PF = false>
__global__ __launch_bounds__(kNormThreads) void rms_norm_vec_kernel(float* x, const float* __restrict__ y,
                                                                    const float* __restrict__ w, float* out,
                                                                    std::uint64_t n, double eps, std::uint32_t splits,
                                                                    std::uint64_t split_stride,
                                                                    const float* __restrict__ bias, NormLoad ld,
                                                                    PrefillRows pf = PrefillRows{}) {
#pragma clang fp contract(off)
    __shared__ double red[kNormThreads / 64];
    __shared__ float redf[kNormThreads / 64];
    const std::uint32_t r = blockIdx.x;
    const std::uint32_t t = threadIdx.x;
    const bool mine = (!LOAD || r < ld.rows) && (!PF || r < pf.rows) && t < n / 8u;
    const std::uint64_t at = static_cast<std::uint64_t>(r) * n + 8u * t;
    float4v v[2], g[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        v[h] = float4v{0.0f, 0.0f, 0.0f, 0.0f};
        g[h] = v[h];
    }
    if (mine) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            v[h] = *reinterpret_cast<const float4v*>(x + at + 4 * h);
            if (w) g[h] = *reinterpret_cast<const float4v*>(w + 8u * t + 4 * h);
        }
        if (y) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float4v b;
                if constexpr (SPLIT) {
                    b = split_sum4(y + at + 4 * h, splits, split_stride);
                    if (bias) b += *reinterpret_cast<const float4v*>(bias + 8u * t + 4 * h);
                } else {
                    b = *reinterpret_cast<const float4v*>(y + at + 4 * h);
                }
                v[h] += b;
                *reinterpret_cast<float4v*>(x + at + 4 * h) = v[h];
            }
        }
    }
    if (!w) return;
    double sum = 0.0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int e = 0; e < 4; ++e) sum += static_cast<double>(v[h][e]) * v[h][e];
    }
    for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
    if ((t & 63u) == 0) red[t >> 6] = sum;
    __syncthreads();
    double total = 0.0;
#pragma unroll
    for (unsigned k = 0; k < kNormThreads / 64; ++k) total += red[k];
    const float scale = static_cast<float>(1.0 / sqrt(total / static_cast<double>(n) + eps));
    float o[8];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float xs = v[h][e] * scale;
            o[4 * h + e] = mine ? xs * g[h][e] : 0.0f;
        }
    }
    if (mine) {
        *reinterpret_cast<float4v*>(out + at) = float4v{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<float4v*>(out + at + 4) = float4v{o[4], o[5], o[6], o[7]};
    }
    if constexpr (LOAD || PF) {
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(o[e]));
        for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        if ((t & 63u) == 0) redf[t >> 6] = amax;
        __syncthreads();
        amax = redf[0];
#pragma unroll
        for (unsigned k = 1; k < kNormThreads / 64; ++k) amax = fmaxf(amax, redf[k]);
        float s, inv;
        block_scale(amax, s, inv);
        if constexpr (LOAD) {
            if (t < 4u * ld.nb) emit_split_run(t, o, s, r, ld.mp, ld.xs, ld.block_sums);
            if (t == 0) ld.inv_scale[r] = inv;
        } else {
            if (8u * t < pf.ldx) {
                half8v h;
#pragma unroll
                for (int e = 0; e < 8; ++e) h[e] = static_cast<_Float16>(mine ? o[e] * s : 0.0f);
                *reinterpret_cast<half8v*>(pf.xh + static_cast<std::uint64_t>(r) * pf.ldx + 8u * t) = h;
            }
            if (t == 0) pf.row_inv[r] = inv;
        }
    }
}

// out[r][i] = silu(g) * u with g, u the sums of a K-split fused gate|up
// linear's columns i and f + i (partials[s][r][2f], summed from zero in split
// order, then + bias): the split reduction and silu_mul_kernel's arithmetic
// in one pass, four columns per thread (f % 4 == 0).
__global__ __launch_bounds__(kThreads) void split_swiglu_kernel(const float4v* __restrict__ partials,
                                                                std::uint32_t splits, std::uint32_t stride4,
                                                                std::uint32_t total4, std::uint32_t f4,
                                                                const float4v* __restrict__ bias,
                                                                float4v* __restrict__ out) {
#pragma clang fp contract(off)
    for (std::uint32_t idx = blockIdx.x * kThreads + threadIdx.x; idx < total4; idx += gridDim.x * kThreads) {
        const std::uint32_t r = idx / f4, c = idx % f4;
        const std::uint32_t gi = r * 2u * f4 + c;
        float4v g = {0.0f, 0.0f, 0.0f, 0.0f}, u = {0.0f, 0.0f, 0.0f, 0.0f};
        for (std::uint32_t s = 0; s < splits; ++s) {
            g += partials[static_cast<std::uint64_t>(s) * stride4 + gi];
            u += partials[static_cast<std::uint64_t>(s) * stride4 + gi + f4];
        }
        if (bias) {
            g += bias[c];
            u += bias[f4 + c];
        }
        float4v o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float sg = g[e] / (1.0f + expf(-g[e]));
            o[e] = sg * u[e];
        }
        out[idx] = o;
    }
}

// silu_mul_kernel's SwiGLU over one padded row per workgroup with PF
// emission as rms_norm_vec_kernel has it (the row's outputs held in
// registers between the max and the conversion: f <= 24576).
constexpr unsigned kSiluHeldRuns = 3;

__global__ __launch_bounds__(kNormThreads) void silu_rows_prefill_kernel(const float* __restrict__ gate_up,
                                                                         float* __restrict__ out, std::uint64_t f,
                                                                         PrefillRows pf) {
#pragma clang fp contract(off)
    __shared__ float redf[kNormThreads / 64];
    const std::uint32_t r = blockIdx.x;
    const std::uint32_t t = threadIdx.x;
    const bool row_live = r < pf.rows;
    const std::uint64_t runs = f / 8u;
    const float* row = gate_up + static_cast<std::uint64_t>(row_live ? r : 0u) * 2u * f;
    float4v g[kSiluHeldRuns][2], u[kSiluHeldRuns][2];
#pragma unroll
    for (unsigned i = 0; i < kSiluHeldRuns; ++i) {
        const std::uint64_t run = t + kNormThreads * i;
        const std::uint64_t at = 8u * (run < runs ? run : 0u);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            g[i][h] = *reinterpret_cast<const float4v*>(row + at + 4 * h);
            u[i][h] = *reinterpret_cast<const float4v*>(row + f + at + 4 * h);
        }
    }
    float o[kSiluHeldRuns][8];
    float amax = 0.0f;
#pragma unroll
    for (unsigned i = 0; i < kSiluHeldRuns; ++i) {
        const std::uint64_t run = t + kNormThreads * i;
        const bool live = row_live && run < runs;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sg = g[i][h][e] / (1.0f + expf(-g[i][h][e]));
                o[i][4 * h + e] = live ? sg * u[i][h][e] : 0.0f;
            }
        }
        if (live) {
            float* dst = out + static_cast<std::uint64_t>(r) * f + 8u * run;
            *reinterpret_cast<float4v*>(dst) = float4v{o[i][0], o[i][1], o[i][2], o[i][3]};
            *reinterpret_cast<float4v*>(dst + 4) = float4v{o[i][4], o[i][5], o[i][6], o[i][7]};
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(o[i][e]));
    }
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((t & 63u) == 0) redf[t >> 6] = amax;
    __syncthreads();
    amax = redf[0];
#pragma unroll
    for (unsigned k = 1; k < kNormThreads / 64; ++k) amax = fmaxf(amax, redf[k]);
    float s, inv;
    block_scale(amax, s, inv);
#pragma unroll
    for (unsigned i = 0; i < kSiluHeldRuns + 1u; ++i) {
        // Runs past f (up to ldx) are zeros; f <= 24576 and ldx < f + 256.
        const std::uint64_t run = t + kNormThreads * i;
        if (8u * run >= pf.ldx) break;
        half8v h;
#pragma unroll
        for (int e = 0; e < 8; ++e) h[e] = static_cast<_Float16>(i < kSiluHeldRuns ? o[i < kSiluHeldRuns ? i : 0][e] * s : 0.0f);
        *reinterpret_cast<half8v*>(pf.xh + static_cast<std::uint64_t>(r) * pf.ldx + 8u * run) = h;
    }
    if (t == 0) pf.row_inv[r] = inv;
}

bool norm_vectorizable(const float* x, const float* y, const float* w, const float* out, std::uint64_t n) {
    const auto aligned = [](const void* p) { return reinterpret_cast<std::uintptr_t>(p) % 16u == 0; };
    return n % 8u == 0 && n <= 8u * static_cast<std::uint64_t>(kNormThreads) && aligned(x) &&
           (!y || aligned(y)) && aligned(w) && aligned(out);
}

unsigned grid_for(std::uint64_t work) {
    const std::uint64_t g = ceil_div(work, kThreads);
    return static_cast<unsigned>(g < 16384u ? (g ? g : 1u) : 16384u);
}

} // namespace

hipError_t launch_matrix_rows(const TilePlanes& p, const std::int32_t* rows, std::uint32_t m, float* out,
                              hipStream_t stream) {
    const unsigned gx = static_cast<unsigned>(ceil_div(p.k, kThreads) < 64u ? ceil_div(p.k, kThreads) : 64u);
    hipLaunchKernelGGL(matrix_rows_kernel, dim3(gx, m), dim3(kThreads), 0, stream, p.type, p.codes, p.scales, p.k,
                       p.n, p.kt, rows, m, out);
    return hipGetLastError();
}

hipError_t launch_rms_norm(const float* x, const float* w, float* out, std::uint32_t m, std::uint64_t n, double eps,
                           hipStream_t stream) {
    if (norm_vectorizable(x, nullptr, w, out, n)) {
        hipLaunchKernelGGL((rms_norm_vec_kernel<false, false>), dim3(m), dim3(kNormThreads), 0, stream,
                           const_cast<float*>(x), static_cast<const float*>(nullptr), w, out, n, eps, 0u,
                           std::uint64_t{0}, static_cast<const float*>(nullptr), NormLoad{});
    } else {
        hipLaunchKernelGGL(rms_norm_kernel, dim3(m), dim3(kThreads), 0, stream, x, w, out, n, eps);
    }
    return hipGetLastError();
}

hipError_t launch_add_rms_norm(float* x, const float* y, const float* w, float* out, std::uint32_t m, std::uint64_t n,
                               double eps, hipStream_t stream) {
    if (norm_vectorizable(x, y, w, out, n)) {
        hipLaunchKernelGGL((rms_norm_vec_kernel<false, false>), dim3(m), dim3(kNormThreads), 0, stream, x, y, w, out,
                           n, eps, 0u, std::uint64_t{0}, static_cast<const float*>(nullptr), NormLoad{});
        return hipGetLastError();
    }
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(static_cast<std::uint64_t>(m) * n)), dim3(kThreads), 0, stream, x, y,
                       static_cast<std::uint64_t>(m) * n);
    hipLaunchKernelGGL(rms_norm_kernel, dim3(m), dim3(kThreads), 0, stream, x, w, out, n, eps);
    return hipGetLastError();
}

hipError_t launch_rope(float* qkv, std::uint64_t stride, std::uint32_t m, const std::int32_t* positions,
                       std::uint32_t q_heads, std::uint32_t kv_heads, std::uint32_t head_dim, std::uint32_t rope_dims,
                       const void* table, std::uint64_t table_positions, hipStream_t stream) {
    const std::uint64_t work = static_cast<std::uint64_t>(m) * (q_heads + kv_heads) * (rope_dims / 2u);
    hipLaunchKernelGGL(rope_kernel, dim3(grid_for(work)), dim3(kThreads), 0, stream, qkv, stride, m, positions,
                       q_heads, kv_heads, head_dim, rope_dims, static_cast<const float2*>(table), table_positions);
    return hipGetLastError();
}

hipError_t launch_kv_append(const KvLayout& kv, const float* qkv, std::uint64_t stride, std::uint64_t q_width,
                            std::uint32_t m, const std::int32_t* positions, const std::int32_t* tables,
                            std::uint32_t layer, hipStream_t stream) {
    const KvGeometry g = kv;
    const unsigned gx = static_cast<unsigned>(ceil_div(kv.kv_width, kThreads));
    hipLaunchKernelGGL(kv_append_kernel, dim3(gx, m), dim3(kThreads), 0, stream, g, qkv, stride, q_width, m,
                       positions, tables, layer);
    return hipGetLastError();
}

hipError_t launch_attention(const KvLayout& kv, const float* qkv, std::uint64_t stride, std::uint32_t m,
                            const std::int32_t* positions, const std::int32_t* tables, std::uint32_t layer,
                            std::uint32_t q_heads, std::uint32_t kv_heads, std::uint32_t head_dim, double* scratch,
                            std::uint64_t score_stride, float* out, hipStream_t stream) {
    if (head_dim > 512u) return hipErrorInvalidValue;
    const KvGeometry g = kv;
    hipLaunchKernelGGL(attention_kernel, dim3(m * q_heads), dim3(kThreads), 0, stream, g, qkv, stride, m, positions,
                       tables, layer, q_heads, kv_heads, head_dim, scratch, score_stride, out);
    return hipGetLastError();
}

namespace {
hipError_t rope_kv_append(const KvLayout& kv, float* qkv, std::uint64_t stride, std::uint64_t q_width,
                          std::uint32_t m, const std::int32_t* positions, const std::int32_t* tables,
                          std::uint32_t layer, std::uint32_t q_heads, std::uint32_t kv_heads, std::uint32_t head_dim,
                          std::uint32_t rope_dims, const void* table, std::uint64_t table_positions,
                          const QkvSplit* split, hipStream_t stream) {
    const KvGeometry g = kv;
    const std::uint64_t per_row = static_cast<std::uint64_t>(q_heads) * (rope_dims / 2u) +
                                  static_cast<std::uint64_t>(kv_heads) * (rope_dims / 2u + head_dim - rope_dims) +
                                  (split ? static_cast<std::uint64_t>(q_heads) * (head_dim - rope_dims) : 0u) +
                                  kv.kv_width;
    const std::uint64_t blocks = ceil_div(per_row, static_cast<std::uint64_t>(kThreads));
    const unsigned gx = static_cast<unsigned>(blocks < 64u ? blocks : 64u);
    if (split) {
        hipLaunchKernelGGL(rope_kv_append_kernel<true>, dim3(gx, m), dim3(kThreads), 0, stream, g, qkv, stride,
                           q_width, m, positions, tables, layer, q_heads, kv_heads, head_dim, rope_dims,
                           static_cast<const float2*>(table), table_positions, *split);
    } else {
        hipLaunchKernelGGL(rope_kv_append_kernel<false>, dim3(gx, m), dim3(kThreads), 0, stream, g, qkv, stride,
                           q_width, m, positions, tables, layer, q_heads, kv_heads, head_dim, rope_dims,
                           static_cast<const float2*>(table), table_positions, QkvSplit{});
    }
    return hipGetLastError();
}
} // namespace

hipError_t launch_rope_kv_append(const KvLayout& kv, float* qkv, std::uint64_t stride, std::uint64_t q_width,
                                 std::uint32_t m, const std::int32_t* positions, const std::int32_t* tables,
                                 std::uint32_t layer, std::uint32_t q_heads, std::uint32_t kv_heads,
                                 std::uint32_t head_dim, std::uint32_t rope_dims, const void* table,
                                 std::uint64_t table_positions, hipStream_t stream) {
    return rope_kv_append(kv, qkv, stride, q_width, m, positions, tables, layer, q_heads, kv_heads, head_dim,
                          rope_dims, table, table_positions, nullptr, stream);
}

bool prefill_norm_fits(std::uint64_t n, std::uint64_t ldx) {
    return n % 8u == 0 && n <= 8u * static_cast<std::uint64_t>(kNormThreads) && ldx >= n && ldx % 8u == 0 &&
           ldx <= 8u * static_cast<std::uint64_t>(kNormThreads);
}

hipError_t launch_rms_norm_prefill(float* x, const float* y, const float* w, float* out, std::uint32_t m,
                                   std::uint64_t n, double eps, _Float16* xh, float* row_inv, std::uint32_t mp,
                                   std::uint64_t ldx, hipStream_t stream) {
    if (!prefill_norm_fits(n, ldx) || !norm_vectorizable(x, y, w, out, n) || mp < m) return hipErrorInvalidValue;
    const PrefillRows pf{xh, row_inv, m, ldx};
    hipLaunchKernelGGL((rms_norm_vec_kernel<false, false, true>), dim3(mp), dim3(kNormThreads), 0, stream, x, y, w,
                       out, n, eps, 0u, std::uint64_t{0}, static_cast<const float*>(nullptr), NormLoad{}, pf);
    return hipGetLastError();
}

bool silu_prefill_fits(std::uint64_t ffn, std::uint64_t ldx) {
    return ffn % 8u == 0 && ffn <= 8u * kSiluHeldRuns * static_cast<std::uint64_t>(kNormThreads) && ldx >= ffn &&
           ldx % 8u == 0 && ldx <= 8u * (kSiluHeldRuns + 1u) * static_cast<std::uint64_t>(kNormThreads);
}

hipError_t launch_silu_mul_prefill(const float* gate_up, float* out, std::uint32_t m, std::uint64_t ffn, _Float16* xh,
                                   float* row_inv, std::uint32_t mp, std::uint64_t ldx, hipStream_t stream) {
    const auto aligned = [](const void* p) { return reinterpret_cast<std::uintptr_t>(p) % 16u == 0; };
    if (!silu_prefill_fits(ffn, ldx) || !aligned(gate_up) || !aligned(out) || !aligned(xh) || mp < m) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(silu_rows_prefill_kernel, dim3(mp), dim3(kNormThreads), 0, stream, gate_up, out, ffn,
                       PrefillRows{xh, row_inv, m, ldx});
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* gate_up, float* out, std::uint32_t m, std::uint64_t ffn, hipStream_t stream) {
    hipLaunchKernelGGL(silu_mul_kernel, dim3(grid_for(static_cast<std::uint64_t>(m) * ffn)), dim3(kThreads), 0, stream,
                       gate_up, out, m, ffn);
    return hipGetLastError();
}

hipError_t launch_add(float* x, const float* y, std::uint64_t count, hipStream_t stream) {
    hipLaunchKernelGGL(add_kernel, dim3(grid_for(count)), dim3(kThreads), 0, stream, x, y, count);
    return hipGetLastError();
}

bool split_epilogue_fits(const SplitEpilogue& e, const float* partials, const float* bias, std::uint32_t m,
                        std::uint64_t n) {
    const auto aligned = [](const void* p) { return reinterpret_cast<std::uintptr_t>(p) % 16u == 0; };
    if (!aligned(partials) || (bias && !aligned(bias)) || !aligned(e.out)) return false;
    if (e.kind == kEpilogueSwiglu) {
        return n % 8u == 0 && static_cast<std::uint64_t>(m) * n / 4u < (1ull << 32);
    }
    if (e.kind == kEpilogueRopeKv) return e.rope != nullptr;
    if (e.kind == kEpilogueResidual) {
        return n % 8u == 0 && n <= 8u * static_cast<std::uint64_t>(kNormThreads) &&
               (!e.norm_weight || (aligned(e.norm_weight) && aligned(e.norm_out))) &&
               (!e.load || (e.norm_weight && m <= 64u && 4u * e.load_blocks <= kNormThreads)) &&
               (!e.prefill || (e.norm_weight && !e.load && e.prefill->mp >= m && aligned(e.prefill->xh) &&
                               prefill_norm_fits(n, e.prefill->ldx)));
    }
    return false;
}

hipError_t launch_split_epilogue(const float* partials, std::uint32_t splits, std::uint32_t m, std::uint64_t n,
                                 const float* bias, const SplitEpilogue& e, hipStream_t stream) {
    if (!split_epilogue_fits(e, partials, bias, m, n)) return hipErrorInvalidValue;
    if (e.kind == kEpilogueRopeKv) {
        const RopeKvArgs& a = *e.rope;
        const QkvSplit split{partials, splits, static_cast<std::uint64_t>(m) * n, bias};
        return rope_kv_append(a.kv, e.out, n, static_cast<std::uint64_t>(a.q_heads) * a.head_dim, m, a.positions,
                              a.tables, a.layer, a.q_heads, a.kv_heads, a.head_dim, a.rope_dims, a.table,
                              a.table_positions, &split, stream);
    }
    if (e.kind == kEpilogueSwiglu) {
        const std::uint32_t f4 = static_cast<std::uint32_t>(n / 8u);
        const std::uint32_t total4 = m * f4;
        const std::uint64_t grid = ceil_div(static_cast<std::uint64_t>(total4), kThreads);
        hipLaunchKernelGGL(split_swiglu_kernel, dim3(static_cast<unsigned>(grid < 2048u ? grid : 2048u)),
                           dim3(kThreads), 0, stream, reinterpret_cast<const float4v*>(partials), splits,
                           static_cast<std::uint32_t>(static_cast<std::uint64_t>(m) * n / 4u), total4, f4,
                           reinterpret_cast<const float4v*>(bias), reinterpret_cast<float4v*>(e.out));
        return hipGetLastError();
    }
    if (e.prefill) {
        const PrefillRows pf{e.prefill->xh, e.prefill->row_inv, m, e.prefill->ldx};
        hipLaunchKernelGGL((rms_norm_vec_kernel<true, false, true>), dim3(e.prefill->mp), dim3(kNormThreads), 0,
                           stream, e.out, partials, e.norm_weight, e.norm_out, n, e.eps, splits,
                           static_cast<std::uint64_t>(m) * n, bias, NormLoad{}, pf);
        return hipGetLastError();
    }
    if (e.load) {
        const NormLoad ld{static_cast<uint4*>(e.load->xs), e.load->block_sums, e.load->inv_scale, m,
                          static_cast<std::uint32_t>(ceil_div(m, 16u) * 16u), e.load_blocks};
        hipLaunchKernelGGL((rms_norm_vec_kernel<true, true>), dim3(ld.mp), dim3(kNormThreads), 0, stream, e.out,
                           partials, e.norm_weight, e.norm_out, n, e.eps, splits, static_cast<std::uint64_t>(m) * n,
                           bias, ld);
    } else {
        hipLaunchKernelGGL((rms_norm_vec_kernel<true, false>), dim3(m), dim3(kNormThreads), 0, stream, e.out,
                           partials, e.norm_weight, e.norm_out, n, e.eps, splits, static_cast<std::uint64_t>(m) * n,
                           bias, NormLoad{});
    }
    return hipGetLastError();
}

std::uint64_t argmax_scratch_bytes(std::uint32_t m, std::uint64_t n) {
    return static_cast<std::uint64_t>(m) * ceil_div(n, kArgmaxSlice) * sizeof(ArgmaxPartial);
}

hipError_t launch_argmax(const float* logits, std::uint32_t m, std::uint64_t n, std::int32_t* out, void* scratch,
                         hipStream_t stream) {
    const std::uint64_t slices = ceil_div(n, kArgmaxSlice);
    if (m == 0u || slices == 0u || slices > 0x7fffffffu || m > 65535u) return hipErrorInvalidValue;
    auto* partials = static_cast<ArgmaxPartial*>(scratch);
    hipLaunchKernelGGL(argmax_slice_kernel, dim3(static_cast<unsigned>(slices), m), dim3(kArgmaxThreads), 0, stream,
                       logits, n, static_cast<std::uint32_t>(slices), partials);
    hipLaunchKernelGGL(argmax_rows_kernel, dim3(m), dim3(64), 0, stream, partials,
                       static_cast<std::uint32_t>(slices), out);
    return hipGetLastError();
}

} // namespace air_hip

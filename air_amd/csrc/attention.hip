// attention.hip -- tiled online-softmax attention over the paged fp32 KV pool.
//
// The online_softmax tactic of AttentionPolicy (the reference's
// attention_batch_paged_online_kernel, src/cuda/cuda_backend.cu:1089-1154,
// keeps one (query token, head) pair per block and walks the keys one at a
// time).  Here a workgroup owns a tile of up to 16 query vectors that share a
// sequence and a KV head -- 16 consecutive prompt rows of one q head in a
// prefill, or the grouped q heads of one KV head of a decode row -- and walks
// the keys in chunks of 32 (decode) or 64 (prefill) tokens staged through LDS, so each K/V element is
// read from memory once per tile instead of once per query vector:
//
//   S = (q . k) * scale        16 x chunk, chunk / 16 dots per thread, float
//   m' = max(m, rowmax S);  p = exp(S - m');  l = l e^(m-m') + rowsum p
//   acc = acc e^(m-m') + p . V 8 (D=128) or 4 (D=64) dims per thread
//
// Causality: row r attends tokens 0..positions[r].  Long key ranges with few
// tiles are split over workgroups (flash-decoding); each split writes its
// (m, l, acc) and a second kernel merges them.  All arithmetic is f32 and
// unfused-exact products are not required: the result differs from the
// reference's double softmax by ~1e-6 relative (the tactic's tolerance is
// that of the linears).
#include "air_hip_kernels.hpp"
#include "air_hip_kv.hpp"
#include "air_hip_layout.hpp"

namespace air_hip {
namespace {

constexpr unsigned kAttnThreads = 256;
// Key tokens per LDS stage: 32 for decode-width steps (half the LDS of 64,
// so three workgroups share a CU, and twice the key splits for short
// grids), 64 for prefill tiles (half the barriers per key).
std::uint32_t chunk_for(std::uint32_t m) { return m <= 64u ? 32u : 64u; }
constexpr unsigned kTileVectors = 16;
constexpr unsigned kMaxSplits = 64;  // one wave reduces a vector's splits in the merge

__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }

// A tile names rows and q heads that exist, at most 16 query vectors, and q
// heads of a single KV head.
__device__ __forceinline__ bool tile_ok(const AttentionTile& t, std::uint32_t m, std::uint32_t q_heads,
                                        std::uint32_t kv_heads) {
    if (t.rows == 0u || t.heads == 0u || t.rows > kTileVectors || t.heads > kTileVectors ||
        t.rows * t.heads > kTileVectors) {
        return false;
    }
    if (t.row >= m || t.rows > m - t.row || t.head >= q_heads || t.heads > q_heads - t.head) return false;
    const std::uint32_t group = q_heads / kv_heads;
    return t.head / group == (t.head + t.heads - 1u) / group;
}

template <unsigned D, unsigned kChunk>
__global__ __launch_bounds__(kAttnThreads) void attention_tile_kernel(
    KvGeometry g, const float* __restrict__ qkv, std::uint64_t stride, std::uint32_t m,
    const std::int32_t* __restrict__ positions,
    const std::int32_t* __restrict__ tables, std::uint32_t layer, std::uint32_t q_heads, std::uint32_t kv_heads,
    const AttentionTile* __restrict__ tiles, std::uint32_t splits, float scale, float* __restrict__ partials,
    float* __restrict__ out) {
    constexpr unsigned kTokJ = kChunk / 16;   // key tokens per thread in a chunk (16 lanes per query vector)
    constexpr unsigned LD = D + 4;            // padded LDS row (floats), keeps float4 alignment
    constexpr unsigned D4 = D / 4;
    constexpr unsigned ACC = D / 16;          // output dims per thread
    __shared__ float qs[kTileVectors][LD];
    __shared__ float ks[kChunk][LD];
    __shared__ float vs[kChunk][LD];
    __shared__ float ps[kTileVectors][kChunk + 1];
    __shared__ std::int64_t slot_off[2][kChunk];   // pool offset of each chunk token's K slot, -1 if absent

    const AttentionTile tile = tiles[blockIdx.x];
    if (!tile_ok(tile, m, q_heads, kv_heads)) return;
    const std::uint32_t split = blockIdx.y;
    const unsigned tid = threadIdx.x;
    const unsigned qi = tid >> 4;             // query vector of this thread
    const unsigned lane16 = tid & 15u;
    const unsigned nq = tile.rows * tile.heads;
    const std::uint32_t kvh = static_cast<std::uint32_t>((static_cast<std::uint64_t>(tile.head) * kv_heads) / q_heads);
    const std::int32_t* table = tables + static_cast<std::uint64_t>(tile.row) * g.max_pages;

    // Keys of the tile: 0 .. max position + 1, in chunks; this split's share.
    std::int64_t tmax = 0;
    for (unsigned r = 0; r < tile.rows; ++r) {
        const std::int64_t p = positions[tile.row + r];
        tmax = p + 1 > tmax ? p + 1 : tmax;
    }
    const std::uint32_t chunks = static_cast<std::uint32_t>((tmax + kChunk - 1) / kChunk);
    const std::uint32_t per_split = (chunks + splits - 1) / splits;
    const std::uint32_t c_begin = split * per_split;
    const std::uint32_t c_end = c_begin + per_split < chunks ? c_begin + per_split : chunks;

    // This thread's query vector: (row, head) and its position.
    const bool active = qi < nq;
    const unsigned q_row = tile.row + (active ? qi / tile.heads : 0u);
    const unsigned q_head = tile.head + (active ? qi % tile.heads : 0u);
    const std::int64_t q_pos = active ? positions[q_row] : -1;

    for (unsigned idx = tid; idx < kTileVectors * D4; idx += kAttnThreads) {
        const unsigned v = idx / D4, d4 = idx % D4;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (v < nq) {
            const unsigned row = tile.row + v / tile.heads, head = tile.head + v % tile.heads;
            x = load4(qkv + static_cast<std::uint64_t>(row) * stride + static_cast<std::uint64_t>(head) * D + 4u * d4);
        }
        *reinterpret_cast<float4*>(&qs[v][4u * d4]) = x;
    }

    float mx = -__builtin_huge_valf();   // running maximum of the scores
    float l = 0.0f;
    float acc[ACC];
#pragma unroll
    for (unsigned i = 0; i < ACC; ++i) acc[i] = 0.0f;

    // V of a token sits page_tokens * kv_width floats after its K in the page.
    const std::uint64_t v_after_k = static_cast<std::uint64_t>(g.page_tokens) * g.kv_width;
    constexpr unsigned kIters = kChunk * D4 / kAttnThreads;   // float4 of K (and of V) per thread per chunk
    // Two-stage pipeline: chunk c+1's page slots are resolved and its K and V
    // loads issued into registers before chunk c is computed from LDS.
    const auto resolve = [&](std::uint32_t c, unsigned buf) __attribute__((always_inline)) {
        if (tid < kChunk) {   // page table lookup, once per token
            const std::int64_t token = static_cast<std::int64_t>(c) * kChunk + tid;
            std::int64_t off = -1;
            if (token < tmax) {
                const float* kp = kv_slot(g, table, layer, static_cast<std::uint64_t>(token), false);
                if (kp) off = kp - g.pool;
            }
            slot_off[buf][tid] = off;
        }
    };
    float4 kr[kIters], vr[kIters];
    const auto fetch = [&](unsigned buf) __attribute__((always_inline)) {
#pragma unroll
        for (unsigned it = 0; it < kIters; ++it) {
            const unsigned idx = tid + it * kAttnThreads;
            const unsigned t = idx / D4, d4 = idx % D4;
            const std::int64_t off = slot_off[buf][t];
            kr[it] = make_float4(0.f, 0.f, 0.f, 0.f);
            vr[it] = kr[it];
            if (off >= 0) {
                const float* kp = g.pool + off + static_cast<std::uint64_t>(kvh) * D + 4u * d4;
                kr[it] = load4(kp);
                vr[it] = load4(kp + v_after_k);
            }
        }
    };
    if (c_begin < c_end) resolve(c_begin, 0u);
    __syncthreads();
    if (c_begin < c_end) fetch(0u);
    for (std::uint32_t c = c_begin; c < c_end; ++c) {
        const std::int64_t c0 = static_cast<std::int64_t>(c) * kChunk;
        const unsigned buf = (c - c_begin) & 1u;
        __syncthreads();  // previous chunk's K, V and P are consumed
#pragma unroll
        for (unsigned it = 0; it < kIters; ++it) {
            const unsigned idx = tid + it * kAttnThreads;
            const unsigned t = idx / D4, d4 = idx % D4;
            *reinterpret_cast<float4*>(&ks[t][4u * d4]) = kr[it];
            *reinterpret_cast<float4*>(&vs[t][4u * d4]) = vr[it];
        }
        if (c + 1u < c_end) resolve(c + 1u, buf ^ 1u);
        __syncthreads();
        if (c + 1u < c_end) fetch(buf ^ 1u);   // in flight while chunk c computes

        // Scores of tokens lane16 + 16 j.  Idle vector slots (a decode tile
        // of 7 grouped heads leaves 9 of 16) skip the LDS reads: whole waves
        // of them branch around the loop.
        float s[kTokJ];
#pragma unroll
        for (unsigned j = 0; j < kTokJ; ++j) s[j] = 0.0f;
        if (active) {
#pragma unroll 4
            for (unsigned d4 = 0; d4 < D4; ++d4) {
                const float4 q4 = *reinterpret_cast<const float4*>(&qs[qi][4u * d4]);
#pragma unroll
                for (unsigned j = 0; j < kTokJ; ++j) {
                    const float4 k4 = *reinterpret_cast<const float4*>(&ks[lane16 + 16u * j][4u * d4]);
                    s[j] += q4.x * k4.x + q4.y * k4.y + q4.z * k4.z + q4.w * k4.w;
                }
            }
        }
        float row_max = -__builtin_huge_valf();
#pragma unroll
        for (unsigned j = 0; j < kTokJ; ++j) {
            const std::int64_t token = c0 + lane16 + 16u * j;
            const bool valid = active && token <= q_pos;
            s[j] = valid ? s[j] * scale : -__builtin_huge_valf();
            row_max = s[j] > row_max ? s[j] : row_max;
        }
        // The 16 threads of one query vector are lanes 16q..16q+15 of a wave.
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            const float o = __shfl_xor(row_max, off, 16);
            row_max = o > row_max ? o : row_max;
        }
        const float m_new = row_max > mx ? row_max : mx;
        const bool none = m_new == -__builtin_huge_valf();   // no key of this vector yet
        const float alpha = none ? 1.0f : __expf(mx - m_new);
        float row_sum = 0.0f;
#pragma unroll
        for (unsigned j = 0; j < kTokJ; ++j) {
            const float p = none || s[j] == -__builtin_huge_valf() ? 0.0f : __expf(s[j] - m_new);
            row_sum += p;
            ps[qi][lane16 + 16u * j] = p;
        }
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) row_sum += __shfl_xor(row_sum, off, 16);
        l = l * alpha + row_sum;
        mx = m_new;
#pragma unroll
        for (unsigned i = 0; i < ACC; ++i) acc[i] *= alpha;
        __syncthreads();

        // acc[dims 4 (lane16 + 16 j) ..] += sum over tokens of p * v.
        const std::int64_t last = q_pos - c0;            // tokens past it have p = 0
        const unsigned count = last < 0 ? 0u : (last >= kChunk ? kChunk : static_cast<unsigned>(last) + 1u);
        for (unsigned t = 0; t < count; ++t) {
            const float p = ps[qi][t];
#pragma unroll
            for (unsigned j = 0; j < ACC / 4; ++j) {
                const float4 v4 = *reinterpret_cast<const float4*>(&vs[t][4u * (lane16 + 16u * j)]);
                acc[4 * j + 0] += p * v4.x;
                acc[4 * j + 1] += p * v4.y;
                acc[4 * j + 2] += p * v4.z;
                acc[4 * j + 3] += p * v4.w;
            }
        }
    }

    if (!active) return;
    if (splits == 1u) {
        const float inv = 1.0f / l;
        float* dst = out + static_cast<std::uint64_t>(q_row) * q_heads * D + static_cast<std::uint64_t>(q_head) * D;
#pragma unroll
        for (unsigned j = 0; j < ACC / 4; ++j) {
            const float4 o = make_float4(acc[4 * j] * inv, acc[4 * j + 1] * inv, acc[4 * j + 2] * inv,
                                         acc[4 * j + 3] * inv);
            *reinterpret_cast<float4*>(dst + 4u * (lane16 + 16u * j)) = o;
        }
        return;
    }
    // Partial of this split: [tile][split][vector] {m, l, pad, pad, acc[D]}.
    float* part = partials + ((static_cast<std::uint64_t>(blockIdx.x) * splits + split) * kTileVectors + qi) * (D + 4u);
    if (lane16 == 0) {
        part[0] = mx;
        part[1] = l;
    }
#pragma unroll
    for (unsigned j = 0; j < ACC / 4; ++j) {
        *reinterpret_cast<float4*>(part + 4u + 4u * (lane16 + 16u * j)) =
            make_float4(acc[4 * j], acc[4 * j + 1], acc[4 * j + 2], acc[4 * j + 3]);
    }
}

// Merges the splits of each tile: o = sum_s acc_s e^(m_s - M) / sum_s l_s e^(m_s - M).
template <unsigned D>
__global__ __launch_bounds__(kAttnThreads) void attention_merge_kernel(const AttentionTile* __restrict__ tiles,
                                                                       std::uint32_t splits, std::uint32_t m,
                                                                       std::uint32_t q_heads, std::uint32_t kv_heads,
                                                                       const float* __restrict__ partials,
                                                                       float* __restrict__ out) {
    __shared__ float weight[kTileVectors][kMaxSplits];   // e^(m_s - M) / L
    const AttentionTile tile = tiles[blockIdx.x];
    if (!tile_ok(tile, m, q_heads, kv_heads) || splits > kMaxSplits) return;
    const unsigned nq = tile.rows * tile.heads;
    const std::uint64_t step = static_cast<std::uint64_t>(kTileVectors) * (D + 4u);   // floats between splits
    const float* tile_base = partials + static_cast<std::uint64_t>(blockIdx.x) * splits * step;
    // One thread per (vector, split) reads its (m, l); a wave reduces each vector.
    for (unsigned idx = threadIdx.x; idx < nq * kMaxSplits; idx += kAttnThreads) {
        const unsigned v = idx / kMaxSplits, s = idx % kMaxSplits;
        float ms = -__builtin_huge_valf(), ls = 0.0f;
        if (s < splits) {
            ms = tile_base[s * step + static_cast<std::uint64_t>(v) * (D + 4u)];
            ls = tile_base[s * step + static_cast<std::uint64_t>(v) * (D + 4u) + 1u];
        }
        float mx = ms;
        for (int off = 32; off > 0; off >>= 1) {
            const float o = __shfl_xor(mx, off);
            mx = o > mx ? o : mx;
        }
        const float w = ms == -__builtin_huge_valf() ? 0.0f : __expf(ms - mx);
        float den = ls * w;
        for (int off = 32; off > 0; off >>= 1) den += __shfl_xor(den, off);
        weight[v][s] = w / den;
    }
    __syncthreads();
    constexpr unsigned D4 = D / 4;
    for (unsigned idx = threadIdx.x; idx < nq * D4; idx += kAttnThreads) {
        const unsigned v = idx / D4, d4 = idx % D4;
        const float* base = tile_base + static_cast<std::uint64_t>(v) * (D + 4u) + 4u + 4u * d4;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        for (std::uint32_t s = 0; s < splits; ++s) {
            const float w = weight[v][s];
            const float4 a = load4(base + s * step);
            o.x += a.x * w;
            o.y += a.y * w;
            o.z += a.z * w;
            o.w += a.w * w;
        }
        const unsigned row = tile.row + v / tile.heads, head = tile.head + v % tile.heads;
        *reinterpret_cast<float4*>(out + static_cast<std::uint64_t>(row) * q_heads * D +
                                   static_cast<std::uint64_t>(head) * D + 4u * d4) = o;
    }
}

} // namespace

std::uint32_t make_attention_tiles(const std::uint32_t* run_rows, std::uint32_t runs, std::uint32_t q_heads,
                                   std::uint32_t kv_heads, AttentionTile* tiles, std::uint32_t capacity) {
    const std::uint32_t group = q_heads / kv_heads;
    std::uint32_t count = 0, row = 0;
    const auto push = [&](std::uint32_t r, std::uint32_t rows, std::uint32_t h, std::uint32_t heads) {
        if (tiles && count < capacity) tiles[count] = AttentionTile{r, rows, h, heads};
        ++count;
    };
    for (std::uint32_t i = 0; i < runs; ++i) {
        const std::uint32_t n = run_rows[i];
        if (n == 1u) {
            // One row: the q heads of each KV head together.
            for (std::uint32_t kvh = 0; kvh < kv_heads; ++kvh) {
                for (std::uint32_t h = 0; h < group; h += kTileVectors) {
                    push(row, 1u, kvh * group + h, group - h < kTileVectors ? group - h : kTileVectors);
                }
            }
        } else {
            // Several rows of one sequence: 16 rows of one q head.
            for (std::uint32_t h = 0; h < q_heads; ++h) {
                for (std::uint32_t r = 0; r < n; r += kTileVectors) {
                    push(row + r, n - r < kTileVectors ? n - r : kTileVectors, h, 1u);
                }
            }
        }
        row += n;
    }
    return count;
}

std::uint32_t attention_splits(std::uint32_t tiles, std::uint64_t max_tokens, std::uint32_t m) {
    const std::uint32_t chunk = chunk_for(m);
    const std::uint64_t chunks = (max_tokens + chunk - 1) / chunk;
    if (tiles == 0 || chunks <= 1) return 1;
    // 32-token chunks: about as many workgroups as fit in one round (three
    // per CU on 256 CUs); 64-token chunks (prefill): about 512.
    const std::uint64_t want = chunk == 32u ? (768u / tiles > 0u ? 768u / tiles : 1u) : (512u + tiles - 1) / tiles;
    const std::uint64_t s = want < chunks ? want : chunks;
    return static_cast<std::uint32_t>(s < 64 ? s : 64);
}

std::uint64_t attention_partials_bytes(std::uint32_t tiles, std::uint32_t splits, std::uint32_t head_dim) {
    if (splits <= 1) return 0;
    return static_cast<std::uint64_t>(tiles) * splits * kTileVectors * (head_dim + 4u) * sizeof(float);
}

hipError_t launch_attention_tiles(const KvLayout& kv, const float* qkv, std::uint64_t stride, std::uint32_t m,
                                  const std::int32_t* positions, const std::int32_t* tables, std::uint32_t layer,
                                  std::uint32_t q_heads, std::uint32_t kv_heads, std::uint32_t head_dim,
                                  const AttentionTile* tiles, std::uint32_t tile_count, std::uint32_t splits,
                                  float* partials, float* out, hipStream_t stream) {
    const KvGeometry g{kv.pool, kv.page_tokens, kv.kv_width, kv.layers, kv.max_pages, kv.pool_pages};
    const float scale = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(head_dim)));
    const dim3 grid(tile_count, splits);
    const bool small = chunk_for(m) == 32u;
    if (head_dim == 128u) {
        if (small) {
            hipLaunchKernelGGL((attention_tile_kernel<128, 32>), grid, dim3(kAttnThreads), 0, stream, g, qkv, stride,
                               m, positions, tables, layer, q_heads, kv_heads, tiles, splits, scale, partials, out);
        } else {
            hipLaunchKernelGGL((attention_tile_kernel<128, 64>), grid, dim3(kAttnThreads), 0, stream, g, qkv, stride,
                               m, positions, tables, layer, q_heads, kv_heads, tiles, splits, scale, partials, out);
        }
        if (splits > 1u) {
            hipLaunchKernelGGL(attention_merge_kernel<128>, dim3(tile_count), dim3(kAttnThreads), 0, stream, tiles,
                               splits, m, q_heads, kv_heads, partials, out);
        }
    } else if (head_dim == 64u) {
        if (small) {
            hipLaunchKernelGGL((attention_tile_kernel<64, 32>), grid, dim3(kAttnThreads), 0, stream, g, qkv, stride,
                               m, positions, tables, layer, q_heads, kv_heads, tiles, splits, scale, partials, out);
        } else {
            hipLaunchKernelGGL((attention_tile_kernel<64, 64>), grid, dim3(kAttnThreads), 0, stream, g, qkv, stride,
                               m, positions, tables, layer, q_heads, kv_heads, tiles, splits, scale, partials, out);
        }
        if (splits > 1u) {
            hipLaunchKernelGGL(attention_merge_kernel<64>, dim3(tile_count), dim3(kAttnThreads), 0, stream, tiles,
                               splits, m, q_heads, kv_heads, partials, out);
        }
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace air_hip

// attention.hip -- tiled online-softmax attention over the paged fp32 KV pool.
//
// The online_softmax tactic of AttentionPolicy (the reference's
// attention_batch_paged_online_kernel, src/cuda/cuda_backend.cu:1093-1154,
// keeps one (query token, head) pair per block and walks the keys one at a
// time).  Here a workgroup owns a tile of up to 16 query vectors that share a
// sequence and a KV head -- 16 consecutive prompt rows of one q head in a
// prefill, or the grouped q heads of one KV head of a decode row -- and walks
// the keys in chunks of 64 tokens staged through LDS, so each K/V element is
// read from memory once per tile instead of once per query vector, with the
// products on the f32 matrix cores (attention_mfma_kernel):
//
//   S = (q . k) * scale        16 vectors x 64 keys, 16 keys per wave
//   m' = max(m, rowmax S);  p = exp(S - m');  l = l e^(m-m') + rowsum p
//   acc = acc e^(m-m') + p . V
//
// Causality: row r attends tokens 0..positions[r].  Long key ranges with few
// tiles are split over workgroups (flash-decoding); each split writes its
// (m, l, acc) and a second kernel merges them.  (A merge by the tile's last
// workgroup, found with an arrival counter, needs agent-scope fences around
// the partials, which write back and invalidate L2 per workgroup: measured
// slower than the second launch.)  All arithmetic is f32: the result differs
// from the reference's double softmax by ~1e-6 relative (the tactic's
// tolerance is that of the linears).
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"
#include "air_hip_kv.hpp"
#include "air_hip_layout.hpp"

namespace air_hip {
namespace {

constexpr unsigned kAttnThreads = 256;
// Key tokens per LDS stage (16 per wave).  The VALU kernel this replaced
// used 32 for decode widths; the matrix-core kernel at 64 is faster there
// too (M = 1: 2.305 -> 2.252 ms per token; 32 rows 6.8k -> 6.9k tok/s).
constexpr std::uint32_t kChunkKeys = 64;
constexpr unsigned kTileVectors = 16;
constexpr unsigned kMaxSplits = 64;  // bounds the partials of a tile

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

// The 64-key chunk steps on the f32 matrix cores (v_mfma_f32_16x16x4_f32:
// fp32 products summed in fp32, the VALU kernel's precision).  Wave w owns
// keys 16w .. 16w + 15 of every chunk and keeps its own online softmax over
// them; the four waves' (m, l, acc) merge once at the end.  Per chunk:
//
//   S^T = K Q^T   A = 16 keys x 4 dims, B = 4 dims x 16 query vectors: D
//                 leaves lane l with the scores of vector l % 16 for keys
//                 4 (l / 16) + r -- its own row of S, so the softmax needs
//                 two lane swaps and no LDS;
//   O  += P V     P enters as the A operand as it lies: in MFMA step j lane
//                 group g supplies key 4 g + j (the sum over keys is the
//                 same in any order), and B takes V's rows in that order.
//
// The reduction dimensions are laid out for 16-byte LDS reads: in S^T lane
// group g covers dims [g D / 4, (g + 1) D / 4) (step s: dim g D / 4 + s),
// and the output column n of PV tile t is dim n D / 16 + t.  Q's operand
// values are loaded once per tile into registers.
template <unsigned D>
__global__ __launch_bounds__(kAttnThreads) void attention_mfma_kernel(
    KvGeometry g, const float* __restrict__ qkv, std::uint64_t stride, std::uint32_t m,
    const std::int32_t* __restrict__ positions,
    const std::int32_t* __restrict__ tables, std::uint32_t layer, std::uint32_t q_heads, std::uint32_t kv_heads,
    const AttentionTile* __restrict__ tiles, std::uint32_t splits, float scale, float* __restrict__ partials,
    float* __restrict__ out) {
    constexpr unsigned kChunk = kChunkKeys;   // keys per stage, 16 per wave
    constexpr unsigned LD = D + 4;            // padded LDS row (floats), keeps float4 alignment
    constexpr unsigned D4 = D / 4;
    constexpr unsigned kQuarter = D / 4;      // dims per lane group in S^T
    constexpr unsigned kDT = D / 16;          // 16-column tiles of the output
    __shared__ float qs[kTileVectors][LD];
    __shared__ float ks[kChunk][LD];
    __shared__ float vs[kChunk][LD];
    __shared__ std::uint64_t slot_addr[2][kChunk];   // K row of each token's slot (0: absent)
    __shared__ float wave_m[4][kTileVectors];
    __shared__ float wave_l[4][kTileVectors];

    const AttentionTile tile = tiles[blockIdx.x];
    if (!tile_ok(tile, m, q_heads, kv_heads)) return;
    const std::uint32_t split = blockIdx.y;
    const unsigned tid = threadIdx.x;
    const unsigned lane = tid & 63u;
    const unsigned wave = tid >> 6;
    const unsigned grp = lane >> 4;           // lane group
    const unsigned col = lane & 15u;          // query vector of this lane's S column
    const unsigned nq = tile.rows * tile.heads;
    const std::uint32_t kvh = static_cast<std::uint32_t>((static_cast<std::uint64_t>(tile.head) * kv_heads) / q_heads);
    const std::int32_t* table = tables + static_cast<std::uint64_t>(tile.row) * g.max_pages;

    const auto resolve = [&](std::uint32_t c, unsigned buf) __attribute__((always_inline)) {
        if (tid < kChunk) {   // page table lookup, once per token
            const std::uint64_t token = static_cast<std::uint64_t>(c) * kChunk + tid;
            const float* kp = kv_slot(g, table, layer, token, false);
            slot_addr[buf][tid] = reinterpret_cast<std::uint64_t>(kp);
        }
    };
    resolve(split, 0u);

    std::int64_t tmax = 0;
    for (unsigned r = 0; r < tile.rows; ++r) {
        const std::int64_t p = positions[tile.row + r];
        tmax = p + 1 > tmax ? p + 1 : tmax;
    }
    const std::uint32_t chunks = static_cast<std::uint32_t>((tmax + kChunk - 1) / kChunk);
    const std::uint32_t live = chunks < splits ? chunks : splits;
    if (split >= live) return;

    const bool col_active = col < nq;
    const std::int64_t col_pos = col_active ? positions[tile.row + col / tile.heads] : -1;

    for (unsigned idx = tid; idx < kTileVectors * D4; idx += kAttnThreads) {
        const unsigned v = idx / D4, d4 = idx % D4;
        float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
        if (v < nq) {
            const unsigned row = tile.row + v / tile.heads, head = tile.head + v % tile.heads;
            x = load4(qkv + static_cast<std::uint64_t>(row) * stride + static_cast<std::uint64_t>(head) * D + 4u * d4);
        }
        *reinterpret_cast<float4*>(&qs[v][4u * d4]) = x;
    }

    float mx = -__builtin_huge_valf();   // running maximum of vector `col`'s scores (this wave's keys)
    float lsum = 0.0f;
    float4v o[kDT];
#pragma unroll
    for (unsigned t = 0; t < kDT; ++t) o[t] = float4v{0.f, 0.f, 0.f, 0.f};

    const std::uint64_t v_after_k = static_cast<std::uint64_t>(g.page_tokens) * g.kv_width;
    constexpr unsigned kIters = kChunk * D4 / kAttnThreads;
    float4 kr[kIters], vr[kIters];
    const auto fetch = [&](unsigned buf) __attribute__((always_inline)) {
#pragma unroll
        for (unsigned it = 0; it < kIters; ++it) {
            const unsigned idx = tid + it * kAttnThreads;
            const unsigned t = idx / D4, d4 = idx % D4;
            const std::uint64_t addr = slot_addr[buf][t];
            kr[it] = make_float4(0.f, 0.f, 0.f, 0.f);
            vr[it] = kr[it];
            if (addr != 0u) {
                const float* kp = reinterpret_cast<const float*>(addr) + static_cast<std::uint64_t>(kvh) * D + 4u * d4;
                kr[it] = load4(kp);
                vr[it] = load4(kp + v_after_k);
            }
        }
    };
    __syncthreads();
    fetch(0u);
    // This lane's B operands of S^T: vector col, dims grp * D / 4 .. + D / 4.
    float4 qf[kQuarter / 4];
#pragma unroll
    for (unsigned i = 0; i < kQuarter / 4; ++i) qf[i] = *reinterpret_cast<const float4*>(&qs[col][grp * kQuarter + 4u * i]);

    unsigned buf = 0u;
    for (std::uint32_t c = split; c < chunks; c += splits, buf ^= 1u) {
        const std::int64_t c0 = static_cast<std::int64_t>(c) * kChunk;
        const std::uint32_t next = c + splits;
        __syncthreads();  // previous chunk's K and V are consumed
#pragma unroll
        for (unsigned it = 0; it < kIters; ++it) {
            const unsigned idx = tid + it * kAttnThreads;
            const unsigned t = idx / D4, d4 = idx % D4;
            *reinterpret_cast<float4*>(&ks[t][4u * d4]) = kr[it];
            *reinterpret_cast<float4*>(&vs[t][4u * d4]) = vr[it];
        }
        if (next < chunks) resolve(next, buf ^ 1u);
        __syncthreads();
        if (next < chunks) fetch(buf ^ 1u);   // in flight while chunk c computes

        // S^T for keys 16 wave .. + 15: lane (col, grp) ends with keys 4 grp + r.
        const float* krow = &ks[wave * 16u + col][grp * kQuarter];
        float4v st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (unsigned i = 0; i < kQuarter / 4; ++i) {
            const float4 a = *reinterpret_cast<const float4*>(krow + 4u * i);
            st = __builtin_amdgcn_mfma_f32_16x16x4f32(a.x, qf[i].x, st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_16x16x4f32(a.y, qf[i].y, st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_16x16x4f32(a.z, qf[i].z, st, 0, 0, 0);
            st = __builtin_amdgcn_mfma_f32_16x16x4f32(a.w, qf[i].w, st, 0, 0, 0);
        }
        // Online softmax of vector col over its four keys here (lane groups
        // hold the wave's other twelve).
        float sv[4];
        float cmax = -__builtin_huge_valf();
#pragma unroll
        for (unsigned r = 0; r < 4; ++r) {
            const std::int64_t key = c0 + wave * 16u + 4u * grp + r;
            sv[r] = col_active && key <= col_pos ? st[r] * scale : -__builtin_huge_valf();
            cmax = sv[r] > cmax ? sv[r] : cmax;
        }
        {
            float o1 = __shfl_xor(cmax, 16);
            cmax = o1 > cmax ? o1 : cmax;
            o1 = __shfl_xor(cmax, 32);
            cmax = o1 > cmax ? o1 : cmax;
        }
        const float m_new = cmax > mx ? cmax : mx;
        const bool none = m_new == -__builtin_huge_valf();
        const float alpha = none ? 1.0f : __expf(mx - m_new);
        float pv[4];
        float rs = 0.0f;
#pragma unroll
        for (unsigned r = 0; r < 4; ++r) {
            pv[r] = none || sv[r] == -__builtin_huge_valf() ? 0.0f : __expf(sv[r] - m_new);
            rs += pv[r];
        }
        rs += __shfl_xor(rs, 16);
        rs += __shfl_xor(rs, 32);
        lsum = lsum * alpha + rs;
        mx = m_new;
        // The output rows of this lane are vectors 4 grp + r: their alphas.
#pragma unroll
        for (unsigned r = 0; r < 4; ++r) {
            const float ar = __shfl(alpha, 4 * grp + r);
#pragma unroll
            for (unsigned t = 0; t < kDT; ++t) o[t][r] *= ar;
        }
        // O += P V: step j takes key 4 grp + j from lane group grp.
#pragma unroll
        for (unsigned j = 0; j < 4; ++j) {
            const float* vrow = &vs[wave * 16u + 4u * grp + j][col * kDT];
            float vb[kDT];
#pragma unroll
            for (unsigned t = 0; t < kDT; t += 4) {
                const float4 v4 = *reinterpret_cast<const float4*>(vrow + t);
                vb[t] = v4.x;
                vb[t + 1] = v4.y;
                vb[t + 2] = v4.z;
                vb[t + 3] = v4.w;
            }
#pragma unroll
            for (unsigned t = 0; t < kDT; ++t) o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(pv[j], vb[t], o[t], 0, 0, 0);
        }
    }

    // Merge the four waves: per vector M = max m_w, e_w = e^(m_w - M),
    // L = sum e_w l_w, O = sum e_w O_w.  The waves' O go through ks
    // ([w * 16 + vector][dim], the K stage is free after the last chunk).
    __syncthreads();
    if (grp == 0u) {
        wave_m[wave][col] = mx;
        wave_l[wave][col] = lsum;
    }
#pragma unroll
    for (unsigned t = 0; t < kDT; ++t) {
#pragma unroll
        for (unsigned r = 0; r < 4; ++r) ks[wave * 16u + 4u * grp + r][col * kDT + t] = o[t][r];
    }
    __syncthreads();
    for (unsigned idx = tid; idx < nq * D4; idx += kAttnThreads) {
        const unsigned v = idx / D4, d4 = idx % D4;
        float mw[4], big = -__builtin_huge_valf();
#pragma unroll
        for (unsigned w = 0; w < 4; ++w) {
            mw[w] = wave_m[w][v];
            big = mw[w] > big ? mw[w] : big;
        }
        float lt = 0.0f;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (unsigned w = 0; w < 4; ++w) {
            const float e = mw[w] == -__builtin_huge_valf() ? 0.0f : __expf(mw[w] - big);
            lt += e * wave_l[w][v];
            const float4 a = *reinterpret_cast<const float4*>(&ks[w * 16u + v][4u * d4]);
            acc.x += e * a.x;
            acc.y += e * a.y;
            acc.z += e * a.z;
            acc.w += e * a.w;
        }
        const unsigned row = tile.row + v / tile.heads, head = tile.head + v % tile.heads;
        // ks holds dims in the PV column order: column n of tile t is dim
        // n * kDT + t, i.e. LDS column c is dim c (n * kDT + t = c).
        if (live == 1u) {
            const float inv = 1.0f / lt;
            *reinterpret_cast<float4*>(out + static_cast<std::uint64_t>(row) * q_heads * D +
                                       static_cast<std::uint64_t>(head) * D + 4u * d4) =
                make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
        } else {
            float* part = partials + ((static_cast<std::uint64_t>(blockIdx.x) * splits + split) * kTileVectors + v) *
                                         (D + 4u);
            if (d4 == 0u) {
                part[0] = big;
                part[1] = lt;
            }
            *reinterpret_cast<float4*>(part + 4u + 4u * d4) = acc;
        }
    }
}

// Merges the live splits of each tile (those holding a chunk at or before
// the tile's last position): o = sum_s acc_s e^(m_s - M) / sum_s l_s
// e^(m_s - M), accumulated with a running M.  The positions and the first
// kBatch splits' partials are loaded together (dead splits' stale partials
// are read and ignored), so a decode tile merges in one round trip.
template <unsigned D>
__global__ __launch_bounds__(kAttnThreads) void attention_merge_kernel(const AttentionTile* __restrict__ tiles,
                                                                       std::uint32_t splits, std::uint32_t chunk,
                                                                       std::uint32_t m, std::uint32_t q_heads,
                                                                       std::uint32_t kv_heads,
                                                                       const std::int32_t* __restrict__ positions,
                                                                       const float* __restrict__ partials,
                                                                       float* __restrict__ out) {
    constexpr unsigned D4 = D / 4;
    constexpr unsigned kBatch = 16;   // splits whose partials are in flight at once
    const AttentionTile tile = tiles[blockIdx.x];
    if (!tile_ok(tile, m, q_heads, kv_heads)) return;
    const unsigned nq = tile.rows * tile.heads;
    const std::uint64_t part_step = static_cast<std::uint64_t>(kTileVectors) * (D + 4u);   // floats between splits
    const float* tile_part = partials + static_cast<std::uint64_t>(blockIdx.x) * splits * part_step;
    for (unsigned idx = threadIdx.x; idx < nq * D4; idx += kAttnThreads) {
        const unsigned v = idx / D4, d4 = idx % D4;
        const float* vbase = tile_part + static_cast<std::uint64_t>(v) * (D + 4u);
        float run_m = -__builtin_huge_valf(), run_l = 0.0f;
        float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
        std::uint32_t live = splits;
        for (std::uint32_t s0 = 0; s0 < live; s0 += kBatch) {
            float ms[kBatch], ls[kBatch];
            float4 as[kBatch];
#pragma unroll
            for (unsigned j = 0; j < kBatch; ++j) {
                // Every load is issued (a clamped split index): a guarded
                // load would wait at its join.
                const std::uint32_t sj = s0 + j < splits ? s0 + j : splits - 1u;
                const float* b = vbase + sj * part_step;
                ms[j] = b[0];
                ls[j] = b[1];
                as[j] = load4(b + 4u + 4u * d4);
            }
            if (s0 == 0) {
                std::int64_t tmax = 0;
                for (unsigned r = 0; r < tile.rows; ++r) {
                    const std::int64_t p = positions[tile.row + r];
                    tmax = p + 1 > tmax ? p + 1 : tmax;
                }
                const std::uint64_t chunks = (static_cast<std::uint64_t>(tmax) + chunk - 1u) / chunk;
                live = chunks < splits ? static_cast<std::uint32_t>(chunks) : splits;
                if (live <= 1u) return;   // the split kernel wrote this tile's output
            }
#pragma unroll
            for (unsigned j = 0; j < kBatch; ++j) {
                // A split with no key at or before this vector's position
                // holds m = -inf and adds nothing.
                if (s0 + j >= live || ms[j] == -__builtin_huge_valf()) continue;
                const float m_new = ms[j] > run_m ? ms[j] : run_m;
                const float c_old = __expf(run_m - m_new);   // 0 while run_m = -inf
                const float c_new = __expf(ms[j] - m_new);
                o.x = o.x * c_old + as[j].x * c_new;
                o.y = o.y * c_old + as[j].y * c_new;
                o.z = o.z * c_old + as[j].z * c_new;
                o.w = o.w * c_old + as[j].w * c_new;
                run_l = run_l * c_old + ls[j] * c_new;
                run_m = m_new;
            }
        }
        const float inv = 1.0f / run_l;
        const unsigned row = tile.row + v / tile.heads, head = tile.head + v % tile.heads;
        *reinterpret_cast<float4*>(out + static_cast<std::uint64_t>(row) * q_heads * D +
                                   static_cast<std::uint64_t>(head) * D + 4u * d4) =
            make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
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
            // Several rows of one sequence: 16 rows of one q head, the last
            // rows (the longest key ranges) first, so the longest tiles start
            // first and the short ones fill the end of the grid (512-row
            // prompt at 7B heads: 76 -> 49 us).
            for (std::uint32_t b = (n + kTileVectors - 1u) / kTileVectors; b-- > 0;) {
                const std::uint32_t r = b * kTileVectors;
                for (std::uint32_t h = 0; h < q_heads; ++h) {
                    push(row + r, n - r < kTileVectors ? n - r : kTileVectors, h, 1u);
                }
            }
        }
        row += n;
    }
    return count;
}

std::uint32_t attention_splits(std::uint32_t tiles, std::uint64_t max_tokens, std::uint32_t m) {
    (void)m;
    const std::uint64_t chunks = (max_tokens + kChunkKeys - 1) / kChunkKeys;
    if (tiles == 0 || chunks <= 1) return 1;
    // About 512 workgroups (two per CU on 256 CUs).
    const std::uint64_t want = (512u + tiles - 1) / tiles;
    const std::uint64_t s = want < chunks ? want : chunks;
    return static_cast<std::uint32_t>(s < kMaxSplits ? s : kMaxSplits);
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
    const KvGeometry g = kv;
    const float scale = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(head_dim)));
    const dim3 grid(tile_count, splits);
#define AIR_ATTENTION_MFMA(D)                                                                                    \
    hipLaunchKernelGGL(attention_mfma_kernel<D>, grid, dim3(kAttnThreads), 0, stream, g, qkv, stride, m, positions, \
                       tables, layer, q_heads, kv_heads, tiles, splits, scale, partials, out)
#define AIR_ATTENTION_MERGE(D)                                                                                   \
    hipLaunchKernelGGL(attention_merge_kernel<D>, dim3(tile_count), dim3(kAttnThreads), 0, stream, tiles, splits, \
                       kChunkKeys, m, q_heads, kv_heads, positions, partials, out)
    if (head_dim == 128u) {
        AIR_ATTENTION_MFMA(128);
        if (splits > 1u) AIR_ATTENTION_MERGE(128);
    } else if (head_dim == 64u) {
        AIR_ATTENTION_MFMA(64);
        if (splits > 1u) AIR_ATTENTION_MERGE(64);
    } else {
        return hipErrorInvalidValue;
    }
#undef AIR_ATTENTION_MFMA
#undef AIR_ATTENTION_MERGE
    return hipGetLastError();
}

} // namespace air_hip

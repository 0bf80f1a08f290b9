// air_hip_kernels.hpp -- host-side launchers of the HIP kernels (internal).
#pragma once

#include "air_hip_kv.hpp"

#include <hip/hip_runtime.h>
#include <cstdint>

namespace air_hip {

struct SplitEpilogue;  // below, with the step kernels

// Resident planes of one matrix in the wavefront tile layout.
struct TilePlanes {
    int type{0};
    std::uint64_t k{0}, n{0};
    std::uint32_t nt{0};   // 16-row tiles
    std::uint32_t kt{0};   // k tiles
    std::uint64_t kp{0};   // padded k = kt * tile_k
    void* codes{nullptr};
    void* scales{nullptr};
    // Power-of-two factors of the prefill GEMM: dequantized weights are
    // formed in f16 as w * prefill_scale, outputs multiplied by prefill_unscale.
    float prefill_scale{1.0f};
    float prefill_unscale{1.0f};
};

// Canonical GGUF bytes (device) -> tile planes.
hipError_t launch_repack(const TilePlanes& planes, const std::uint8_t* canonical, hipStream_t stream);
// Tile planes -> f32 [n][k] (device), bit-exact decode.
hipError_t launch_dequantize_tiles(const TilePlanes& planes, float* out, hipStream_t stream);
// Canonical GGUF bytes (device) -> f32, bit-exact decode (every type of
// canonical_block).
hipError_t launch_dequantize_canonical(int type, const std::uint8_t* canonical,
                                       std::uint64_t elements, float* out, hipStream_t stream);
// Q5_0 blocks (device) -> Q8_0 blocks of the same values.
hipError_t launch_q5_0_to_q8_0(const std::uint8_t* q5_0, std::uint64_t blocks, std::uint8_t* q8_0, hipStream_t stream);
// Linears over dense rows w[n][k] stored as `storage` (kF32, or the f16 /
// bf16 bits of kF16 / kBF16; k a multiple of 32, x and y 16-byte aligned):
// y[m][n] = sum_k x[m][k] w[n][k] (+ bias[n]).
// Dense linears on the matrix cores (linear_dense_mfma.hip): F16, BF16 and
// Q6_K storage, any m (one launch per 64 rows).  A shape field of 0 is the
// planner's choice.
struct DenseMfmaShape {
    std::uint32_t tile_n{0};   // 16-row weight tiles per workgroup: 1, 2 or 4
    std::uint32_t waves{0};    // waves splitting K (1..8)
    std::uint32_t depth{0};    // weight steps per wave ring: 2 or 4
};
// path 0 = automatic (the matrix-core kernel for 2..64 rows), 1 = the
// matrix-core kernel wherever it applies, 2 = the FMA kernels (dense_rows /
// dense_gemm / q6k_gemv).
struct DenseTuning {
    std::uint32_t path{0};
    DenseMfmaShape shape{};
};
// Activation rows per launch of the matrix-core kernel.
std::uint32_t dense_mfma_rows(int storage);
DenseMfmaShape plan_dense_mfma(int storage, std::uint64_t k, std::uint64_t n, std::uint32_t m,
                               const DenseMfmaShape& tuning);
bool dense_mfma_supported(int storage, std::uint64_t k);
// Whether a linear of m rows over `storage` runs on the matrix-core kernel.
bool dense_mfma_route(int storage, std::uint64_t k, std::uint64_t n, std::uint32_t m, const DenseTuning& tuning);
hipError_t launch_dense_mfma(const void* w, int storage, std::uint64_t k, std::uint64_t n, const float* x,
                             const float* bias, float* y, std::uint32_t m, const DenseMfmaShape& tuning,
                             hipStream_t stream);
hipError_t launch_dense_linear(const void* w, int storage, std::uint64_t k, std::uint64_t n, const float* x,
                               const float* bias, float* y, std::uint32_t m, hipStream_t stream,
                               const DenseTuning& tuning = DenseTuning{});
// out[i][k] = w[rows[i]][k], decoded exactly, for rows in [0, n); other ids
// leave out[i] as is.
// XOR checksum of `bytes` (a multiple of 16) of device memory: one word per
// chunk stored in `sink` (sink_words >= 1; the caller zeroes it and XORs
// its words), read once with the decode GEMV's access pattern -- the
// streaming floor of a launch of that size.
hipError_t launch_stream_read(const void* data, std::uint64_t bytes, unsigned* sink, std::uint64_t sink_words,
                              hipStream_t stream);
// Resident bytes of a dense matrix stored as `storage` (kQ6_K: 208-byte
// super-block records plus 2 bytes of d each; 0 when k does not fit).
std::uint64_t dense_resident_bytes(int storage, std::uint64_t k, std::uint64_t n);
// Waves per workgroup of the M = 1 Q6_K GEMV (one 16-row tile per
// workgroup); `waves` != 0 overrides the planner (1..16).
std::uint32_t q6k_gemv_waves(std::uint64_t k, std::uint64_t n, std::uint32_t waves);
// Its launch: waves, super-blocks per work unit (1, 2), units in flight per
// wave (1, 2); sweeps override them through DenseTuning's shape (waves;
// tile_n = 2 for two super-blocks per unit; depth = 4 for one unit in
// flight, 2 for two).
struct Q6kGemvPlan {
    std::uint32_t waves{1};
    std::uint32_t units{1};
    std::uint32_t depth{2};
};
Q6kGemvPlan plan_q6k_gemv(std::uint64_t k, std::uint64_t n, const DenseMfmaShape& tuning);
// Canonical Q6_K blocks (device) -> 208-byte records and the d plane.
hipError_t launch_q6k_records(const void* canonical, std::uint64_t blocks, void* records, hipStream_t stream);
// Dense matrix -> f32 [n][k], bit-exact decode.
hipError_t launch_dense_dequantize(const void* w, int storage, std::uint64_t k, std::uint64_t n, float* out,
                                   hipStream_t stream);
hipError_t launch_dense_rows(const void* w, int storage, std::uint64_t k, std::uint64_t n, const std::int32_t* rows,
                             std::uint32_t count, float* out, hipStream_t stream);

// Workspace of the split activations for `m` rows of width kp (padded).
struct SplitWorkspace {
    void* xs{nullptr};          // [kp/32][mp/16][2][64][8] f16  (hi, lo), scaled per (block, row)
    float* block_sums{nullptr}; // [kp/32][mp] f32  sum of the unscaled x of each 32-block
    float* inv_scale{nullptr};  // [kp/32][mp] f32  inverse power-of-two scale of each (block, row)
};

// Launch-shape override of the decode linear (0 = automatic choice).
struct DecodeTuning {
    std::uint32_t rows_per_wave{0};   // 16-row tiles per wave: 1, 2 or 4
    std::uint32_t waves_per_group{0}; // waves splitting K inside a workgroup
    std::uint32_t k_splits{0};        // workgroups splitting K (fused path)
    std::uint32_t pair_split{0};      // M = 1 GEMV pair split: 0 automatic, 1 never, 2 always (where it applies)
    std::uint32_t units_per_chunk{0}; // M = 1 GEMV work units per 16-block chunk: 0 automatic, 1 or 2
    std::uint32_t depth{0};           // M = 1 GEMV chunk buffers per wave: 0 automatic, 1 or 2
};
std::uint64_t split_workspace_bytes(std::uint64_t kp, std::uint32_t m);
SplitWorkspace carve_split_workspace(void* base, std::uint64_t kp, std::uint32_t m);

// Activation split: x [m][k] f32 -> f16 hi/lo tiles scaled per (32-block, row)
// by a power of two, block sums and inverse scales.  Rows m..mp-1 are zeroed.
hipError_t launch_split_activations(const float* x, std::uint32_t m, std::uint64_t k,
                                    std::uint64_t kp, const SplitWorkspace& ws, hipStream_t stream);

// Decode linear over the split activations: y[m][n] (+ bias[n]).
hipError_t launch_decode_linear(const TilePlanes& planes, const SplitWorkspace& ws,
                                const float* bias, float* y, std::uint32_t m,
                                const DecodeTuning& tuning, hipStream_t stream);

// Single-launch decode linear for up to kFusedMaxRows rows: reads x [m][k]
// f32 directly and splits it in registers (no workspace).
constexpr std::uint32_t kFusedMaxRows = 16;
struct FusedShape {
    std::uint32_t rows_per_wave{1};
    std::uint32_t waves_per_group{1};
    std::uint32_t k_splits{1};
    std::uint32_t groups{0};          // row-tile groups (grid x)
};
FusedShape plan_decode_fused(const TilePlanes& planes, std::uint32_t m, const DecodeTuning& tuning);
// Device bytes of the cross-workgroup partials of a K-split launch (0 if none);
// the launch also needs `groups` zero-initialised uint32 counters, which it
// leaves at zero.
std::uint64_t fused_split_workspace_bytes(const FusedShape& shape);
hipError_t launch_decode_fused(const TilePlanes& planes, const float* x, const float* bias, float* y,
                               std::uint32_t m, const FusedShape& shape, void* partials,
                               std::uint32_t* counters, hipStream_t stream);

// M = 1 decode linear (matrix-vector product) with block-diagonal activation
// operands and whole-chunk prefetch.
struct GemvShape {
    std::uint32_t rows_per_wave{1};
    std::uint32_t waves_per_group{1};
    std::uint32_t depth{2};           // chunk buffers per wave (1 or 2)
    std::uint32_t units_per_chunk{1}; // work units per 16-block chunk (1, or 2 for one-tile waves)
    // Two workgroups per row tile, each half the work units, meeting through
    // one 64-bit slot per output row (waves_per_group is per workgroup).
    std::uint32_t pair_split{0};
};
// Rows a pair-split GEMV can address: the slot array holds this many 64-bit
// words, zero between launches.
constexpr std::uint64_t kGemvPairSlots = 8192;
GemvShape plan_decode_gemv(const TilePlanes& planes, const DecodeTuning& tuning);
hipError_t launch_decode_gemv(const TilePlanes& planes, const float* x, const float* bias, float* y,
                              const GemvShape& shape, std::uint64_t* pair_slots, hipStream_t stream);
// The M = 1 linear with the step's element-wise neighbours fused in:
// norm_weight != null RMS-normalises x first (eps); epilogue 0 stores
// y = W x + b, 1 adds it to y (residual), 2 writes silu(g) * u of a fused
// gate|up matrix (y has N / 2 entries).
struct GemvFusion {
    const float* norm_weight{nullptr};
    double eps{0.0};
    int epilogue{0};
};
GemvShape plan_decode_gemv_fused(const TilePlanes& planes, const DecodeTuning& tuning, int epilogue);
hipError_t launch_decode_gemv_fused(const TilePlanes& planes, const float* x, const float* bias, float* y,
                                    const GemvShape& shape, const GemvFusion& fusion, std::uint64_t* pair_slots,
                                    hipStream_t stream);

// Prefill linear on f16 MFMA (M = 1..4096; planned for M >= 65).
struct PrefillTuning {
    std::uint32_t tile_m{0};   // 16-row activation tiles per wave: 4 or 8 (0 = automatic)
    std::uint32_t tile_n{0};   // 16-row weight tiles per wave: 2 or 4
    std::uint32_t k_splits{0}; // workgroups splitting K (0 = automatic)
    std::uint32_t prefetch{0}; // weight prefetch distance in steps: 1 or 2 (8x4 tile only)
    // Operand staging: 0 automatic, 1 registers (prefill_gemm_kernel), 2..4
    // an LDS ring of that many 64-k steps (prefill_lds_kernel; Q8_0, 8x4 and
    // 4x2 tiles); 0x12 / 0x13 activations alone through an LDS ring of 2 / 3
    // stages with the weights in registers (prefill_hyb_kernel; any format,
    // 8x4, 8x2 and 4x2 tiles).
    std::uint32_t lds_stages{0};
    std::uint32_t cus{256};        // compute units of the device (round sizes)
    std::uint32_t rem_splits{0};   // remainder launch K split: 0 automatic, 1 none, n splits
};
struct PrefillShape {
    std::uint32_t tile_m{8};
    std::uint32_t tile_n{4};
    std::uint32_t prefetch{1};
    std::uint32_t lds_stages{0};   // 0: registers; 2..4: LDS ring stages
    std::uint32_t hybrid{0};       // 2, 3: activation-only LDS ring (prefill_hyb_kernel)
    // Rows past the first `groups` weight groups (a grid that would end in a
    // mostly empty round of workgroups) run as a second launch on the 4x2
    // tile: rem_groups groups of 128 rows from row tile 4 * tile_n * groups.
    std::uint32_t rem_groups{0};
    std::uint32_t rem_m_tiles{0};
    // The remainder launch's K split (partials of its columns only, summed
    // in split order by a column reduction).
    std::uint32_t rem_splits{1};
    std::uint32_t rem_steps_per_split{0};
    std::uint32_t m_tiles{0};
    std::uint32_t groups{0};
    std::uint32_t steps{0};
    std::uint32_t steps_per_split{0};
    std::uint32_t splits{1};
};
PrefillShape plan_prefill(const TilePlanes& planes, std::uint32_t m, const PrefillTuning& tuning);
// Workspace of one prefill linear: f16 activations, row scales and (with a K
// split) the f32 partials.
// Padded f16 row stride and padded row count of the prefill operand, and
// the byte offset of the K-split partials after the operand in the workspace.
std::uint64_t prefill_ldx(std::uint64_t k);
std::uint32_t prefill_rows_padded(std::uint32_t m);
std::uint64_t prefill_partials_offset(std::uint64_t k, std::uint32_t m);
std::uint64_t prefill_workspace_bytes(std::uint64_t k, std::uint32_t m, const PrefillShape& shape, std::uint64_t n);
// With `epilogue`, a K-split launch's reduction applies it instead of
// writing y (the caller checks split_epilogue_fits on the partials, which
// follow the operand in the workspace).
hipError_t launch_prefill_linear(const TilePlanes& planes, const float* x, const float* bias, float* y,
                                 std::uint32_t m, const PrefillShape& shape, void* workspace, hipStream_t stream,
                                 bool converted = false, const SplitEpilogue* epilogue = nullptr);
// y[m][n] = sum over splits of partials[s][m][n] (in split order) + bias[n].
hipError_t launch_split_reduce(const float* partials, std::uint32_t splits, std::uint32_t m, std::uint64_t n,
                               const float* bias, float* y, hipStream_t stream);

// Activation split for the skinny kernel: the same hi/lo tile layout, but one
// power-of-two scale per row (inv_scale[m], m < mp) and block sums of the
// scaled values (block_sums[b][m]).
hipError_t launch_split_activations_rows(const float* x, std::uint32_t m, std::uint64_t k, std::uint64_t kp,
                                         const SplitWorkspace& ws, hipStream_t stream);

// Skinny decode linear (M = 1..64) over split activations: activations staged
// once per workgroup in LDS, exact weight codes streamed per wave, optional K
// split with a deterministic reduction.
struct SkinnyShape {
    std::uint32_t mt{1};       // 16-row activation tiles (all M rows)
    std::uint32_t tile_n{1};   // 16-row weight tiles per wave (1 or 2)
    std::uint32_t groups{0};
    std::uint32_t steps{0};
    std::uint32_t steps_per_split{0};
    std::uint32_t splits{1};
    std::uint32_t lds_stages{0};  // Q8_0 from split activations: stages of the LDS pipeline (0 = registers)
    std::uint32_t waves{4};       // waves per workgroup: 4, or 8 on the LDS pipeline
};
// lds_stages: 0 automatic, 1 the register pipeline, 2..4 the LDS ring
// (Q8_0 from split activations; other formats and f32 inputs ignore it).
// waves: 0 or 4, or 8 (the LDS pipeline with two stages and two or four
// activation tiles; otherwise 4).
SkinnyShape plan_skinny(const TilePlanes& planes, std::uint32_t m, std::uint32_t tile_n, std::uint32_t k_splits,
                        std::uint32_t lds_stages = 0, std::uint32_t waves = 0);
std::uint64_t skinny_partials_bytes(const SkinnyShape& shape, std::uint32_t m, std::uint64_t n);
// With `epilogue` (only when shape.splits > 1 and split_epilogue_fits), the
// split reduction applies it and y is not written.  Without one, a non-null
// `chain` (chain_slot_bytes(shape.splits, m, n) of slots, zero between
// launches) combines a K split inside the kernel instead of a reduction
// launch, with the reduction's bits.
hipError_t launch_skinny_linear(const TilePlanes& planes, const SplitWorkspace& ws, const float* bias, float* y,
                                std::uint32_t m, const SkinnyShape& shape, float* partials, hipStream_t stream,
                                const SplitEpilogue* epilogue = nullptr, std::uint64_t* chain = nullptr);
// The same linear straight from f32 activations x [m][k]: each workgroup
// splits the activations it stages (one power-of-two scale per (row,
// 32-block)), so no split launch and no activation workspace.
hipError_t launch_skinny_linear_x(const TilePlanes& planes, const float* x, const float* bias, float* y,
                                  std::uint32_t m, const SkinnyShape& shape, float* partials, hipStream_t stream,
                                  const SplitEpilogue* epilogue = nullptr, std::uint64_t* chain = nullptr);
// Bytes of the in-kernel K-split chain's slots: splits - 1 words per output.
constexpr std::uint64_t chain_slot_bytes(std::uint32_t splits, std::uint32_t m, std::uint64_t n) {
    return splits > 1u ? static_cast<std::uint64_t>(splits - 1u) * m * n * 8u : 0u;
}

// Decode linear (M = 2..64) with K split over the waves of a workgroup
// (linear_wsplit.hip): TN weight tiles per workgroup, every activation row,
// `waves` waves each streaming a contiguous K range with `depth` - 1 steps of
// weight codes in flight; K split over workgroups only for narrow matrices.
struct WsplitShape {
    std::uint32_t mt{1};
    std::uint32_t tile_n{1};     // 16-row weight tiles per workgroup: 1, 2 or 4
    std::uint32_t waves{1};      // waves per workgroup (1..8)
    std::uint32_t depth{4};      // weight-code steps per wave ring: 2 or 4
    std::uint32_t groups{0};
    std::uint32_t steps{0};
    std::uint32_t steps_per_split{0};
    std::uint32_t splits{1};
    std::uint32_t split_x{0};    // 1: activations split once into the workspace first
};
// 0 = automatic choice for each field (split_x: 1 = split into the
// workspace first, 2 = in each wave).
struct WsplitTuning {
    std::uint32_t tile_n{0};
    std::uint32_t waves{0};
    std::uint32_t depth{0};
    std::uint32_t k_splits{0};
    std::uint32_t split_x{0};
};
// Whether the automatic route takes the wave-split kernel for m rows.
bool wsplit_preferred(const TilePlanes& planes, std::uint32_t m);
WsplitShape plan_wsplit(const TilePlanes& planes, std::uint32_t m, const WsplitTuning& tuning);
std::uint64_t wsplit_partials_bytes(const WsplitShape& shape, std::uint32_t m, std::uint64_t n);
// x: f32 rows [m][k] (split in the kernel) when ws is null, else the
// row-scaled split in ws (split_rows_kernel's layout).
hipError_t launch_wsplit_linear(const TilePlanes& planes, const float* x, const SplitWorkspace* ws, const float* bias,
                                float* y, std::uint32_t m, const WsplitShape& shape, float* partials,
                                hipStream_t stream, const SplitEpilogue* epilogue = nullptr,
                                std::uint64_t* chain = nullptr);

// ---- the Qwen2 step around the linears ----------------------------------

// Paged fp32 KV pool: page p holds [layer][2 (K, V)][page_tokens][kv_width]
// floats, in one allocation or in a table of chunks (air_hip_kv.hpp).
using KvLayout = KvGeometry;
hipError_t launch_matrix_rows(const TilePlanes& planes, const std::int32_t* rows, std::uint32_t m, float* out,
                              hipStream_t stream);
hipError_t launch_rms_norm(const float* x, const float* w, float* out, std::uint32_t m, std::uint64_t n, double eps,
                           hipStream_t stream);
// x += y (m x n), then out = rms_norm(x) * w; out must not alias x.
hipError_t launch_add_rms_norm(float* x, const float* y, const float* w, float* out, std::uint32_t m, std::uint64_t n,
                               double eps, hipStream_t stream);
hipError_t launch_rope(float* qkv, std::uint64_t stride, std::uint32_t m, const std::int32_t* positions,
                       std::uint32_t q_heads, std::uint32_t kv_heads, std::uint32_t head_dim, std::uint32_t rope_dims,
                       const void* table, std::uint64_t table_positions, hipStream_t stream);
hipError_t launch_kv_append(const KvLayout& kv, const float* qkv, std::uint64_t stride, std::uint64_t q_width,
                            std::uint32_t m, const std::int32_t* positions, const std::int32_t* tables,
                            std::uint32_t layer, hipStream_t stream);
// launch_rope then launch_kv_append in one launch (same results).
hipError_t launch_rope_kv_append(const KvLayout& kv, float* qkv, std::uint64_t stride, std::uint64_t q_width,
                                 std::uint32_t m, const std::int32_t* positions, const std::int32_t* tables,
                                 std::uint32_t layer, std::uint32_t q_heads, std::uint32_t kv_heads,
                                 std::uint32_t head_dim, std::uint32_t rope_dims, const void* table,
                                 std::uint64_t table_positions, hipStream_t stream);
hipError_t launch_attention(const KvLayout& kv, const float* qkv, std::uint64_t stride, std::uint32_t m,
                            const std::int32_t* positions, const std::int32_t* tables, std::uint32_t layer,
                            std::uint32_t q_heads, std::uint32_t kv_heads, std::uint32_t head_dim, double* scratch,
                            std::uint64_t score_stride, float* out, hipStream_t stream);
// Tiled online-softmax attention (attention.hip).  A tile is up to 16 query
// vectors of one sequence and one KV head: rows [row, row + rows) x q heads
// [head, head + heads), rows * heads <= 16.
struct AttentionTile {
    std::uint32_t row, rows, head, heads;
};
// Tiles of a step whose rows form `runs` consecutive runs of one sequence
// each (run_rows[i] rows): a one-row run gives one tile per KV head (its
// grouped q heads), a longer run tiles of 16 rows per q head.  Writes up to
// `capacity` tiles (tiles may be null) and returns the count.
std::uint32_t make_attention_tiles(const std::uint32_t* run_rows, std::uint32_t runs, std::uint32_t q_heads,
                                   std::uint32_t kv_heads, AttentionTile* tiles, std::uint32_t capacity);
// Workgroups per tile over the key range of a step of m rows (1 = no merge).
std::uint32_t attention_splits(std::uint32_t tiles, std::uint64_t max_tokens, std::uint32_t m);
std::uint64_t attention_partials_bytes(std::uint32_t tiles, std::uint32_t splits, std::uint32_t head_dim);
// head_dim 64 or 128.  tiles: device array; partials: attention_partials_bytes.
// A tile outside the m rows or q heads, or with more than 16 vectors or heads
// of two KV heads, is skipped by the kernel.
hipError_t launch_attention_tiles(const KvLayout& kv, const float* qkv, std::uint64_t stride, std::uint32_t m,
                                  const std::int32_t* positions, const std::int32_t* tables, std::uint32_t layer,
                                  std::uint32_t q_heads, std::uint32_t kv_heads, std::uint32_t head_dim,
                                  const AttentionTile* tiles, std::uint32_t tile_count, std::uint32_t splits,
                                  float* partials, float* out, hipStream_t stream);
hipError_t launch_silu_mul(const float* gate_up, float* out, std::uint32_t m, std::uint64_t ffn, hipStream_t stream);
// The RMSNorm (with the residual add first when y is given) and the SwiGLU,
// each also writing its output as the next prefill linear's operand
// (xh [mp][ldx] f16 rows scaled by a power of two per row, row_inv [mp]),
// bit-identical to that linear converting the f32 output itself.
bool prefill_norm_fits(std::uint64_t n, std::uint64_t ldx);
hipError_t launch_rms_norm_prefill(float* x, const float* y, const float* w, float* out, std::uint32_t m,
                                   std::uint64_t n, double eps, _Float16* xh, float* row_inv, std::uint32_t mp,
                                   std::uint64_t ldx, hipStream_t stream);
bool silu_prefill_fits(std::uint64_t ffn, std::uint64_t ldx);
hipError_t launch_silu_mul_prefill(const float* gate_up, float* out, std::uint32_t m, std::uint64_t ffn, _Float16* xh,
                                   float* row_inv, std::uint32_t mp, std::uint64_t ldx, hipStream_t stream);

// The step's element-wise work after a K-split linear, run by the launch
// that sums the split partials (partials[s][m][n]) instead of a plain
// reduction into y -- bit-identical to the reduction followed by the
// separate kernel:
//   kEpilogueSwiglu: out [m][n/2] = silu(g) * u, g and u the reduced
//     columns i and n/2 + i (launch_silu_mul);
//   kEpilogueResidual: out [m][n] += the reduced rows, then with
//     norm_weight, norm_out = rms_norm(out) * norm_weight (launch_add_rms_norm;
//     norm_out must not alias out);
//     With `load`, norm_out is also split into that activation workspace
//     as launch_split_activations_rows splits it (kp = 32 * load_blocks), so
//     the next linear on norm_out needs no split launch;
//   kEpilogueRopeKv: out [m][n] = the reduced q|k|v rows with RoPE applied
//     and k, v appended to the KV pool (launch_rope_kv_append over rows of
//     stride n).
constexpr int kEpilogueResidual = 1;
constexpr int kEpilogueSwiglu = 2;
constexpr int kEpilogueRopeKv = 3;
struct RopeKvArgs {
    KvLayout kv;
    const std::int32_t* positions{nullptr};
    const std::int32_t* tables{nullptr};
    std::uint32_t layer{0};
    std::uint32_t q_heads{0};
    std::uint32_t kv_heads{0};
    std::uint32_t head_dim{0};
    std::uint32_t rope_dims{0};
    const void* table{nullptr};
    std::uint64_t table_positions{0};
};
// The f16 operand area of a prefill linear (xh [mp][ldx], row_inv [mp]).
struct PrefillOperandArgs {
    _Float16* xh{nullptr};
    float* row_inv{nullptr};
    std::uint32_t mp{0};
    std::uint64_t ldx{0};
};
struct SplitEpilogue {
    int kind{0};
    float* out{nullptr};
    const float* norm_weight{nullptr};
    float* norm_out{nullptr};
    double eps{0.0};
    const RopeKvArgs* rope{nullptr};
    const SplitWorkspace* load{nullptr};
    std::uint32_t load_blocks{0};
    // kEpilogueResidual with a norm: norm_out also converted into this
    // prefill operand (as launch_rms_norm_prefill converts it).
    const PrefillOperandArgs* prefill{nullptr};
};
// Whether the reduction can carry `e` for this shape (alignment, widths).
bool split_epilogue_fits(const SplitEpilogue& e, const float* partials, const float* bias, std::uint32_t m,
                         std::uint64_t n);
hipError_t launch_split_epilogue(const float* partials, std::uint32_t splits, std::uint32_t m, std::uint64_t n,
                                 const float* bias, const SplitEpilogue& e, hipStream_t stream);
hipError_t launch_add(float* x, const float* y, std::uint64_t count, hipStream_t stream);
// Greedy selection in two passes (slices of a row, then each row's slices);
// scratch holds argmax_scratch_bytes(m, n) bytes.
std::uint64_t argmax_scratch_bytes(std::uint32_t m, std::uint64_t n);
hipError_t launch_argmax(const float* logits, std::uint32_t m, std::uint64_t n, std::int32_t* out, void* scratch,
                         hipStream_t stream);

// Sets planes.prefill_scale / prefill_unscale from the largest dequantized
// magnitude of the resident matrix (synchronous; `bound_scratch` is one
// device uint32).
// The prefill GEMM over dense storage (planes.type kF16 / kBF16 / kQ6_K,
// planes.codes the rows or records, planes.kt = k): its weight exponent.
hipError_t compute_dense_prefill_scale(TilePlanes& planes, std::uint32_t* bound_scratch, hipStream_t stream);
hipError_t compute_prefill_scale(TilePlanes& planes, std::uint32_t* bound_scratch, hipStream_t stream);

} // namespace air_hip

/*
 * air_hip.h -- C ABI of the MI355X quantized linear engine (libair_hip.so).
 *
 * The engine executes AIR's quantized linear contract -- a GGUF Q8_0 / Q4_0 /
 * Q4_K weight matrix with GGML dims {K, N} applied to M f32 activation rows --
 * on one AMD Instinct MI355X (gfx950) with hand-written HIP kernels.  It is
 * the device half of a HIP executor that plugs in behind AIR's executor
 * contract (src/runtime/backend.hpp:97-145) the way CudaExecutor does.
 *
 * Conventions
 *   - Plain C: no C++ or HIP types cross this boundary.  Streams are passed
 *     as `void*` holding a hipStream_t (NULL = the legacy default stream).
 *   - Every function returns an air_hip_status; on failure
 *     air_hip_last_error() holds a message for the calling thread.  Nothing
 *     throws across the boundary (src/cuda/cuda_backend.cu:1180-1182 checks
 *     every launch the same way).
 *   - Activation and output pointers are non-owning device pointers; matrices
 *     and contexts are owned by the library and released explicitly.
 *   - Results are deterministic: a fixed launch configuration sums in a fixed
 *     order.
 *
 * Type ids are GGML/GGUF on-disk tensor type ids (the reference's
 * TensorDescriptor::format_type, src/formats/gguf/gguf_format.cpp:24-63).
 */
#ifndef AIR_HIP_H
#define AIR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AIR_HIP_ABI_VERSION 2

/* Mirrors air::ErrorCode (include/air/status.hpp:8-17). */
typedef enum air_hip_status {
    AIR_HIP_OK = 0,
    AIR_HIP_INVALID_ARGUMENT = 1,
    AIR_HIP_INVALID_STATE = 2,
    AIR_HIP_IO_ERROR = 3,
    AIR_HIP_CANCELLED = 4,
    AIR_HIP_DATA_ERROR = 5,
    AIR_HIP_UNSUPPORTED = 6,
    AIR_HIP_INTERNAL_ERROR = 7
} air_hip_status;

/* GGML type ids this engine executes: every encoding the reference's
 * decode_element takes (cuda_backend.cu:241-344).  Q8_0, Q4_0 and Q4_K run
 * on their resident tile formats; Q5_0 is rewritten exactly as Q8_0 (same
 * scale, code q - 16) and runs as Q8_0; F32, F16, BF16 and Q6_K keep their
 * own rows (Q6_K its 210-byte super-blocks padded to 212 bytes: 0.83 bytes
 * per weight) and run on plain f32 FMA kernels that decode as they load. */
enum {
    AIR_HIP_TYPE_F32 = 0,
    AIR_HIP_TYPE_F16 = 1,
    AIR_HIP_TYPE_Q4_0 = 2,
    AIR_HIP_TYPE_Q5_0 = 6,
    AIR_HIP_TYPE_Q8_0 = 8,
    AIR_HIP_TYPE_Q4_K = 12,
    AIR_HIP_TYPE_Q6_K = 14,
    AIR_HIP_TYPE_BF16 = 30
};

/* Linear tactics: the HIP members of AIR's QuantizedLinearExecutionKind
 * (include/air/execution.hpp:35-41).
 *   DECODE  exact integer codes as f16 MFMA operands, activations split into
 *           f16 hi+lo parts with a per-row power-of-two scale, per-block f32
 *           scale epilogue.  M = 1..64.  Relative L2 error vs the double
 *           oracle ~1e-6 (gate 1e-4).  Replaces specialized_matvec_kernel /
 *           specialized_matmul_batch_reuse_kernel (cuda_backend.cu:501-606).
 *   PREFILL weights dequantised to f16 in registers (exact codes times an
 *           f16 block scale), activations rounded to f16 after a per-row
 *           power-of-two scale, f16 MFMA with f32 accumulation, for
 *           prefill-sized M (any M >= 1; gate 1e-2, measured ~3e-4).
 *           Replaces the dense-f32 dequantise + GEMM tactic
 *           (cuda_backend.cu:375-382,1971-1992).
 *   AUTO    DECODE for M <= 64, PREFILL above. */
enum {
    AIR_HIP_LINEAR_AUTO = 0,
    AIR_HIP_LINEAR_DECODE = 1,
    AIR_HIP_LINEAR_PREFILL = 2
};

#define AIR_HIP_MAX_DECODE_ROWS 64u

typedef struct air_hip_context air_hip_context;
typedef struct air_hip_matrix air_hip_matrix;

typedef struct air_hip_matrix_desc {
    int32_t type;               /* GGML type id */
    int32_t device;             /* device ordinal holding the planes */
    uint64_t k;                 /* input width (GGML dim 0) */
    uint64_t n;                 /* output width (GGML dim 1) */
    uint64_t canonical_bytes;   /* exact GGUF storage size */
    uint64_t resident_bytes;    /* device bytes of the repacked planes */
} air_hip_matrix_desc;

/* Hot-path evidence counters, the HIP analogue of CudaExecutionStats
 * (include/air/cuda.hpp:19-54).  Cumulative per context; relaxed atomics. */
typedef struct air_hip_stats {
    uint64_t resident_matrix_bytes;
    uint64_t workspace_bytes;
    uint64_t host_to_device_bytes;
    uint64_t prepared_matrices;
    uint64_t decode_linear_calls;
    uint64_t prefill_linear_calls;
    uint64_t decode_rows;
    uint64_t prefill_rows;
    /* Bumped whenever the context grows a workspace or scratch buffer:
     * launches captured into a HIP graph use the current buffers while it is
     * unchanged.  A buffer replaced by a larger one is kept (not freed) until
     * the context is destroyed, so a graph captured before the growth still
     * replays on valid memory -- but shares it with no later launch.  Growth
     * is geometric (at least 1.5x), so kept buffers total less than twice the
     * live ones.  No counterpart in the reference. */
    uint64_t workspace_generation;
} air_hip_stats;

/* ---- library ---------------------------------------------------------- */

/* Version of this C ABI (no counterpart in the reference). */
int air_hip_abi_version(void);
/* Name of an AIR_HIP_* status: the values mirror air::ErrorCode
 * (include/air/status.hpp:8-17), whose names they return. */
const char* air_hip_status_string(int status);
/* Message of the calling thread's most recent failure ("" if none): the
 * message a failing air::Status carries (include/air/status.hpp:19-40). */
const char* air_hip_last_error(void);

/* Number of visible HIP devices.  cuda_devices() (cuda_backend.cu:2447-2471). */
int air_hip_device_count(int* count);
/* Free and total device memory of `device` via hipMemGetInfo; the source of
 * PreparedModel::free_device_bytes / sequence_capacity_bytes
 * (src/runtime/backend.cpp:541-560). */
int air_hip_mem_info(int device, uint64_t* free_bytes, uint64_t* total_bytes);

/* ---- context: one device, one stream, one workspace -------------------- */

/* Binds `device` and `stream` (a hipStream_t or NULL), like
 * CudaExecutor::create / Impl::initialize (cuda_backend.cu:1773-1776).  The
 * context owns the activation workspace; calls through one context are
 * ordered on its stream, so one context must not be used from two threads
 * at once. */
int air_hip_context_create(int device, void* stream, air_hip_context** out);
/* Frees the context's buffers after its stream drains (the executor's
 * teardown of the same workspace). */
int air_hip_context_destroy(air_hip_context* ctx);
/* Rebinds the context to another stream, as cublasSetStream rebinds the
 * reference's handle (cuda_backend.cu:1780); work already queued stays on
 * the old one. */
int air_hip_context_set_stream(air_hip_context* ctx, void* stream);
/* Grows the workspaces so linears with input width <= max_k and up to max_m
 * rows never allocate on the hot path (workspace sizing,
 * cuda_backend.cu:1825-1869); the f32 partials of a K-split prefill GEMM,
 * which depend on the output width, are sized by the first call that needs
 * them.  Without it the first call that needs more space allocates. */
int air_hip_context_reserve(air_hip_context* ctx, uint64_t max_k, uint32_t max_m);
/* Counters and buffer sizes of the context (air_hip_stats above; no
 * counterpart in the reference). */
int air_hip_context_stats(const air_hip_context* ctx, air_hip_stats* out);
/* Overrides the decode linear's launch shape for this context (autotuning):
 * rows_per_wave = 16-row tiles per wavefront (1, 2 or 4), waves_per_group =
 * wavefronts splitting K inside one workgroup (1..16), k_splits =
 * workgroups splitting K (1..64, single-launch path only).  0 keeps the
 * automatic choice; wave counts beyond what a compiled variant supports are
 * clamped to its maximum.  Tunes the replacement of specialized_matvec_kernel
 * (src/cuda/cuda_backend.cu:585-606). */
int air_hip_context_set_tuning(air_hip_context* ctx, uint32_t rows_per_wave, uint32_t waves_per_group,
                               uint32_t k_splits);
/* One-row decode GEMV launch shape (autotuning; 0 keeps the automatic
 * choice).  pair_mode 1 = one workgroup per 16-row tile, 2 = two wherever
 * it applies (at most 8192 output rows, not the fused gate|up SwiGLU): each
 * takes half the tile's K and they combine through a per-row 64-bit slot
 * that the context zeroes at creation and every launch leaves zero, so
 * launches of one context must not overlap in time.  units_per_chunk =
 * work units per 512-weight chunk (1, or 2 for Q8_0; other formats keep 1),
 * depth = chunk buffers per wave (1 or 2).  Same kernels as specialized_matvec_kernel's replacement
 * (src/cuda/cuda_backend.cu:585-606). */
int air_hip_context_set_gemv_shape(air_hip_context* ctx, uint32_t pair_mode, uint32_t units_per_chunk,
                                   uint32_t depth);
/* How the skinny and wave-split decode kernels (2..64 rows) sum a K split
 * over workgroups when no epilogue rides on the sum (autotuning): mode 0 =
 * automatic (in the kernel for small outputs: a 2-way split up to 256k
 * outputs, longer splits up to 56k outputs per added split; otherwise the
 * reduction launch), 1 = always the reduction launch, 2 = always in the
 * kernel.  In the kernel,
 * the workgroups of an output meet through context-owned 64-bit slots (a
 * chain in split order, so the bits equal the reduction launch's); the
 * slots grow on demand outside graph capture, and a call that would need
 * them to grow during capture takes the reduction launch.  Replaces the
 * second pass of the reference's batch-reuse matmul
 * (src/cuda/cuda_backend.cu:529-583) for these widths. */
int air_hip_context_set_split_chain(air_hip_context* ctx, uint32_t mode);
/* Waves per workgroup of the LDS-pipelined skinny kernel (autotuning): 0 =
 * automatic (eight for Q8_0 gate|up-sized matrices at 17..32 rows, else
 * four), 4, or 8 = eight waves over twice the weight rows sharing each
 * step's activations (two stages, 17..32 or 49..64 rows; other widths keep
 * four).  Same arithmetic and bits as four waves.  Tunes the replacement of
 * the reference's batch-reuse matmul (src/cuda/cuda_backend.cu:529-583). */
int air_hip_context_set_skinny_waves(air_hip_context* ctx, uint32_t waves);
/* Chooses the decode kernel for 2..64 rows (autotuning): path 0 = automatic
 * (the skinny kernel: activations split once into the workspace and staged
 * through LDS, every weight read once, K split over workgroups when the
 * weight tiles cannot fill the GPU), 1 = the single-launch fused kernel for
 * M <= 16 and the per-wave K-split kernel above, 2 = skinny.  tile_n = 16-row
 * weight tiles per wavefront of the skinny kernel (1 or 2), k_splits its K
 * split (1..64); 0 keeps the automatic choice.  No counterpart in the
 * reference. */
int air_hip_context_set_decode_path(air_hip_context* ctx, uint32_t path, uint32_t tile_n, uint32_t k_splits);
/* Chooses how the decode linear (2..64 rows, skinny route) stages its
 * operands (autotuning): 0 = automatic, 1 = through registers
 * (skinny_kernel), 2..4 = an LDS ring of that many 64-k steps filled by
 * direct global -> LDS loads (skinny_lds_kernel, every format; above 16
 * rows the linear then runs on split activations).  No counterpart in the
 * reference. */
int air_hip_context_set_decode_pipeline(air_hip_context* ctx, uint32_t lds_stages);
/* Chooses the wave-split decode kernel for 2..64 rows (autotuning): mode 0 =
 * automatic, 1 = always, 2 = never.  A workgroup owns tile_n 16-row weight
 * tiles (1, 2 or 4) and every activation row; its `waves` waves (1..8) split
 * K, each keeping depth - 1 steps of weight codes in flight (depth 2 or 4);
 * k_splits workgroups split K further (1..64, with a deterministic
 * reduction); split_x = 1 splits the activations into the workspace first,
 * 2 in each wave.  0 keeps the automatic choice.  Mode 0 takes the kernel
 * where it measured faster than the skinny kernels (every 7B matrix but the
 * lm_head at M <= 16, the narrow ones above) and only while the decode path
 * is automatic.  No counterpart in the reference. */
int air_hip_context_set_wsplit(air_hip_context* ctx, uint32_t mode, uint32_t tile_n, uint32_t waves, uint32_t depth,
                               uint32_t k_splits, uint32_t split_x);
/* Chooses the kernel of the dense matrices (F16, BF16 and Q6_K storage;
 * autotuning): path 0 = automatic (the matrix-core kernel for 2..64 rows,
 * the f16 prefill GEMM on the rows at prefill widths, FMA kernels
 * otherwise), 1 = the matrix-core kernel at every width, 2 = the FMA
 * kernels.
 * tile_n = 16-row weight tiles per workgroup (1, 2 or 4), waves = waves
 * splitting K (1..8; the one-row Q6_K GEMV 1..16), depth = weight steps per
 * wave ring (2 or 4); for the one-row Q6_K GEMV tile_n = 2 takes two
 * super-blocks per work unit and depth 4 / 2 one / two units in flight.  0
 * keeps the automatic choice.  No counterpart in the reference. */
int air_hip_context_set_dense_path(air_hip_context* ctx, uint32_t path, uint32_t tile_n, uint32_t waves,
                                   uint32_t depth);
/* Reads `bytes` (a multiple of 16) of device memory once on the context's
 * stream and stores the XOR of each chunk's 32-bit words in a word of
 * `sink` (sink_words >= 1 words of device memory the caller zeroes; the
 * checksum, the XOR of all sink words, does not depend on the chunking): the
 * streaming floor of one launch of that size, with the decode GEMV's access
 * pattern (a workgroup per contiguous chunk, 16-byte non-temporal loads).
 * The benchmark prices each linear against it.  No counterpart in the
 * reference. */
int air_hip_stream_read(air_hip_context* ctx, const void* data, uint64_t bytes, uint32_t* sink,
                        uint64_t sink_words);
/* Chooses how the prefill GEMM stages its operands (autotuning): 0 =
 * automatic, 1 = through registers (prefill_gemm_kernel), 2..4 = an LDS ring
 * of that many 64-k steps filled by direct global -> LDS loads
 * (prefill_lds_kernel; Q8_0 with the 8x4 or 4x2 tile, others keep the
 * register path); 0x12 / 0x13 = the activation fragments alone through a
 * ring of 2 / 3 steps with every wave's weight records loaded straight into
 * registers (prefill_hyb_kernel; any storage format, 8x4, 8x2 and 4x2
 * tiles; the automatic choice for Q4_K).  No counterpart in the reference. */
int air_hip_context_set_prefill_pipeline(air_hip_context* ctx, uint32_t lds_stages);
/* Overrides the prefill GEMM's launch shape for this context: tile_m =
 * 16-row activation tiles per wavefront (4 or 8), tile_n = 16-row weight
 * tiles per wavefront (2 or 4), k_splits = workgroups splitting K (1..64; a
 * split sums its partials in a second, deterministic pass), prefetch = steps
 * of weight codes in flight (1 or 2; only the 8x4 tile has both).  0 keeps
 * the automatic choice.  No counterpart in the reference (its tactics have
 * fixed shapes); it exists for autotuning sweeps. */
int air_hip_context_set_prefill_tuning(air_hip_context* ctx, uint32_t tile_m, uint32_t tile_n,
                                       uint32_t k_splits, uint32_t prefetch);
/* Overrides the K split of the prefill GEMM's remainder launch (the rows past
 * the 8x4 tile's whole rounds, run on the 4x2 tile): 1 = unsplit, 2..64 that
 * many splits (a column reduction sums them in split order), 0 = automatic
 * (enough splits to fill a round, at least 8 steps each).  No counterpart in
 * the reference; it exists for autotuning sweeps. */
int air_hip_context_set_prefill_remainder_splits(air_hip_context* ctx, uint32_t splits);

/* ---- matrices ----------------------------------------------------------- */

/* Exact GGUF storage size of a {k, n} matrix of `type`, 0 if unsupported
 * (gguf_format.cpp:246-259). */
uint64_t air_hip_canonical_bytes(int type, uint64_t k, uint64_t n);

/* Makes a {k, n} matrix resident: canonical GGUF bytes (host memory when
 * bytes_on_device == 0, else device memory of the context's device) are
 * repacked once into the wavefront tile layout.  This is the residency step
 * of Impl::initialize (cuda_backend.cu:1790-1822) plus the one-time repack
 * the reference does only for dp4a (pack_signed32_weights_kernel,
 * cuda_backend.cu:398-427).  k must be a multiple of the block size
 * (cuda_backend.cu:1797-1801).  Blocks until the repack has finished.
 * Dense types (F32, F16, BF16, Q6_K) need k a multiple of 32 (Q6_K: 256); their
 * matrices take f32 rows through air_hip_linear (any tactic and width, the
 * epilogue entry points running their epilogues as separate launches), not
 * air_hip_linear_loaded or air_hip_decode_linear_fused (UNSUPPORTED).
 * air_hip_matrix_describe reports the type the matrix was prepared from. */
int air_hip_matrix_prepare(air_hip_context* ctx, int type, uint64_t k, uint64_t n,
                           const void* canonical, uint64_t canonical_bytes,
                           int bytes_on_device, air_hip_matrix** out);
/* Frees the resident matrix (the prepared weights' device buffer of
 * cuda_backend.cu:1797-1801). */
int air_hip_matrix_release(air_hip_matrix* matrix);
/* Type, shape and sizes of a resident matrix (no counterpart in the
 * reference, which keeps its GGUF tensor info on the host). */
int air_hip_matrix_describe(const air_hip_matrix* matrix, air_hip_matrix_desc* out);

/* Decodes the resident matrix to f32 out[n][k] (device pointer), bit-exact
 * with decode_all (src/reference/tensor_reader.cpp:51-247). */
int air_hip_matrix_dequantize(air_hip_context* ctx, const air_hip_matrix* matrix, float* out);

/* Decodes `elements` values of canonical GGUF bytes that are already in
 * device memory into f32 `out` (device), bit-exact; the device analogue of
 * decode_element / dequantize_to_f32_kernel (cuda_backend.cu:241-344,375-382). */
int air_hip_dequantize_canonical(air_hip_context* ctx, int type, const void* canonical,
                                 uint64_t canonical_bytes, uint64_t elements, float* out);

/* ---- the linear --------------------------------------------------------- */

/* Stage 1: loads activations x [m][k] (device f32, row-major) into the
 * context workspace as the engine's split f16 hi/lo operand tiles with a
 * per-row power-of-two scale -- the staging that the reference's
 * batch-reuse matmul does per launch (src/cuda/cuda_backend.cu:529-583).  One load serves every following
 * air_hip_linear_loaded call with the same input width k (q/k/v and
 * gate/up share their input).  Asynchronous on the context's stream. */
int air_hip_activations_load(air_hip_context* ctx, const float* x, uint64_t k, uint32_t m);

/* Stage 2: y[m][n] = sum_k w[n][k] * x[m][k] (+ bias[n]) over the activations
 * last loaded into ctx (specialized_matmul_batch_reuse_kernel's product,
 * cuda_backend.cu:529-583); the matrix input width must equal the loaded k.
 * Decode tactic only (PREFILL returns unsupported: it loads its own f16
 * operand inside air_hip_linear).  Asynchronous on the context's stream. */
int air_hip_linear_loaded(air_hip_context* ctx, const air_hip_matrix* matrix,
                          float* y, const float* bias, int tactic);

/* Both stages in one call: y[m][n] = sum_k w[n][k] * x[m][k] (+ bias[n]).
 *   x    device f32 [M][k], row-major
 *   y    device f32 [M][n], row-major (must not alias x)
 *   bias device f32 [n] or NULL (fused; add_optional_tensor,
 *        cuda_backend.cu:2143-2161 / reference_executor.cpp:315-323)
 * Asynchronous on the context's stream.  Replaces Impl::matvec / matmul /
 * linear_single (cuda_backend.cu:1898-2124). */
int air_hip_linear(air_hip_context* ctx, const air_hip_matrix* matrix,
                   const float* x, float* y, const float* bias,
                   uint32_t m, int tactic);

/* One line of text naming the kernels and launch shape air_hip_linear would
 * use for this matrix, m rows and tactic through this context (with its
 * tuning overrides), e.g. "decode_gemv_kernel<q8_0> rows_per_wave=1 depth=1
 * units_per_chunk=2 waves=8 groups=2368".  Launches nothing; text is cut to
 * capacity - 1 characters and NUL-terminated.  For tests and profiles that
 * name the variant they exercised.  No counterpart in the reference. */
int air_hip_linear_plan(const air_hip_context* ctx, const air_hip_matrix* matrix, uint32_t m, int tactic,
                        char* text, uint64_t capacity);

/* air_hip_linear for decode widths m = 1..64 (tactic AUTO or DECODE) that
 * allocates nothing: no hipMalloc / hipFree and no allocating library call,
 * so code under HIP graph capture, tight serving loops and harnesses that
 * forbid allocation can call it.  Same kernels and launch shapes as
 * air_hip_linear through this context (its tuning overrides included), so
 * the outputs are bit-identical; a K split that air_hip_linear sums inside
 * the kernel (air_hip_context_set_split_chain) takes the reduction launch
 * here, which the in-kernel sum reproduces bit for bit.  Its split
 * activations and K-split partials live in a 16 MiB device array per GPU,
 * and the one-row GEMV's pair-split row slots in a second one of 8192
 * words, both held from library load until the process ends (every
 * Qwen2-7B projection and lm_head at m <= 64 needs at most 12.5 MiB); a
 * linear needing more, m > 64, the PREFILL tactic, and the
 * fused kernel's cross-workgroup K split (a tuning override) return
 * AIR_HIP_UNSUPPORTED.  The array keeps the last call's contents and is
 * shared by every call on that GPU: calls that overlap on one GPU (other
 * streams, other contexts, other threads) race and must be serialised by
 * the caller.  No counterpart in the reference: it exists for the callers
 * that cannot allocate. */
int air_hip_linear_noalloc(air_hip_context* ctx, const air_hip_matrix* matrix, const float* x, float* y,
                           const float* bias, uint32_t m, int tactic);

/* The M = 1 decode linear with its element-wise neighbours in the step
 * fused into the one launch, for a single-sequence decode loop: the
 * reference runs them as separate kernels around the projection
 * (rms_norm_kernel, add_vector_kernel, silu_mul_kernel, cuda_backend.cu:789,
 * 849-860), in the arithmetic of reference_executor.cpp:17-35.
 *   norm_weight  NULL, or the RMSNorm weight (k floats): x is first
 *                normalised, x_i * float(1 / sqrt(mean(x^2) + eps)) * w_i,
 *                the sum of squares in double (as air_hip_rms_norm; the
 *                summation order differs);
 *   epilogue     STORE     y = W x + b (n floats);
 *                RESIDUAL  y += W x + b (y: the residual stream, n floats);
 *                SWIGLU    the matrix is a fused gate|up of n = 2F rows
 *                          (F a multiple of 16): y[i] = silu(g_i) * u_i for
 *                          the F outputs, silu(g) = g / (1 + e^-g).
 * Every combination but (norm, RESIDUAL).  x is one
 * 16-byte aligned row of k floats and must not alias y.  Same tolerance as
 * the DECODE tactic.  No counterpart in the reference's linear API. */
enum {
    AIR_HIP_EPILOGUE_STORE = 0,
    AIR_HIP_EPILOGUE_RESIDUAL = 1,
    AIR_HIP_EPILOGUE_SWIGLU = 2,
    AIR_HIP_EPILOGUE_RESIDUAL_LOAD = 3,
    AIR_HIP_EPILOGUE_RESIDUAL_PREFILL = 4
};
int air_hip_decode_linear_fused(air_hip_context* ctx, const air_hip_matrix* matrix, const float* x, float* y,
                                const float* bias, const float* norm_weight, double eps, int epilogue);

/* A linear over `rows` rows followed by the step's element-wise work on its
 * output, the two Qwen2 steps after a projection (reference_executor.cpp:
 * 29-31 add_in_place, 17-27 rms_norm, 325-428 the SiLU * up of the FFN):
 *   AIR_HIP_EPILOGUE_SWIGLU: out [rows][n/2] = silu(g) * u, g and u the
 *     linear's columns i and n/2 + i of a fused gate|up matrix
 *     (air_hip_silu_mul); norm_weight must be null;
 *   AIR_HIP_EPILOGUE_RESIDUAL: out [rows][n] += x W^T + bias, then, with
 *     norm_weight, norm_out[r] = rms_norm(out[r]) * norm_weight
 *     (air_hip_add_rms_norm; norm_out must not alias out);
 *   AIR_HIP_EPILOGUE_RESIDUAL_LOAD: RESIDUAL with its norm (required), and
 *     norm_out is also split into the context's activation workspace as
 *     air_hip_activations_load(norm_out, n, rows) would split it; the next
 *     linear this context runs on x == norm_out with the same width and rows
 *     uses that split instead of splitting again.  Any other call through
 *     this context that writes device memory cancels it (that linear then
 *     splits norm_out itself); changing norm_out by other means in between
 *     is the caller's error.
 *   AIR_HIP_EPILOGUE_RESIDUAL_PREFILL: RESIDUAL with its norm (required), and
 *     norm_out is also converted for the next prefill linear as
 *     air_hip_rms_norm_prefill converts it, with the same reuse rules.
 *     Prefill-width linears with a K split carry it in their reduction.
 * Bit-identical to air_hip_linear (same tactic) followed by that call.  Where
 * the linear runs with a K split (a skinny launch at decode widths 2..64,
 * or a prefill GEMM), its split reduction
 * applies the epilogue, so the epilogue costs no launch of its own; other
 * routes run the linear into a context buffer and the separate kernel.  out must not alias x.  No counterpart in the reference's
 * linear API: it replaces the executor's linear then add / SiLU sequence
 * (cuda_backend.cu:789, 849-860). */
int air_hip_linear_epilogue(air_hip_context* ctx, const air_hip_matrix* matrix, const float* x, uint32_t rows,
                            float* out, const float* bias, int epilogue, const float* norm_weight, float* norm_out,
                            double eps, int tactic);

/* ---- the Qwen2 step around the linears ---------------------------------- */
/* Device primitives of one Qwen2 step over M rows, each row a (sequence,
 * position, token).  Arithmetic follows the reference executor operation by
 * operation (src/reference/reference_executor.cpp:17-138): double RMSNorm
 * sums, host-built double RoPE tables, double attention scores and softmax
 * with float probabilities, unfused float products.  All pointers are device
 * pointers; every call is asynchronous on the context's stream. */

/* out[i][k] = W[rows[i]][k], decoded bit-exactly from a resident matrix: the
 * embedding lookup (ReferenceTensorReader::row, tensor_reader.cpp:347-367).
 * rows: int32 [m]; rows outside [0, n) leave their output row untouched. */
int air_hip_matrix_rows(air_hip_context* ctx, const air_hip_matrix* matrix, const int32_t* rows,
                        uint32_t m, float* out);

/* out[r] = x[r] * float(1 / sqrt(mean(x[r]^2) + eps)) * weight, rows of n
 * (rms_norm, reference_executor.cpp:17-27).  out may alias x. */
int air_hip_rms_norm(air_hip_context* ctx, const float* x, const float* weight, float* out, uint32_t m,
                     uint64_t n, double eps);

/* The residual add and the RMSNorm that follows it in one pass over each row
 * (add_in_place then rms_norm, reference_executor.cpp:29-31, 17-27):
 * x[r] += y[r], then out[r] = rms_norm(x[r]) * weight.  out must not alias
 * x or y. */
int air_hip_add_rms_norm(air_hip_context* ctx, float* x, const float* y, const float* weight, float* out, uint32_t m,
                         uint64_t n, double eps);

/* air_hip_add_rms_norm (y given) or air_hip_rms_norm (y NULL; out may then
 * alias x), and out is also converted into the context's prefill
 * workspace as the next prefill linear converts its f32 input (f16 rows,
 * one power-of-two scale per row): the next linear this context runs on
 * x == out with the prefill route, the same width and rows uses that
 * operand instead of converting again (bit-identical).  Any other call
 * through the context in between cancels it, as for
 * AIR_HIP_EPILOGUE_RESIDUAL_LOAD.  Rows wider than 8192 get the plain norm.
 * No counterpart in the reference: it replaces the norm and the conversion
 * pass of the prefill GEMM's input. */
int air_hip_rms_norm_prefill(air_hip_context* ctx, float* x, const float* y, const float* weight, float* out,
                             uint32_t m, uint64_t n, double eps);

/* In-place rotary embedding of the q and k heads of fused q|k|v rows
 * (apply_rope, reference_executor.cpp:37-72): row r (stride floats apart)
 * rotates by position positions[r] with table[position][i] = {cos, sin} of
 * the reference's double angle for pair i < rope_dims / 2 (table_positions
 * positions; positions beyond it are the caller's error). */
int air_hip_rope(air_hip_context* ctx, float* qkv, uint64_t row_stride, uint32_t m, const int32_t* positions,
                 uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t rope_dims,
                 const float* table, uint64_t table_positions);

/* Paged fp32 KV cache.  A page holds [layer][K, V][page_tokens][kv_width]
 * floats for `layers` layers; a sequence is the list of its pages (int32),
 * max_pages entries per page-table row.  The pages live either in one
 * allocation (`pool`: page p at pool + p pages; `chunks` null) or, for a pool
 * that grows, in separately allocated chunks of 2^chunk_shift pages: `chunks`
 * is a device array of pool_pages >> chunk_shift chunk bases, page p lives at
 * page p & (2^chunk_shift - 1) of chunks[p >> chunk_shift], and a null base is
 * a chunk not allocated yet.  Entries outside [0, pool_pages), and pages of
 * unallocated chunks, are skipped by the kernels.  The reference's CUDA pool
 * grows page by page (src/cuda/cuda_backend.cu:1186-1300); a chunk table
 * keeps every page where it was, so launches captured before the pool grew
 * stay valid. */
typedef struct air_hip_kv_layout {
    float* pool;
    uint32_t page_tokens;
    uint32_t kv_width;       /* kv_heads * head_dim */
    uint32_t layers;
    uint32_t max_pages;
    uint32_t pool_pages;
    float* const* chunks;    /* device chunk table, or null for a single pool */
    uint32_t chunk_shift;    /* log2 of the pages per chunk (<= 30) */
} air_hip_kv_layout;

/* Writes each row's k and v (the q|k|v row after RoPE) into the slot of
 * positions[r] of its sequence: page_tables is int32 [m][max_pages].
 * append_kv_batch_kernel (src/cuda/cuda_backend.cu:1156-1173). */
int air_hip_kv_append(air_hip_context* ctx, const air_hip_kv_layout* kv, const float* qkv, uint64_t row_stride,
                      uint64_t q_width, uint32_t m, const int32_t* positions, const int32_t* page_tables,
                      uint32_t layer);

/* air_hip_rope then air_hip_kv_append in one launch, with the same results
 * (rope_batch_kernel then append_kv_batch_kernel, cuda_backend.cu:883-906,
 * 1156-1173): the q and k heads of each row are rotated in place and k
 * (kv_heads * head_dim = kv->kv_width floats after the q heads) and v are
 * stored in the row's slot.  A position outside the table is not rotated; a
 * row without a valid page slot is rotated but not stored. */
int air_hip_rope_kv_append(air_hip_context* ctx, const air_hip_kv_layout* kv, float* qkv, uint64_t row_stride,
                           uint32_t m, const int32_t* positions, const int32_t* page_tables, uint32_t layer,
                           uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t rope_dims,
                           const float* table, uint64_t table_positions);

/* The q|k|v linear and air_hip_rope_kv_append in one call: qkv [rows][n]
 * (n = (q_heads + 2 * kv_heads) * head_dim) receives x W^T + bias with the q
 * and k heads rotated, and k, v are appended to the pool -- bit-identical to
 * air_hip_linear (same tactic) followed by air_hip_rope_kv_append over rows
 * of stride n.  Where the linear runs with a K split (a skinny launch at
 * decode widths 2..64, or a prefill GEMM), its split reduction does the RoPE
 * and the append, so they cost no launch of their own.  qkv must not alias x.  Replaces the
 * executor's q|k|v projection, apply_rope and KV store sequence
 * (cuda_backend.cu:883-906, 1156-1173; reference_executor.cpp:37-72). */
int air_hip_linear_rope_kv(air_hip_context* ctx, const air_hip_matrix* matrix, const float* x, uint32_t rows,
                           float* qkv, const float* bias, const air_hip_kv_layout* kv, const int32_t* positions,
                           const int32_t* page_tables, uint32_t layer, uint32_t q_heads, uint32_t kv_heads,
                           uint32_t head_dim, uint32_t rope_dims, const float* table, uint64_t table_positions,
                           int tactic);

/* Attention of every row's q heads over tokens 0..positions[r] of its
 * sequence for one layer (attention, reference_executor.cpp:74-138):
 * out[r][q_heads * head_dim].  max_tokens bounds positions[r] + 1 and sizes
 * the context's score scratch (m * q_heads * max_tokens doubles). */
int air_hip_attention(air_hip_context* ctx, const air_hip_kv_layout* kv, const float* qkv, uint64_t row_stride,
                      uint32_t m, const int32_t* positions, const int32_t* page_tables, uint32_t layer,
                      uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim, uint64_t max_tokens, float* out);

/* The online_softmax attention tactic (AttentionExecutionKind::online_softmax,
 * include/air/execution.hpp:47-50; the reference's
 * attention_batch_paged_online_kernel, cuda_backend.cu:1093-1154): the same
 * output as air_hip_attention, computed in f32 with a running maximum over
 * key chunks staged through LDS, ~1e-6 relative from the double softmax.
 * Work is cut into tiles of up to 16 query vectors that share a sequence and
 * a KV head. */
typedef struct air_hip_attention_tile {
    uint32_t row;    /* first row */
    uint32_t rows;   /* rows of one sequence, consecutive in the step */
    uint32_t head;   /* first q head */
    uint32_t heads;  /* q heads of one KV head; rows * heads <= 16 */
} air_hip_attention_tile;

/* Host helper (no counterpart in the reference, whose online kernel takes
 * one (token, head) per block): the tiles of a step whose rows form `runs` consecutive runs,
 * run i holding run_rows[i] rows of one sequence at consecutive positions.
 * A one-row run (decode) gives a tile per KV head of its grouped q heads; a
 * longer run (prefill) tiles of 16 rows per q head, its last rows (the
 * longest key ranges) first.  tiles may be NULL (the
 * count is still returned). */
int air_hip_attention_make_tiles(const uint32_t* run_rows, uint32_t runs, uint32_t q_heads, uint32_t kv_heads,
                                 air_hip_attention_tile* tiles, uint32_t capacity, uint32_t* count);

/* Attention through tiles made by air_hip_attention_make_tiles for these m
 * rows (device array, uploaded by the caller; the kernel skips a tile that
 * names rows or heads outside the call): the online_softmax tactic, in place
 * of attention_batch_paged_online_kernel (src/cuda/cuda_backend.cu:1093-1154).  head_dim 64 or 128; q|k|v rows,
 * out and the pool 16-byte aligned.  Tiles with long key ranges are split
 * over workgroups and merged in a second pass (context scratch). */
int air_hip_attention_online(air_hip_context* ctx, const air_hip_kv_layout* kv, const float* qkv, uint64_t row_stride,
                             uint32_t m, const int32_t* positions, const int32_t* page_tables, uint32_t layer,
                             uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                             const air_hip_attention_tile* tiles, uint32_t tile_count, uint64_t max_tokens,
                             float* out);

/* out[r][i] = silu(gate_up[r][i]) * gate_up[r][ffn + i] over fused gate|up
 * rows (reference_executor.cpp:33-35, 400). */
int air_hip_silu_mul(air_hip_context* ctx, const float* gate_up, float* out, uint32_t m, uint64_t ffn);

/* air_hip_silu_mul with out also converted for the next prefill linear, as
 * air_hip_rms_norm_prefill does (ffn up to 24576; wider rows get the plain
 * SwiGLU).  No counterpart in the reference. */
int air_hip_silu_mul_prefill(air_hip_context* ctx, const float* gate_up, float* out, uint32_t m, uint64_t ffn);

/* x[i] += y[i] (the residual adds, add_in_place, reference_executor.cpp:29-31). */
int air_hip_add(air_hip_context* ctx, float* x, const float* y, uint64_t count);

/* out[r] = index of the first maximum of logits[r][0..n) (greedy selection,
 * src/runtime/sampling.cpp:13-16), or -1 when row r holds a non-finite value
 * (NaN or +-inf): the reference's device selection flags such a value and
 * fails the step with "non-finite logits" (src/cuda/cuda_backend.cu:613-624,
 * 2368), so a caller treats -1 as internal_error. */
int air_hip_argmax(air_hip_context* ctx, const float* logits, uint32_t m, uint64_t n, int32_t* out);

#ifdef __cplusplus
}
#endif

#endif /* AIR_HIP_H */

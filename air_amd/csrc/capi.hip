// capi.hip -- the C ABI of libair_hip.so (include/air_hip.h).
//
// Host-side owner of contexts (device + stream + workspace) and resident
// matrices; validates every argument, launches the kernels and maps HIP
// failures onto air_hip_status.  Structure follows CudaExecutor::Impl's
// residency/dispatch duties (src/cuda/cuda_backend.cu:1435-1478,1773-1869,
// 1898-2124) without its per-call tensor-name lookup: callers hold matrix
// handles.
#include "../../include/air_hip.h"

#include "air_hip_kernels.hpp"
#include "air_hip_layout.hpp"

#include <hip/hip_runtime.h>
#include <rocprofiler-sdk-roctx/roctx.h>

#include <algorithm>
#include <atomic>
#include <vector>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <limits>
#include <mutex>
#include <new>
#include <string>

using namespace air_hip;

// Device memory of air_hip_linear_noalloc: one array per GPU, allocated with
// the code object when the library is loaded on that GPU and held until the
// process ends.  In host code this name is a host-side stand-in, not a
// device address: host code uses only the per-device pointer that
// hipGetSymbolAddress returns for it (noalloc_scratch below).
constexpr std::uint64_t kNoAllocScratchBytes = 16ull << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];
// The pair-split GEMV's row slots for air_hip_linear_noalloc: zero when the
// code object is loaded, and every launch leaves them zero (the scratch
// array's contents are not, so the slots cannot live there).
__device__ __align__(256) std::uint64_t noalloc_pair_slots[kGemvPairSlots];

struct air_hip_context {
    int device{0};
    hipStream_t stream{nullptr};
    void* workspace{nullptr};
    std::uint64_t workspace_bytes{0};
    std::atomic<std::uint64_t> resident_matrix_bytes{0};
    std::atomic<std::uint64_t> host_to_device_bytes{0};
    std::atomic<std::uint64_t> prepared_matrices{0};
    std::atomic<std::uint64_t> decode_linear_calls{0};
    std::atomic<std::uint64_t> prefill_linear_calls{0};
    std::atomic<std::uint64_t> decode_rows{0};
    std::atomic<std::uint64_t> prefill_rows{0};
    std::uint64_t loaded_k{0};       // width of the activations in the workspace
    std::uint32_t loaded_rows{0};    // rows of the activations in the workspace (0 = none)
    bool loaded_row_scaled{false};   // split with one scale per row (skinny kernel layout)
    // The rows the loaded activations were split from by an epilogue
    // (AIR_HIP_EPILOGUE_RESIDUAL_LOAD); the next linear on the same rows
    // uses them instead of splitting again.  Null after any other load and
    // once used.
    const void* loaded_source{nullptr};
    // The last call left the next prefill linear's operand for these f32
    // rows in the prefill workspace (air_hip_rms_norm_prefill /
    // air_hip_silu_mul_prefill); good for the next call only.
    const void* prefill_source{nullptr};
    std::uint64_t prefill_source_k{0};
    std::uint32_t prefill_source_rows{0};
    DecodeTuning tuning{};
    // Cross-workgroup K-split of the fused decode linear: partial sums and one
    // arrival counter per row group.  Counters are zeroed when allocated and
    // every launch leaves them at zero.
    void* split_partials{nullptr};
    std::uint64_t split_partials_bytes{0};
    std::uint32_t* split_counters{nullptr};
    std::uint32_t split_counter_count{0};
    // Prefill GEMM: f16 activations, row scales and K-split partials.
    void* prefill_workspace{nullptr};
    std::uint64_t prefill_workspace_bytes{0};
    PrefillTuning prefill_tuning{};
    // Decode widths 2..64: 0 = automatic (skinny kernel), 1 = the earlier
    // kernels (fused for M <= 16, decode_linear above), 2 = skinny.
    std::uint32_t decode_path{0};
    std::uint32_t skinny_tile_n{0};
    std::uint32_t skinny_splits{0};
    std::uint32_t skinny_lds_stages{0};   // 0 automatic, 1 registers, 2..4 LDS ring stages
    std::uint32_t skinny_waves{0};        // 0 automatic, 4, or 8 waves per workgroup on the LDS pipeline
    // Decode widths 2..64 on the wave-split kernel: 0 = automatic, 1 = always,
    // 2 = never; and its launch-shape overrides.
    std::uint32_t wsplit_mode{0};
    WsplitTuning wsplit_tuning{};
    // Dense matrices (F16 / BF16 / Q6_K storage): kernel choice and shape.
    DenseTuning dense_tuning{};
    std::uint32_t* bound_scratch{nullptr};  // one uint32 for the weight exponent at residency
    void* attention_scratch{nullptr};       // attention scores, grown on demand
    void* argmax_partials{nullptr};         // per-slice partials of the greedy selection
    std::uint64_t argmax_partials_bytes{0};
    std::uint64_t attention_scratch_bytes{0};
    void* epilogue_rows{nullptr};           // linear output of air_hip_linear_epilogue's unfused route
    std::uint64_t epilogue_rows_bytes{0};
    // This device's `scratch` array (hipGetSymbolAddress at context creation).
    void* noalloc_scratch{nullptr};
    // The pair-split GEMV's row slots: kGemvPairSlots words, zeroed at
    // context creation and left zero by every launch (noalloc_pairs: the
    // device's noalloc_pair_slots array, for air_hip_linear_noalloc).
    std::uint64_t* gemv_pairs{nullptr};
    std::uint64_t* noalloc_pairs{nullptr};
    // Slots of the in-kernel K-split chain (chain_combine) of the skinny and
    // wave-split kernels, zeroed when allocated and left zero by every
    // launch; chain_mode 0 = automatic, 1 = reduction launches, 2 = chain
    // for every split.
    std::uint64_t* chain_slots{nullptr};
    std::uint64_t chain_slots_bytes{0};
    std::uint32_t chain_mode{0};
    // Bumped whenever a context-owned buffer is (re)allocated: launches
    // recorded into a graph use the current buffers while it is unchanged.
    std::uint64_t generation{0};
    // Buffers replaced by a larger one.  They are freed only with the
    // context: a graph captured before the growth still holds their address.
    // Growth is geometric, so they total less than twice the live size.
    std::vector<void*> retired;
};

struct air_hip_matrix {
    air_hip_context* owner{nullptr};
    TilePlanes planes;             // planes.type is the resident format (Q5_0 arrives as Q8_0)
    int type{0};                   // the canonical type it was prepared from
    void* dense{nullptr};          // dense_type(type): rows [n][k] instead of tile planes
    int dense_storage{0};          // the type of the rows: kF32, kF16 / kBF16 (GGUF rows) or kQ6_K (208-byte
                                   // super-block records, then a plane of f16 d)
    TilePlanes gemm;               // F16 / BF16 / Q6_K storage as the prefill GEMM's weight operand (codes =
                                   // dense, kt = k); codes null when the GEMM does not take it
    std::uint64_t canonical_bytes{0};
    std::uint64_t resident_bytes{0};
};

namespace {

// ROCTX range around a linear entry point: air.hip.matvec (one row) or
// air.hip.matmul, the names of the reference's ranges around its linears
// (src/cuda/cuda_backend.cu:1899,1958, air.cuda.*), for rocprofv3
// --marker-trace.
struct LinearRange {
    explicit LinearRange(uint32_t rows) noexcept { roctxRangePushA(rows == 1u ? "air.hip.matvec" : "air.hip.matmul"); }
    ~LinearRange() { roctxRangePop(); }
    LinearRange(const LinearRange&) = delete;
    LinearRange& operator=(const LinearRange&) = delete;
};

thread_local std::string g_last_error;

// Activations are split over k padded to whole 256-element units, which
// covers the k tile of every format.
constexpr std::uint64_t kSplitK = 256;
constexpr std::uint32_t kMaxRows = 4096;

int fail(int status, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

int hip_fail(hipError_t err, const char* what) {
    return fail(AIR_HIP_INTERNAL_ERROR, "%s: %s", what, hipGetErrorString(err));
}

// Makes ctx->device current for the scope and restores the caller's device.
class DeviceScope {
public:
    explicit DeviceScope(int device) {
        if (hipGetDevice(&previous_) != hipSuccess) previous_ = -1;
        status_ = hipSetDevice(device);
    }
    ~DeviceScope() {
        if (previous_ >= 0) (void)hipSetDevice(previous_);
    }
    hipError_t status() const { return status_; }

private:
    int previous_{-1};
    hipError_t status_{hipSuccess};
};

std::uint64_t resident_plane_bytes(const TilePlanes& p, std::uint64_t& scale_bytes) {
    const auto geo = geometry_of(p.type);
    const std::uint64_t tiles = static_cast<std::uint64_t>(p.nt) * p.kt;
    scale_bytes = tiles * geo.scale_tile_bytes;
    return tiles * geo.code_tile_bytes;
}

// Replaces the context buffer *buf (of *size bytes) by one of at least
// `bytes`, grown geometrically.  The old buffer is retired, not freed: queued
// kernels and graphs captured earlier may still use it.  keep: the old
// contents are copied over (stream-ordered), e.g. loaded activations.
int grow_buffer(air_hip_context* ctx, void** buf, std::uint64_t* size, std::uint64_t bytes, const char* what,
                bool keep = false) {
    if (bytes <= *size) return AIR_HIP_OK;
    const std::uint64_t grown = std::max<std::uint64_t>(bytes, *size + *size / 2);
    void* p = nullptr;
    hipError_t err = hipMalloc(&p, grown);
    if (err == hipSuccess && keep && *buf) err = hipMemcpyAsync(p, *buf, *size, hipMemcpyDeviceToDevice, ctx->stream);
    if (err != hipSuccess) {
        (void)hipFree(p);
        return fail(AIR_HIP_INTERNAL_ERROR, "hipMalloc(%s): %s", what, hipGetErrorString(err));
    }
    if (*buf) ctx->retired.push_back(*buf);
    *buf = p;
    *size = grown;
    ++ctx->generation;
    return AIR_HIP_OK;
}

int ensure_workspace(air_hip_context* ctx, std::uint64_t bytes) {
    // Keeps activations loaded before a later reserve.
    return grow_buffer(ctx, &ctx->workspace, &ctx->workspace_bytes, bytes, "workspace", ctx->loaded_rows != 0);
}

// Loads x as the activations of a loaded linear unless the epilogue of the
// call just before it already split exactly these rows (`ready` = the source
// it recorded, taken by the linear entry point) into the workspace.
int load_activations_for(air_hip_context* ctx, const float* x, std::uint64_t k, std::uint32_t rows,
                         const void* ready) {
    const bool row_scaled = rows <= AIR_HIP_MAX_DECODE_ROWS && ctx->decode_path != 1u;
    const bool split = ready == x && ctx->loaded_k == k && ctx->loaded_rows == rows &&
                       ctx->loaded_row_scaled == row_scaled;
    return split ? AIR_HIP_OK : air_hip_activations_load(ctx, x, k, rows);
}

// Per-device address of `scratch`, looked up once per device with that
// device current (each GPU holds its own copy at its own address).
std::mutex g_scratch_mutex;
std::vector<void*> g_scratch_address;
std::vector<void*> g_pair_slots_address;

int noalloc_scratch(int device, void** out, void** pairs_out) {
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (static_cast<std::size_t>(device) >= g_scratch_address.size()) {
        g_scratch_address.resize(device + 1u, nullptr);
        g_pair_slots_address.resize(device + 1u, nullptr);
    }
    if (!g_scratch_address[device]) {
        void* p = nullptr;
        hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (err != hipSuccess || !p) return hip_fail(err != hipSuccess ? err : hipErrorInvalidSymbol,
                                                     "hipGetSymbolAddress(scratch)");
        void* q = nullptr;
        err = hipGetSymbolAddress(&q, HIP_SYMBOL(noalloc_pair_slots));
        if (err != hipSuccess || !q) return hip_fail(err != hipSuccess ? err : hipErrorInvalidSymbol,
                                                     "hipGetSymbolAddress(noalloc_pair_slots)");
        g_scratch_address[device] = p;
        g_pair_slots_address[device] = q;
    }
    *out = g_scratch_address[device];
    *pairs_out = g_pair_slots_address[device];
    return AIR_HIP_OK;
}

// Every entry point that writes device memory through the context forgets
// the rows an epilogue last split (AIR_HIP_EPILOGUE_RESIDUAL_LOAD) and the
// rows a *_prefill call last converted: after any such write the split or
// the f16 operand may no longer match its source.
void forget_loaded_source(air_hip_context* ctx) {
    ctx->loaded_source = nullptr;
    ctx->prefill_source = nullptr;
}

int ensure_prefill_workspace(air_hip_context* ctx, std::uint64_t bytes, bool keep = false) {
    return grow_buffer(ctx, &ctx->prefill_workspace, &ctx->prefill_workspace_bytes, bytes, "prefill workspace", keep);
}

// The prefill workspace's operand area for rows of width k: xh then row_inv
// (the layout launch_prefill_linear reads).
using PrefillOperand = PrefillOperandArgs;

int prefill_operand(air_hip_context* ctx, std::uint64_t k, std::uint32_t m, PrefillOperand* op) {
    const std::uint64_t mp = prefill_rows_padded(m);
    const std::uint64_t ldx = prefill_ldx(k);
    const std::uint64_t xh_bytes = ceil_div(mp * ldx * 2u, 256u) * 256u;
    const int rc = ensure_prefill_workspace(ctx, xh_bytes + ceil_div(mp * 4u, 256u) * 256u);
    if (rc != AIR_HIP_OK) return rc;
    auto* base = static_cast<std::uint8_t*>(ctx->prefill_workspace);
    *op = PrefillOperand{reinterpret_cast<_Float16*>(base), reinterpret_cast<float*>(base + xh_bytes),
                         static_cast<std::uint32_t>(mp), ldx};
    return AIR_HIP_OK;
}

void remember_prefill(air_hip_context* ctx, const void* source, std::uint64_t k, std::uint32_t m) {
    ctx->prefill_source = source;
    ctx->prefill_source_k = k;
    ctx->prefill_source_rows = m;
}

// Prefill linear: x [rows][k] -> y [rows][n] on the f16 MFMA GEMM; `ready`
// (taken by the linear entry point) names rows whose f16 operand the call
// before left in the workspace, which then skips the conversion.
int run_prefill(air_hip_context* ctx, const air_hip_matrix* m, const float* x, float* y, const float* bias,
                std::uint32_t rows, const void* ready = nullptr, std::uint64_t ready_k = 0,
                std::uint32_t ready_rows = 0, const SplitEpilogue* epilogue = nullptr, bool* applied = nullptr) {
    const TilePlanes& planes = m->dense ? m->gemm : m->planes;
    const PrefillShape shape = plan_prefill(planes, rows, ctx->prefill_tuning);
    const bool converted = ready == x && ready_k == planes.k && ready_rows == rows;
    int rc = ensure_prefill_workspace(ctx, prefill_workspace_bytes(planes.k, rows, shape, planes.n), converted);
    if (rc != AIR_HIP_OK) return rc;
    // A K-split launch's reduction carries the epilogue when it fits.
    const auto* partials = reinterpret_cast<const float*>(static_cast<const std::uint8_t*>(ctx->prefill_workspace) +
                                                          prefill_partials_offset(m->planes.k, rows));
    const SplitEpilogue* epi = epilogue && applied && shape.splits > 1u &&
                                       split_epilogue_fits(*epilogue, partials, bias, rows, m->planes.n)
                                   ? epilogue
                                   : nullptr;
    if (epi) *applied = true;
    const hipError_t err = launch_prefill_linear(planes, x, bias, y, rows, shape, ctx->prefill_workspace, ctx->stream,
                                                 converted, epi);
    if (err != hipSuccess) return hip_fail(err, "prefill_gemm_kernel");
    ctx->prefill_linear_calls.fetch_add(1, std::memory_order_relaxed);
    ctx->prefill_rows.fetch_add(rows, std::memory_order_relaxed);
    return AIR_HIP_OK;
}

int ensure_split_buffers(air_hip_context* ctx, std::uint64_t partial_bytes, std::uint32_t counters);
std::uint64_t* chain_for(air_hip_context* ctx, std::uint32_t splits, std::uint32_t m, std::uint64_t n);
int linear_loaded(air_hip_context* ctx, const air_hip_matrix* m, float* y, const float* bias, int tactic,
                  const SplitEpilogue* epilogue, bool* applied);

// The epilogue when the skinny launch's split reduction can carry it, else
// null (the linear then writes y).
const SplitEpilogue* reduction_epilogue(air_hip_context* ctx, const air_hip_matrix* m, const SkinnyShape& shape,
                                        const float* bias, std::uint32_t rows, const SplitEpilogue* epilogue,
                                        bool* applied) {
    if (!epilogue || shape.splits < 2u ||
        !split_epilogue_fits(*epilogue, static_cast<const float*>(ctx->split_partials), bias, rows, m->planes.n)) {
        return nullptr;
    }
    *applied = true;
    return epilogue;
}

// A dense matrix (F16 / BF16 / Q6_K storage) at prefill widths runs the f16
// MFMA prefill GEMM on its rows (measured at M = 512 on 3584 x 18944: F16
// 1411 -> 133 us, Q6_K 1590 -> 208 against the FMA GEMM); F32 and the
// autotuning paths 1 and 2 keep their kernels.
bool dense_prefill(const air_hip_context* ctx, const air_hip_matrix* m, std::uint32_t rows, int tactic) {
    if (!m->dense || !m->gemm.codes || ctx->dense_tuning.path != 0u || rows > kMaxRows) return false;
    return tactic == AIR_HIP_LINEAR_PREFILL || (tactic == AIR_HIP_LINEAR_AUTO && rows > AIR_HIP_MAX_DECODE_ROWS);
}

// Which kernels a linear of `rows` rows runs on, decided in one place for
// the launch path and for air_hip_linear_plan.
enum class Route { prefill, gemv, fused, skinny_x, skinny_loaded, decode_linear, dense, wsplit };

// The skinny kernel straight from the f32 rows, or over activations split
// into the workspace first.  The in-workgroup split repeats the activation
// split in every workgroup: it pays on narrow matrices, where the separate
// split launch dominates (Qwen2-7B q|k|v, o, down at M <= 32: 10-25 %
// faster), and loses on wide ones (gate|up, lm_head: up to 2x slower) and at
// M = 64.  Q4_K with four activation tiles would also spill in it.
Route skinny_route(const air_hip_context* ctx, const air_hip_matrix* m, std::uint32_t rows) {
    const SkinnyShape shape = plan_skinny(m->planes, rows, ctx->skinny_tile_n, ctx->skinny_splits, ctx->skinny_lds_stages,
                                          ctx->skinny_waves);
    // From 17 rows the split activations feed the LDS pipeline, which beats
    // the f32-input kernel on the narrow 7B matrices too, split launch
    // included (Q8_0, M = 32: q|k|v 18.4 -> 16.2 us, o 16.3 -> 14.7, down
    // 41.5 -> 32.1).  At M = 8 the two are even per call, and in a graph the
    // split's extra launch made the step slower (2.60 -> 2.78 ms).
    if (rows > 16u && shape.lds_stages >= 2u) return Route::skinny_loaded;
    const bool narrow = m->planes.nt <= 512u && (rows <= 32u || m->planes.k <= 4096u);
    return (!narrow || (m->planes.type == kQ4_K && shape.mt == 4u)) ? Route::skinny_loaded : Route::skinny_x;
}

// tactic is already validated; rows >= 1.
Route route_linear(const air_hip_context* ctx, const air_hip_matrix* m, std::uint32_t rows, int tactic) {
    if (m->dense) return Route::dense;   // every tactic and width
    if (tactic == AIR_HIP_LINEAR_PREFILL || (tactic == AIR_HIP_LINEAR_AUTO && rows > AIR_HIP_MAX_DECODE_ROWS)) {
        return Route::prefill;
    }
    if (rows == 1u) return Route::gemv;
    if (rows <= AIR_HIP_MAX_DECODE_ROWS &&
        (ctx->wsplit_mode == 1u ||
         (ctx->wsplit_mode == 0u && ctx->decode_path == 0u && wsplit_preferred(m->planes, rows)))) {
        return Route::wsplit;
    }
    if (rows <= kFusedMaxRows) {
        // Measured on the Qwen2-7B shapes (M = 2..16): the single-launch fused
        // kernel wins for small square matrices (o: N, K <= 4096) and for very
        // large ones at M <= 4; the skinny kernel everywhere else (down, with
        // its long K, by 10-30 %) and for Q4_K (o at M = 16: 25 %).
        const std::uint64_t weight_bytes = static_cast<std::uint64_t>(m->planes.nt) * m->planes.kt *
                                           geometry_of(m->planes.type).code_tile_bytes;
        const bool prefer_fused = m->planes.type != kQ4_K &&
                                  ((m->planes.n <= 4096u && m->planes.k <= 4096u) ||
                                   (rows <= 4u && weight_bytes >= (256ull << 20)));
        if (ctx->decode_path == 2u || (ctx->decode_path == 0u && !prefer_fused)) return skinny_route(ctx, m, rows);
        return Route::fused;
    }
    if (rows <= AIR_HIP_MAX_DECODE_ROWS && ctx->decode_path != 1u) return skinny_route(ctx, m, rows);
    return Route::decode_linear;
}

// Skinny decode linear straight from the f32 rows (M = 2..64): one launch
// (two with a K split), no activation workspace.
int run_skinny_x(air_hip_context* ctx, const air_hip_matrix* m, const float* x, float* y, const float* bias,
                 std::uint32_t rows, const SplitEpilogue* epilogue, bool* applied, const void* ready) {
    const SkinnyShape shape = plan_skinny(m->planes, rows, ctx->skinny_tile_n, ctx->skinny_splits, ctx->skinny_lds_stages,
                                          ctx->skinny_waves);
    if (skinny_route(ctx, m, rows) == Route::skinny_loaded) {
        int rc = load_activations_for(ctx, x, m->planes.k, rows, ready);
        if (rc != AIR_HIP_OK) return rc;
        return linear_loaded(ctx, m, y, bias, AIR_HIP_LINEAR_DECODE, epilogue, applied);
    }
    const std::uint64_t partial_bytes = skinny_partials_bytes(shape, rows, m->planes.n);
    if (partial_bytes > 0u) {
        const int rc = ensure_split_buffers(ctx, partial_bytes, 0u);
        if (rc != AIR_HIP_OK) return rc;
    }
    const SplitEpilogue* epi = reduction_epilogue(ctx, m, shape, bias, rows, epilogue, applied);
    std::uint64_t* chain = epi ? nullptr : chain_for(ctx, shape.splits, rows, m->planes.n);
    const hipError_t err = launch_skinny_linear_x(m->planes, x, bias, y, rows, shape,
                                                  static_cast<float*>(ctx->split_partials), ctx->stream, epi, chain);
    if (err != hipSuccess) return hip_fail(err, "skinny_kernel");
    ctx->decode_linear_calls.fetch_add(1, std::memory_order_relaxed);
    ctx->decode_rows.fetch_add(rows, std::memory_order_relaxed);
    return AIR_HIP_OK;
}

// The wave-split decode linear (M = 2..64): one launch from the f32 rows,
// or from the row-scaled split when the plan asks for it; a K split over
// workgroups adds the deterministic reduction (which may carry `epilogue`).
int run_wsplit(air_hip_context* ctx, const air_hip_matrix* m, const float* x, float* y, const float* bias,
               std::uint32_t rows, const SplitEpilogue* epilogue, bool* applied, const void* ready) {
    const WsplitShape shape = plan_wsplit(m->planes, rows, ctx->wsplit_tuning);
    SplitWorkspace ws{};
    if (shape.split_x) {
        const int rc = load_activations_for(ctx, x, m->planes.k, rows, ready);
        if (rc != AIR_HIP_OK) return rc;
        forget_loaded_source(ctx);
        if (!ctx->loaded_row_scaled) return fail(AIR_HIP_INVALID_STATE, "activations were not split per row");
        ws = carve_split_workspace(ctx->workspace, ceil_div(m->planes.k, kSplitK) * kSplitK, rows);
    }
    const std::uint64_t partial_bytes = wsplit_partials_bytes(shape, rows, m->planes.n);
    if (partial_bytes > 0u) {
        const int rc = ensure_split_buffers(ctx, partial_bytes, 0u);
        if (rc != AIR_HIP_OK) return rc;
    }
    const SplitEpilogue* epi = nullptr;
    if (epilogue && shape.splits >= 2u &&
        split_epilogue_fits(*epilogue, static_cast<const float*>(ctx->split_partials), bias, rows, m->planes.n)) {
        *applied = true;
        epi = epilogue;
    }
    std::uint64_t* chain = epi ? nullptr : chain_for(ctx, shape.splits, rows, m->planes.n);
    const hipError_t err = launch_wsplit_linear(m->planes, x, shape.split_x ? &ws : nullptr, bias, y, rows, shape,
                                                static_cast<float*>(ctx->split_partials), ctx->stream, epi, chain);
    if (err != hipSuccess) return hip_fail(err, "wsplit_kernel");
    ctx->decode_linear_calls.fetch_add(1, std::memory_order_relaxed);
    ctx->decode_rows.fetch_add(rows, std::memory_order_relaxed);
    return AIR_HIP_OK;
}

// Whether the automatic mode sums a K split in the kernel.  Measured per
// linear on the Qwen2-7B shapes (graph replay, all three formats): a 2-way
// split gains 0.2-1.2 us over the reduction launch up to about 230k outputs
// (o at 64 rows) and loses 9 us on gate|up at 32 rows (1.2M outputs); every
// further split adds a level of exchanges that an output passes in turn, so
// 8-way splits gain only at about 50k outputs (down at 2 rows) and lose 3-42
// us beyond.
bool chain_auto(std::uint32_t splits, std::uint32_t m, std::uint64_t n) {
    const std::uint64_t outputs = static_cast<std::uint64_t>(m) * n;
    return (splits == 2u && outputs <= (256u << 10)) || outputs * (splits - 1u) <= (56u << 10);
}

// The chain slots for a K split of `splits` over m x n outputs, or null for
// the reduction launch: the mode asks for it, or the slots would have to grow
// (and be zeroed) while the stream is being captured.
std::uint64_t* chain_for(air_hip_context* ctx, std::uint32_t splits, std::uint32_t m, std::uint64_t n) {
    if (splits < 2u || ctx->chain_mode == 1u) return nullptr;
    if (ctx->chain_mode == 0u && !chain_auto(splits, m, n)) return nullptr;
    const std::uint64_t bytes = chain_slot_bytes(splits, m, n);
    if (bytes <= ctx->chain_slots_bytes) return ctx->chain_slots;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone) {
        return nullptr;
    }
    const std::uint64_t grown = std::max<std::uint64_t>(bytes, ctx->chain_slots_bytes + ctx->chain_slots_bytes / 2);
    void* p = nullptr;
    if (hipMalloc(&p, grown) != hipSuccess) return nullptr;
    if (hipMemsetAsync(p, 0, grown, ctx->stream) != hipSuccess) {
        (void)hipFree(p);
        return nullptr;
    }
    if (ctx->chain_slots) ctx->retired.push_back(ctx->chain_slots);
    ctx->chain_slots = static_cast<std::uint64_t*>(p);
    ctx->chain_slots_bytes = grown;
    ++ctx->generation;
    return ctx->chain_slots;
}

int ensure_split_buffers(air_hip_context* ctx, std::uint64_t partial_bytes, std::uint32_t counters) {
    int rc = grow_buffer(ctx, &ctx->split_partials, &ctx->split_partials_bytes, partial_bytes, "split partials");
    if (rc != AIR_HIP_OK) return rc;
    if (counters > ctx->split_counter_count) {
        // Counters start at zero and every launch leaves them at zero.
        const std::uint32_t count = std::max<std::uint32_t>(counters < 4096u ? 4096u : counters,
                                                            ctx->split_counter_count + ctx->split_counter_count / 2);
        void* p = nullptr;
        hipError_t err = hipMalloc(&p, count * sizeof(std::uint32_t));
        if (err == hipSuccess) err = hipMemset(p, 0, count * sizeof(std::uint32_t));
        if (err != hipSuccess) {
            (void)hipFree(p);
            return hip_fail(err, "hipMalloc(split counters)");
        }
        if (ctx->split_counters) ctx->retired.push_back(ctx->split_counters);
        ctx->split_counters = static_cast<std::uint32_t*>(p);
        ctx->split_counter_count = count;
        ++ctx->generation;
    }
    return AIR_HIP_OK;
}

// A matrix of a dense type (F32, F16, BF16, Q6_K): rows [n][k] in the
// file's own encoding.  F32, F16 and BF16 keep the GGUF rows; Q6_K keeps its
// super-blocks, each padded from 210 to 212 bytes (4-byte aligned words).
// The kernels decode as they load, bit for bit as decode_element
// (cuda_backend.cu:241-344) decodes each element.  k is a multiple of 32
// (256 for Q6_K, its super-block).
int prepare_dense(air_hip_context* ctx, int type, std::uint64_t k, std::uint64_t n, const void* canonical,
                  std::uint64_t canonical_bytes, int bytes_on_device, air_hip_matrix** out) {
    const std::uint64_t expected = air_hip_canonical_bytes(type, k, n);
    if (expected == 0 || canonical_bytes != expected) {
        return fail(AIR_HIP_DATA_ERROR, "canonical size %llu does not match %llu for {%llu, %llu}",
                    static_cast<unsigned long long>(canonical_bytes), static_cast<unsigned long long>(expected),
                    static_cast<unsigned long long>(k), static_cast<unsigned long long>(n));
    }
    if (n > std::numeric_limits<std::uint64_t>::max() / sizeof(float) / k) {
        return fail(AIR_HIP_UNSUPPORTED, "matrix is too large");
    }
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    auto* m = new (std::nothrow) air_hip_matrix();
    if (!m) return fail(AIR_HIP_INTERNAL_ERROR, "out of host memory");
    m->owner = ctx;
    m->type = type;
    m->canonical_bytes = canonical_bytes;
    m->planes.type = type;
    m->planes.k = k;
    m->planes.n = n;
    const int storage = type;
    const std::uint64_t bytes = dense_resident_bytes(storage, k, n);
    if (bytes == 0) return fail(AIR_HIP_UNSUPPORTED, "dense storage of type %d does not fit k = %llu", type,
                                static_cast<unsigned long long>(k));
    void* dense = nullptr;
    hipError_t err = hipMalloc(&dense, bytes);
    if (err != hipSuccess) {
        delete m;
        return hip_fail(err, "hipMalloc(dense rows)");
    }
    const std::uint8_t* src = static_cast<const std::uint8_t*>(canonical);
    void* staging = nullptr;
    if (type != kQ6_K) {
        // The rows as they are (F32 little-endian, F16 / BF16 bits).
        err = hipMemcpyAsync(dense, canonical, canonical_bytes,
                             bytes_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, ctx->stream);
        if (err == hipSuccess && !bytes_on_device) {
            ctx->host_to_device_bytes.fetch_add(canonical_bytes, std::memory_order_relaxed);
        }
    } else {
        if (!bytes_on_device) {
            err = hipMalloc(&staging, canonical_bytes);
            if (err == hipSuccess) {
                err = hipMemcpyAsync(staging, canonical, canonical_bytes, hipMemcpyHostToDevice, ctx->stream);
            }
            if (err == hipSuccess) ctx->host_to_device_bytes.fetch_add(canonical_bytes, std::memory_order_relaxed);
            src = static_cast<const std::uint8_t*>(staging);
        }
        if (err == hipSuccess) err = launch_q6k_records(src, k * n / 256u, dense, ctx->stream);
    }
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    if (staging) {
        if (err != hipSuccess) (void)hipStreamSynchronize(ctx->stream);
        (void)hipFree(staging);
    }
    if (err != hipSuccess) {
        (void)hipFree(dense);
        delete m;
        return hip_fail(err, "dense rows");
    }
    m->dense = dense;
    m->dense_storage = storage;
    if ((storage == kF16 || storage == kBF16 || storage == kQ6_K) && k % 32u == 0u && k <= 0xffffffffu) {
        TilePlanes g{};
        g.type = storage;
        g.k = k;
        g.n = n;
        g.nt = static_cast<std::uint32_t>(ceil_div(n, 16u));
        g.kt = static_cast<std::uint32_t>(k);   // the row length, for the dense loads
        g.kp = ceil_div(k, 64u) * 64u;          // whole 64-k steps
        g.codes = dense;
        if (!ctx->bound_scratch) {
            void* b = nullptr;
            err = hipMalloc(&b, 256);
            ctx->bound_scratch = static_cast<std::uint32_t*>(b);
        }
        if (err == hipSuccess) err = compute_dense_prefill_scale(g, ctx->bound_scratch, ctx->stream);
        if (err != hipSuccess) {
            (void)hipFree(dense);
            delete m;
            return hip_fail(err, "dense prefill scale");
        }
        m->gemm = g;
    }
    m->resident_bytes = bytes;
    ctx->resident_matrix_bytes.fetch_add(bytes, std::memory_order_relaxed);
    ctx->prepared_matrices.fetch_add(1, std::memory_order_relaxed);
    *out = m;
    return AIR_HIP_OK;
}

} // namespace

extern "C" {

int air_hip_abi_version(void) { return AIR_HIP_ABI_VERSION; }

const char* air_hip_status_string(int status) {
    switch (status) {
    case AIR_HIP_OK: return "ok";
    case AIR_HIP_INVALID_ARGUMENT: return "invalid_argument";
    case AIR_HIP_INVALID_STATE: return "invalid_state";
    case AIR_HIP_IO_ERROR: return "io_error";
    case AIR_HIP_CANCELLED: return "cancelled";
    case AIR_HIP_DATA_ERROR: return "data_error";
    case AIR_HIP_UNSUPPORTED: return "unsupported";
    case AIR_HIP_INTERNAL_ERROR: return "internal_error";
    default: return "unknown";
    }
}

const char* air_hip_last_error(void) { return g_last_error.c_str(); }

int air_hip_device_count(int* count) {
    if (!count) return fail(AIR_HIP_INVALID_ARGUMENT, "count must not be null");
    int n = 0;
    const hipError_t err = hipGetDeviceCount(&n);
    if (err == hipErrorNoDevice) { *count = 0; return AIR_HIP_OK; }
    if (err != hipSuccess) return hip_fail(err, "hipGetDeviceCount");
    *count = n;
    return AIR_HIP_OK;
}

int air_hip_mem_info(int device, uint64_t* free_bytes, uint64_t* total_bytes) {
    if (!free_bytes || !total_bytes) return fail(AIR_HIP_INVALID_ARGUMENT, "outputs must not be null");
    DeviceScope scope(device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    std::size_t f = 0, t = 0;
    const hipError_t err = hipMemGetInfo(&f, &t);
    if (err != hipSuccess) return hip_fail(err, "hipMemGetInfo");
    *free_bytes = f;
    *total_bytes = t;
    return AIR_HIP_OK;
}

int air_hip_context_create(int device, void* stream, air_hip_context** out) {
    if (!out) return fail(AIR_HIP_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    int n = 0;
    hipError_t err = hipGetDeviceCount(&n);
    if (err != hipSuccess || n == 0) return fail(AIR_HIP_UNSUPPORTED, "no HIP device is available");
    if (device < 0 || device >= n) return fail(AIR_HIP_INVALID_ARGUMENT, "device %d is out of range", device);
    hipDeviceProp_t prop{};
    err = hipGetDeviceProperties(&prop, device);
    if (err != hipSuccess) return hip_fail(err, "hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        return fail(AIR_HIP_UNSUPPORTED, "device %d is %s; this library is built for gfx950", device, prop.gcnArchName);
    }
    void* scratch_ptr = nullptr;
    void* noalloc_pairs = nullptr;
    void* pairs = nullptr;
    {
        DeviceScope scope(device);
        if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
        if (int rc = noalloc_scratch(device, &scratch_ptr, &noalloc_pairs); rc != AIR_HIP_OK) return rc;
        const std::size_t bytes = kGemvPairSlots * sizeof(std::uint64_t);
        err = hipMalloc(&pairs, bytes);
        if (err != hipSuccess) return hip_fail(err, "hipMalloc (GEMV pair slots)");
        err = hipMemset(pairs, 0, bytes);
        if (err == hipSuccess) err = hipDeviceSynchronize();
        if (err != hipSuccess) {
            (void)hipFree(pairs);
            return hip_fail(err, "hipMemset (GEMV pair slots)");
        }
    }
    auto* ctx = new (std::nothrow) air_hip_context();
    if (!ctx) {
        DeviceScope scope(device);
        (void)hipFree(pairs);
        return fail(AIR_HIP_INTERNAL_ERROR, "out of host memory");
    }
    ctx->device = device;
    ctx->stream = static_cast<hipStream_t>(stream);
    ctx->noalloc_scratch = scratch_ptr;
    ctx->noalloc_pairs = static_cast<std::uint64_t*>(noalloc_pairs);
    ctx->gemv_pairs = static_cast<std::uint64_t*>(pairs);
    ctx->prefill_tuning.cus = static_cast<std::uint32_t>(prop.multiProcessorCount);
    *out = ctx;
    return AIR_HIP_OK;
}

int air_hip_context_destroy(air_hip_context* ctx) {
    if (!ctx) return AIR_HIP_OK;
    {
        DeviceScope scope(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
        if (ctx->workspace) (void)hipFree(ctx->workspace);
        if (ctx->split_partials) (void)hipFree(ctx->split_partials);
        if (ctx->split_counters) (void)hipFree(ctx->split_counters);
        if (ctx->prefill_workspace) (void)hipFree(ctx->prefill_workspace);
        if (ctx->bound_scratch) (void)hipFree(ctx->bound_scratch);
        if (ctx->attention_scratch) (void)hipFree(ctx->attention_scratch);
        if (ctx->argmax_partials) (void)hipFree(ctx->argmax_partials);
        if (ctx->epilogue_rows) (void)hipFree(ctx->epilogue_rows);
        if (ctx->gemv_pairs) (void)hipFree(ctx->gemv_pairs);
        if (ctx->chain_slots) (void)hipFree(ctx->chain_slots);
        for (void* p : ctx->retired) (void)hipFree(p);
    }
    delete ctx;
    return AIR_HIP_OK;
}

int air_hip_context_set_stream(air_hip_context* ctx, void* stream) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    ctx->stream = static_cast<hipStream_t>(stream);
    return AIR_HIP_OK;
}

int air_hip_context_reserve(air_hip_context* ctx, uint64_t max_k, uint32_t max_m) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (max_k == 0 || max_m == 0) return AIR_HIP_OK;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const std::uint64_t kp = ceil_div(max_k, kSplitK) * kSplitK;
    int rc = ensure_workspace(ctx, split_workspace_bytes(kp, max_m < kMaxRows ? max_m : kMaxRows));
    if (rc != AIR_HIP_OK || max_m <= kFusedMaxRows) return rc;
    PrefillShape unsplit{};
    return ensure_prefill_workspace(ctx, prefill_workspace_bytes(max_k, max_m < kMaxRows ? max_m : kMaxRows, unsplit, 0));
}

int air_hip_context_set_decode_path(air_hip_context* ctx, uint32_t path, uint32_t tile_n, uint32_t k_splits) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (path > 2u) return fail(AIR_HIP_INVALID_ARGUMENT, "path must be 0, 1 or 2");
    if (tile_n > 2u) return fail(AIR_HIP_INVALID_ARGUMENT, "tile_n must be 0, 1 or 2");
    if (k_splits > 64u) return fail(AIR_HIP_INVALID_ARGUMENT, "k_splits must be at most 64");
    ctx->decode_path = path;
    ctx->skinny_tile_n = tile_n;
    ctx->skinny_splits = k_splits;
    return AIR_HIP_OK;
}

int air_hip_context_set_wsplit(air_hip_context* ctx, uint32_t mode, uint32_t tile_n, uint32_t waves, uint32_t depth,
                               uint32_t k_splits, uint32_t split_x) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (mode > 2u) return fail(AIR_HIP_INVALID_ARGUMENT, "mode must be 0, 1 or 2");
    if (tile_n != 0u && tile_n != 1u && tile_n != 2u && tile_n != 4u) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "tile_n must be 0, 1, 2 or 4");
    }
    if (waves > 8u) return fail(AIR_HIP_INVALID_ARGUMENT, "waves must be 0 .. 8");
    if (depth != 0u && depth != 2u && depth != 4u) return fail(AIR_HIP_INVALID_ARGUMENT, "depth must be 0, 2 or 4");
    if (k_splits > 64u) return fail(AIR_HIP_INVALID_ARGUMENT, "k_splits must be at most 64");
    if (split_x > 2u) return fail(AIR_HIP_INVALID_ARGUMENT, "split_x must be 0, 1 or 2");
    ctx->wsplit_mode = mode;
    ctx->wsplit_tuning = WsplitTuning{tile_n, waves, depth, k_splits, split_x};
    return AIR_HIP_OK;
}

int air_hip_context_set_dense_path(air_hip_context* ctx, uint32_t path, uint32_t tile_n, uint32_t waves,
                                   uint32_t depth) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (path > 2u) return fail(AIR_HIP_INVALID_ARGUMENT, "path must be 0, 1 or 2");
    if (tile_n != 0u && tile_n != 1u && tile_n != 2u && tile_n != 4u) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "tile_n must be 0, 1, 2 or 4");
    }
    if (waves > 16u) return fail(AIR_HIP_INVALID_ARGUMENT, "waves must be 0 .. 16");
    if (depth != 0u && depth != 2u && depth != 4u) return fail(AIR_HIP_INVALID_ARGUMENT, "depth must be 0, 2 or 4");
    ctx->dense_tuning = DenseTuning{path, DenseMfmaShape{tile_n, waves, depth}};
    return AIR_HIP_OK;
}

int air_hip_context_set_decode_pipeline(air_hip_context* ctx, uint32_t lds_stages) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (lds_stages > 4u) return fail(AIR_HIP_INVALID_ARGUMENT, "lds_stages must be 0 .. 4");
    ctx->skinny_lds_stages = lds_stages;
    return AIR_HIP_OK;
}

int air_hip_context_set_prefill_pipeline(air_hip_context* ctx, uint32_t lds_stages) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (lds_stages > 4u && lds_stages != 0x12u && lds_stages != 0x13u)
        return fail(AIR_HIP_INVALID_ARGUMENT, "lds_stages must be 0 .. 4, 0x12 or 0x13");
    ctx->prefill_tuning.lds_stages = lds_stages;
    return AIR_HIP_OK;
}

int air_hip_context_set_prefill_tuning(air_hip_context* ctx, uint32_t tile_m, uint32_t tile_n, uint32_t k_splits,
                                       uint32_t prefetch) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (tile_m != 0 && tile_m != 4 && tile_m != 8) return fail(AIR_HIP_INVALID_ARGUMENT, "tile_m must be 0, 4 or 8");
    if (tile_n != 0 && tile_n != 2 && tile_n != 4) return fail(AIR_HIP_INVALID_ARGUMENT, "tile_n must be 0, 2 or 4");
    if (k_splits > 64) return fail(AIR_HIP_INVALID_ARGUMENT, "k_splits must be at most 64");
    if (prefetch > 2) return fail(AIR_HIP_INVALID_ARGUMENT, "prefetch must be 0, 1 or 2");
    ctx->prefill_tuning.prefetch = prefetch;
    ctx->prefill_tuning.tile_m = tile_m;
    ctx->prefill_tuning.tile_n = tile_n;
    ctx->prefill_tuning.k_splits = k_splits;
    return AIR_HIP_OK;
}

int air_hip_context_set_prefill_remainder_splits(air_hip_context* ctx, uint32_t splits) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (splits > 64u) return fail(AIR_HIP_INVALID_ARGUMENT, "splits must be at most 64");
    ctx->prefill_tuning.rem_splits = splits;
    return AIR_HIP_OK;
}

int air_hip_context_set_tuning(air_hip_context* ctx, uint32_t rows_per_wave, uint32_t waves_per_group,
                               uint32_t k_splits) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (rows_per_wave != 0 && rows_per_wave != 1 && rows_per_wave != 2 && rows_per_wave != 4) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "rows_per_wave must be 0, 1, 2 or 4");
    }
    if (waves_per_group > 16) return fail(AIR_HIP_INVALID_ARGUMENT, "waves_per_group must be at most 16");
    if (k_splits > 64) return fail(AIR_HIP_INVALID_ARGUMENT, "k_splits must be at most 64");
    ctx->tuning.rows_per_wave = rows_per_wave;
    ctx->tuning.waves_per_group = waves_per_group;
    ctx->tuning.k_splits = k_splits;
    return AIR_HIP_OK;
}

int air_hip_context_set_skinny_waves(air_hip_context* ctx, uint32_t waves) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (waves != 0u && waves != 4u && waves != 8u) return fail(AIR_HIP_INVALID_ARGUMENT, "waves must be 0, 4 or 8");
    ctx->skinny_waves = waves;
    return AIR_HIP_OK;
}

int air_hip_context_set_split_chain(air_hip_context* ctx, uint32_t mode) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (mode > 2u) return fail(AIR_HIP_INVALID_ARGUMENT, "mode must be 0, 1 or 2");
    ctx->chain_mode = mode;
    return AIR_HIP_OK;
}

int air_hip_context_set_gemv_shape(air_hip_context* ctx, uint32_t pair_mode, uint32_t units_per_chunk,
                                   uint32_t depth) {
    if (!ctx) return fail(AIR_HIP_INVALID_ARGUMENT, "context must not be null");
    if (pair_mode > 2u) return fail(AIR_HIP_INVALID_ARGUMENT, "pair_mode must be 0, 1 or 2");
    if (units_per_chunk > 2u) return fail(AIR_HIP_INVALID_ARGUMENT, "units_per_chunk must be 0, 1 or 2");
    if (depth > 2u) return fail(AIR_HIP_INVALID_ARGUMENT, "depth must be 0, 1 or 2");
    ctx->tuning.pair_split = pair_mode;
    ctx->tuning.units_per_chunk = units_per_chunk;
    ctx->tuning.depth = depth;
    return AIR_HIP_OK;
}

int air_hip_context_stats(const air_hip_context* ctx, air_hip_stats* out) {
    if (!ctx || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    out->resident_matrix_bytes = ctx->resident_matrix_bytes.load(std::memory_order_relaxed);
    out->workspace_bytes = ctx->workspace_bytes;
    out->host_to_device_bytes = ctx->host_to_device_bytes.load(std::memory_order_relaxed);
    out->prepared_matrices = ctx->prepared_matrices.load(std::memory_order_relaxed);
    out->decode_linear_calls = ctx->decode_linear_calls.load(std::memory_order_relaxed);
    out->prefill_linear_calls = ctx->prefill_linear_calls.load(std::memory_order_relaxed);
    out->decode_rows = ctx->decode_rows.load(std::memory_order_relaxed);
    out->prefill_rows = ctx->prefill_rows.load(std::memory_order_relaxed);
    out->workspace_generation = ctx->generation;
    return AIR_HIP_OK;
}

int air_hip_stream_read(air_hip_context* ctx, const void* data, uint64_t bytes, uint32_t* sink,
                        uint64_t sink_words) {
    if (!ctx || !data || !sink) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    if (sink_words == 0u) return fail(AIR_HIP_INVALID_ARGUMENT, "the sink needs at least one word");
    if (bytes % 16u != 0u) return fail(AIR_HIP_INVALID_ARGUMENT, "byte count must be a multiple of 16");
    if (reinterpret_cast<std::uintptr_t>(data) % 16u != 0u) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "data must be 16-byte aligned");
    }
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = launch_stream_read(data, bytes, sink, sink_words, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "stream_read_kernel");
}

uint64_t air_hip_canonical_bytes(int type, uint64_t k, uint64_t n) {
    const auto geo = canonical_block(type);
    if (geo.elements == 0 || k % geo.elements != 0) return 0;
    const std::uint64_t blocks = k / geo.elements;
    if (n != 0 && blocks > std::numeric_limits<std::uint64_t>::max() / geo.bytes / n) return 0;
    return blocks * geo.bytes * n;
}

int air_hip_matrix_prepare(air_hip_context* ctx, int type, uint64_t k, uint64_t n,
                           const void* canonical, uint64_t canonical_bytes, int bytes_on_device,
                           air_hip_matrix** out) {
    if (!out) return fail(AIR_HIP_INVALID_ARGUMENT, "out must not be null");
    *out = nullptr;
    if (!ctx || !canonical) return fail(AIR_HIP_INVALID_ARGUMENT, "context and bytes must not be null");
    const auto block = canonical_block(type);
    if (block.elements == 0) return fail(AIR_HIP_UNSUPPORTED, "tensor type %d is not executed by the HIP engine", type);
    if (k == 0 || n == 0) return fail(AIR_HIP_INVALID_ARGUMENT, "matrix dims must be non-zero");
    if (k % block.elements != 0) {
        return fail(AIR_HIP_UNSUPPORTED, "input width %llu is not a multiple of the %u-element block",
                    static_cast<unsigned long long>(k), block.elements);
    }
    if (dense_type(type)) {
        if (k % 32u != 0) {
            return fail(AIR_HIP_UNSUPPORTED, "input width %llu of a dense matrix is not a multiple of 32",
                        static_cast<unsigned long long>(k));
        }
        return prepare_dense(ctx, type, k, n, canonical, canonical_bytes, bytes_on_device, out);
    }
    // Q5_0 runs as Q8_0 (rewritten exactly on the device below).
    const int resident_type = type == kQ5_0 ? static_cast<int>(kQ8_0) : type;
    const auto geo = geometry_of(resident_type);
    const std::uint64_t expected = air_hip_canonical_bytes(type, k, n);
    if (expected == 0 || canonical_bytes != expected) {
        return fail(AIR_HIP_DATA_ERROR, "canonical size %llu does not match %llu for {%llu, %llu}",
                    static_cast<unsigned long long>(canonical_bytes), static_cast<unsigned long long>(expected),
                    static_cast<unsigned long long>(k), static_cast<unsigned long long>(n));
    }
    const std::uint64_t nt64 = ceil_div(n, kTileRows);
    const std::uint64_t kt64 = ceil_div(k, geo.tile_k);
    if (nt64 > std::numeric_limits<std::uint32_t>::max() / 4u || kt64 > std::numeric_limits<std::uint32_t>::max()) {
        return fail(AIR_HIP_UNSUPPORTED, "matrix is too large for the tile grid");
    }

    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");

    auto* m = new (std::nothrow) air_hip_matrix();
    if (!m) return fail(AIR_HIP_INTERNAL_ERROR, "out of host memory");
    m->owner = ctx;
    m->type = type;
    m->canonical_bytes = canonical_bytes;
    TilePlanes& p = m->planes;
    p.type = resident_type;
    p.k = k;
    p.n = n;
    p.nt = static_cast<std::uint32_t>(nt64);
    p.kt = static_cast<std::uint32_t>(kt64);
    p.kp = kt64 * geo.tile_k;
    std::uint64_t scale_bytes = 0;
    const std::uint64_t code_bytes = resident_plane_bytes(p, scale_bytes);

    hipError_t err = hipMalloc(&p.codes, code_bytes);
    if (err == hipSuccess) err = hipMalloc(&p.scales, scale_bytes);
    if (err != hipSuccess) {
        (void)hipFree(p.codes);
        delete m;
        return hip_fail(err, "hipMalloc(resident planes)");
    }

    const std::uint8_t* src = static_cast<const std::uint8_t*>(canonical);
    void* staging = nullptr;
    if (!bytes_on_device) {
        err = hipMalloc(&staging, canonical_bytes);
        if (err == hipSuccess) err = hipMemcpyAsync(staging, canonical, canonical_bytes, hipMemcpyHostToDevice, ctx->stream);
        if (err != hipSuccess) {
            (void)hipFree(staging);
            (void)hipFree(p.codes);
            (void)hipFree(p.scales);
            delete m;
            return hip_fail(err, "upload of canonical bytes");
        }
        src = static_cast<const std::uint8_t*>(staging);
        ctx->host_to_device_bytes.fetch_add(canonical_bytes, std::memory_order_relaxed);
    }
    void* transcoded = nullptr;
    if (type == kQ5_0) {
        const std::uint64_t blocks = canonical_bytes / canonical_block(kQ5_0).bytes;
        err = hipMalloc(&transcoded, blocks * canonical_block(kQ8_0).bytes);
        if (err == hipSuccess) {
            err = launch_q5_0_to_q8_0(src, blocks, static_cast<std::uint8_t*>(transcoded), ctx->stream);
        }
        if (err != hipSuccess) {
            if (transcoded) (void)hipStreamSynchronize(ctx->stream);
            (void)hipFree(transcoded);
            if (staging) (void)hipFree(staging);
            (void)hipFree(p.codes);
            (void)hipFree(p.scales);
            delete m;
            return hip_fail(err, "Q5_0 -> Q8_0");
        }
        src = static_cast<const std::uint8_t*>(transcoded);
    }
    err = launch_repack(p, src, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
    if (staging) (void)hipFree(staging);
    if (transcoded) (void)hipFree(transcoded);
    if (err == hipSuccess && !ctx->bound_scratch) {
        void* b = nullptr;
        err = hipMalloc(&b, 256);
        ctx->bound_scratch = static_cast<std::uint32_t*>(b);
    }
    if (err == hipSuccess) err = compute_prefill_scale(p, ctx->bound_scratch, ctx->stream);
    if (err != hipSuccess) {
        (void)hipFree(p.codes);
        (void)hipFree(p.scales);
        delete m;
        return hip_fail(err, "repack");
    }
    m->resident_bytes = code_bytes + scale_bytes;
    ctx->resident_matrix_bytes.fetch_add(m->resident_bytes, std::memory_order_relaxed);
    ctx->prepared_matrices.fetch_add(1, std::memory_order_relaxed);
    *out = m;
    return AIR_HIP_OK;
}

int air_hip_matrix_release(air_hip_matrix* m) {
    if (!m) return AIR_HIP_OK;
    {
        DeviceScope scope(m->owner->device);
        (void)hipStreamSynchronize(m->owner->stream);
        (void)hipFree(m->planes.codes);
        (void)hipFree(m->planes.scales);
        (void)hipFree(m->dense);
    }
    m->owner->resident_matrix_bytes.fetch_sub(m->resident_bytes, std::memory_order_relaxed);
    delete m;
    return AIR_HIP_OK;
}

int air_hip_matrix_describe(const air_hip_matrix* m, air_hip_matrix_desc* out) {
    if (!m || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    out->type = m->type;
    out->device = m->owner->device;
    out->k = m->planes.k;
    out->n = m->planes.n;
    out->canonical_bytes = m->canonical_bytes;
    out->resident_bytes = m->resident_bytes;
    return AIR_HIP_OK;
}

int air_hip_matrix_dequantize(air_hip_context* ctx, const air_hip_matrix* m, float* out) {
    if (!ctx || !m || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (m->owner->device != ctx->device) return fail(AIR_HIP_INVALID_ARGUMENT, "matrix belongs to another device");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    if (m->dense) {
        const std::uint64_t elements = m->planes.k * m->planes.n;
        const hipError_t err =
            m->dense_storage == kF32
                ? hipMemcpyAsync(out, m->dense, elements * sizeof(float), hipMemcpyDeviceToDevice, ctx->stream)
                : launch_dense_dequantize(m->dense, m->dense_storage, m->planes.k, m->planes.n, out, ctx->stream);
        return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "decode of dense rows");
    }
    const hipError_t err = launch_dequantize_tiles(m->planes, out, ctx->stream);
    if (err != hipSuccess) return hip_fail(err, "dequantize_tiles_kernel");
    return AIR_HIP_OK;
}

int air_hip_dequantize_canonical(air_hip_context* ctx, int type, const void* canonical,
                                 uint64_t canonical_bytes, uint64_t elements, float* out) {
    if (!ctx || !canonical || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    const auto geo = canonical_block(type);
    if (geo.elements == 0) return fail(AIR_HIP_UNSUPPORTED, "tensor type %d is not decoded by the HIP engine", type);
    if (elements % geo.elements != 0 || canonical_bytes != (elements / geo.elements) * geo.bytes) {
        return fail(AIR_HIP_DATA_ERROR, "canonical storage geometry mismatch");
    }
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = launch_dequantize_canonical(type, static_cast<const std::uint8_t*>(canonical),
                                                       elements, out, ctx->stream);
    if (err != hipSuccess) return hip_fail(err, "dequantize_canonical_kernel");
    return AIR_HIP_OK;
}

int air_hip_decode_linear_fused(air_hip_context* ctx, const air_hip_matrix* m, const float* x, float* y,
                                const float* bias, const float* norm_weight, double eps, int epilogue) {
    const LinearRange range(1u);
    if (!ctx || !m || !x || !y) return fail(AIR_HIP_INVALID_ARGUMENT, "context, matrix, x and y must not be null");
    forget_loaded_source(ctx);
    if (static_cast<const void*>(x) == static_cast<const void*>(y)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "y must not alias x");
    }
    if (epilogue != AIR_HIP_EPILOGUE_STORE && epilogue != AIR_HIP_EPILOGUE_RESIDUAL &&
        epilogue != AIR_HIP_EPILOGUE_SWIGLU) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "unknown epilogue %d", epilogue);
    }
    const bool norm = norm_weight != nullptr;
    if (norm && epilogue == AIR_HIP_EPILOGUE_RESIDUAL) {
        return fail(AIR_HIP_UNSUPPORTED, "this norm / epilogue combination is not provided");
    }
    if (norm && !(eps >= 0.0)) return fail(AIR_HIP_INVALID_ARGUMENT, "eps must be non-negative");
    if (m->dense) return fail(AIR_HIP_UNSUPPORTED, "the fused decode GEMV runs the quantized tile formats only");
    if (epilogue == AIR_HIP_EPILOGUE_SWIGLU && m->planes.n % 32u != 0u) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "a fused gate|up matrix needs n = 2F with F a multiple of 16");
    }
    if (m->owner->device != ctx->device) return fail(AIR_HIP_INVALID_ARGUMENT, "matrix belongs to another device");
    if (reinterpret_cast<std::uintptr_t>(x) % 16u != 0 ||
        (norm && reinterpret_cast<std::uintptr_t>(norm_weight) % 16u != 0)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "x and the norm weight must be 16-byte aligned");
    }
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const GemvShape shape = plan_decode_gemv_fused(m->planes, ctx->tuning, epilogue);
    const hipError_t err = launch_decode_gemv_fused(m->planes, x, bias, y, shape,
                                                    GemvFusion{norm_weight, eps, epilogue}, ctx->gemv_pairs,
                                                    ctx->stream);
    if (err != hipSuccess) return hip_fail(err, "decode_gemv_kernel (fused)");
    ctx->decode_linear_calls.fetch_add(1, std::memory_order_relaxed);
    ctx->decode_rows.fetch_add(1, std::memory_order_relaxed);
    return AIR_HIP_OK;
}

int air_hip_activations_load(air_hip_context* ctx, const float* x, uint64_t k, uint32_t rows) {
    if (!ctx || !x) return fail(AIR_HIP_INVALID_ARGUMENT, "context and x must not be null");
    if (rows == 0) return fail(AIR_HIP_INVALID_ARGUMENT, "linear batch width must be non-zero");
    if (rows > kMaxRows) return fail(AIR_HIP_UNSUPPORTED, "linear batch width %u exceeds %u", rows, kMaxRows);
    if (k == 0 || k % 32u != 0) return fail(AIR_HIP_UNSUPPORTED, "input width must be a non-zero multiple of 32");
    if (reinterpret_cast<std::uintptr_t>(x) % 16u != 0) return fail(AIR_HIP_INVALID_ARGUMENT, "x must be 16-byte aligned");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const std::uint64_t kp = ceil_div(k, kSplitK) * kSplitK;
    int rc = ensure_workspace(ctx, split_workspace_bytes(kp, rows));
    if (rc != AIR_HIP_OK) return rc;
    const SplitWorkspace ws = carve_split_workspace(ctx->workspace, kp, rows);
    // The skinny kernel (M <= 64) takes one scale per row, the K-split
    // kernel one per (row, block).
    const bool row_scaled = rows <= AIR_HIP_MAX_DECODE_ROWS && ctx->decode_path != 1u;
    const hipError_t err = row_scaled ? launch_split_activations_rows(x, rows, k, kp, ws, ctx->stream)
                                      : launch_split_activations(x, rows, k, kp, ws, ctx->stream);
    if (err != hipSuccess) return hip_fail(err, "split_activations_kernel");
    ctx->loaded_k = k;
    ctx->loaded_rows = rows;
    ctx->loaded_row_scaled = row_scaled;
    forget_loaded_source(ctx);
    return AIR_HIP_OK;
}

int air_hip_linear_loaded(air_hip_context* ctx, const air_hip_matrix* m, float* y, const float* bias, int tactic) {
    return linear_loaded(ctx, m, y, bias, tactic, nullptr, nullptr);
}

} // extern "C"

namespace {

int linear_loaded(air_hip_context* ctx, const air_hip_matrix* m, float* y, const float* bias, int tactic,
                  const SplitEpilogue* epilogue, bool* applied) {
    if (!ctx || !m || !y) return fail(AIR_HIP_INVALID_ARGUMENT, "context, matrix and y must not be null");
    forget_loaded_source(ctx);
    if (m->owner->device != ctx->device) return fail(AIR_HIP_INVALID_ARGUMENT, "matrix belongs to another device");
    if (tactic != AIR_HIP_LINEAR_AUTO && tactic != AIR_HIP_LINEAR_DECODE && tactic != AIR_HIP_LINEAR_PREFILL) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "unknown linear tactic %d", tactic);
    }
    if (tactic == AIR_HIP_LINEAR_PREFILL) {
        return fail(AIR_HIP_UNSUPPORTED, "the prefill tactic runs through air_hip_linear, not loaded activations");
    }
    if (m->dense) return fail(AIR_HIP_UNSUPPORTED, "a dense matrix takes f32 rows through air_hip_linear");
    if (ctx->loaded_rows == 0) return fail(AIR_HIP_INVALID_STATE, "no activations are loaded in this context");
    if (ctx->loaded_k != m->planes.k) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "loaded activations have width %llu, matrix expects %llu",
                    static_cast<unsigned long long>(ctx->loaded_k), static_cast<unsigned long long>(m->planes.k));
    }
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const std::uint32_t rows = ctx->loaded_rows;
    const std::uint64_t kp = ceil_div(ctx->loaded_k, kSplitK) * kSplitK;
    const SplitWorkspace ws = carve_split_workspace(ctx->workspace, kp, rows);
    const bool skinny = rows <= AIR_HIP_MAX_DECODE_ROWS && ctx->decode_path != 1u;
    if (skinny != ctx->loaded_row_scaled) {
        return fail(AIR_HIP_INVALID_STATE, "activations were loaded for another decode path; load them again");
    }
    if (skinny) {
        const SkinnyShape shape = plan_skinny(m->planes, rows, ctx->skinny_tile_n, ctx->skinny_splits, ctx->skinny_lds_stages,
                                          ctx->skinny_waves);
        const std::uint64_t partial_bytes = skinny_partials_bytes(shape, rows, m->planes.n);
        if (partial_bytes > 0u) {
            const int rc = ensure_split_buffers(ctx, partial_bytes, 0u);
            if (rc != AIR_HIP_OK) return rc;
        }
        const SplitEpilogue* epi = reduction_epilogue(ctx, m, shape, bias, rows, epilogue, applied);
        std::uint64_t* chain = epi ? nullptr : chain_for(ctx, shape.splits, rows, m->planes.n);
        const hipError_t err = launch_skinny_linear(m->planes, ws, bias, y, rows, shape,
                                                    static_cast<float*>(ctx->split_partials), ctx->stream, epi, chain);
        if (err != hipSuccess) return hip_fail(err, "skinny_kernel");
        ctx->decode_linear_calls.fetch_add(1, std::memory_order_relaxed);
        ctx->decode_rows.fetch_add(rows, std::memory_order_relaxed);
        return AIR_HIP_OK;
    }
    const hipError_t err = launch_decode_linear(m->planes, ws, bias, y, rows, ctx->tuning, ctx->stream);
    if (err != hipSuccess) return hip_fail(err, "decode_linear_kernel");
    ctx->decode_linear_calls.fetch_add(1, std::memory_order_relaxed);
    ctx->decode_rows.fetch_add(rows, std::memory_order_relaxed);
    return AIR_HIP_OK;
}

// air_hip_linear; with `epilogue`, a skinny launch with a K split applies it
// in its reduction (*applied set, y not written).
int linear_rows(air_hip_context* ctx, const air_hip_matrix* m, const float* x, float* y, const float* bias,
                uint32_t rows, int tactic, const SplitEpilogue* epilogue, bool* applied) {
    const void* ready = ctx ? ctx->loaded_source : nullptr;  // good for this call only
    const void* prefill_ready = ctx ? ctx->prefill_source : nullptr;
    if (ctx) forget_loaded_source(ctx);
    if (!ctx || !m || !x || !y) return fail(AIR_HIP_INVALID_ARGUMENT, "context, matrix, x and y must not be null");
    if (static_cast<const void*>(x) == static_cast<const void*>(y)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "y must not alias x");
    }
    if (tactic != AIR_HIP_LINEAR_AUTO && tactic != AIR_HIP_LINEAR_DECODE && tactic != AIR_HIP_LINEAR_PREFILL) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "unknown linear tactic %d", tactic);
    }
    if (m->owner->device != ctx->device) return fail(AIR_HIP_INVALID_ARGUMENT, "matrix belongs to another device");
    if (rows == 0) return fail(AIR_HIP_INVALID_ARGUMENT, "linear batch width must be non-zero");
    const Route route = route_linear(ctx, m, rows, tactic);
    if (route == Route::dense) {
        if (reinterpret_cast<std::uintptr_t>(x) % 16u != 0) return fail(AIR_HIP_INVALID_ARGUMENT, "x must be 16-byte aligned");
        DeviceScope scope(ctx->device);
        if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
        if (dense_prefill(ctx, m, rows, tactic)) {
            return run_prefill(ctx, m, x, y, bias, rows, prefill_ready, ctx->prefill_source_k, ctx->prefill_source_rows,
                               epilogue, applied);
        }
        const hipError_t err = launch_dense_linear(m->dense, m->dense_storage, m->planes.k, m->planes.n, x, bias, y, rows,
                                                     ctx->stream, ctx->dense_tuning);
        if (err != hipSuccess) return hip_fail(err, "dense_rows_kernel / dense_gemm_kernel");
        const bool prefill = tactic == AIR_HIP_LINEAR_PREFILL ||
                             (tactic == AIR_HIP_LINEAR_AUTO && rows > AIR_HIP_MAX_DECODE_ROWS);
        (prefill ? ctx->prefill_linear_calls : ctx->decode_linear_calls).fetch_add(1, std::memory_order_relaxed);
        (prefill ? ctx->prefill_rows : ctx->decode_rows).fetch_add(rows, std::memory_order_relaxed);
        return AIR_HIP_OK;
    }
    if (route == Route::prefill) {
        if (rows > kMaxRows) return fail(AIR_HIP_UNSUPPORTED, "linear batch width %u exceeds %u", rows, kMaxRows);
        if (reinterpret_cast<std::uintptr_t>(x) % 16u != 0) return fail(AIR_HIP_INVALID_ARGUMENT, "x must be 16-byte aligned");
        DeviceScope scope(ctx->device);
        if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
        return run_prefill(ctx, m, x, y, bias, rows, prefill_ready, ctx->prefill_source_k, ctx->prefill_source_rows,
                           epilogue, applied);
    }
    if (route == Route::decode_linear) {
        int rc = load_activations_for(ctx, x, m->planes.k, rows, ready);
        if (rc != AIR_HIP_OK) return rc;
        return linear_loaded(ctx, m, y, bias, tactic, epilogue, applied);
    }
    // The single-launch routes split the activations in registers.
    if (reinterpret_cast<std::uintptr_t>(x) % 16u != 0) return fail(AIR_HIP_INVALID_ARGUMENT, "x must be 16-byte aligned");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    if (route == Route::gemv) {
        const GemvShape gshape = plan_decode_gemv(m->planes, ctx->tuning);
        const hipError_t gerr = launch_decode_gemv(m->planes, x, bias, y, gshape, ctx->gemv_pairs, ctx->stream);
        if (gerr != hipSuccess) return hip_fail(gerr, "decode_gemv_kernel");
        ctx->decode_linear_calls.fetch_add(1, std::memory_order_relaxed);
        ctx->decode_rows.fetch_add(1, std::memory_order_relaxed);
        return AIR_HIP_OK;
    }
    if (route == Route::skinny_x || route == Route::skinny_loaded) {
        return run_skinny_x(ctx, m, x, y, bias, rows, epilogue, applied, ready);
    }
    if (route == Route::wsplit) return run_wsplit(ctx, m, x, y, bias, rows, epilogue, applied, ready);
    const FusedShape shape = plan_decode_fused(m->planes, rows, ctx->tuning);
    if (shape.k_splits > 1u) {
        const int rc = ensure_split_buffers(ctx, fused_split_workspace_bytes(shape), shape.groups);
        if (rc != AIR_HIP_OK) return rc;
    }
    const hipError_t err = launch_decode_fused(m->planes, x, bias, y, rows, shape, ctx->split_partials,
                                               ctx->split_counters, ctx->stream);
    if (err != hipSuccess) return hip_fail(err, "decode_fused_kernel");
    ctx->decode_linear_calls.fetch_add(1, std::memory_order_relaxed);
    ctx->decode_rows.fetch_add(rows, std::memory_order_relaxed);
    return AIR_HIP_OK;
}

// How a plain linear's K split of `splits` workgroups is summed.
const char* split_tail(const air_hip_context* ctx, std::uint32_t splits, std::uint32_t m, std::uint64_t n) {
    if (splits < 2u) return "";
    const bool chain = ctx->chain_mode == 2u || (ctx->chain_mode == 0u && chain_auto(splits, m, n));
    return chain ? " + in-kernel chain" : " + split reduction";
}

// Text description of the launches of a linear (air_hip_linear_plan).
std::string describe_linear(const air_hip_context* ctx, const air_hip_matrix* m, std::uint32_t rows, int tactic) {
    const char* fmt = m->planes.type == kQ8_0 ? (m->type == kQ5_0 ? "q8_0 from q5_0" : "q8_0")
                      : m->planes.type == kQ4_0 ? "q4_0" : "q4_k";
    char buf[256];
    switch (route_linear(ctx, m, rows, tactic)) {
    case Route::dense: {
        const char* t = m->type == kF32 ? "f32" : m->type == kF16 ? "f16" : m->type == kBF16 ? "bf16" : "q6_k";
        if (dense_prefill(ctx, m, rows, tactic)) {
            const PrefillShape s = plan_prefill(m->gemm, rows, ctx->prefill_tuning);
            std::snprintf(buf, sizeof buf, "%s<%s> tile_m=%u tile_n=%u prefetch=%u m_tiles=%u "
                          "groups=%u splits=%u (dense %s %s)", s.hybrid ? "prefill_hyb_kernel" : "prefill_gemm_kernel",
                          t, s.tile_m, s.tile_n, s.prefetch, s.m_tiles, s.groups,
                          s.splits, t, m->type == kQ6_K ? "super-block rows" : "rows");
            if (s.rem_groups) {
                const std::size_t used = std::strlen(buf);
                std::snprintf(buf + used, sizeof buf - used, " + remainder tile_m=4 tile_n=2 m_tiles=%u groups=%u splits=%u",
                              s.rem_m_tiles, s.rem_groups, s.rem_splits);
            }
            break;
        }
        if (m->type == kQ6_K && rows == 1u && ctx->dense_tuning.path == 0u) {
            const Q6kGemvPlan g = plan_q6k_gemv(m->planes.k, m->planes.n, ctx->dense_tuning.shape);
            std::snprintf(buf, sizeof buf, "q6k_gemv_kernel waves=%u units=%u depth=%u (dense q6_k super-block rows)",
                          g.waves, g.units, g.depth);
            break;
        }
        if (dense_mfma_route(m->dense_storage, m->planes.k, m->planes.n, rows, ctx->dense_tuning)) {
            const DenseMfmaShape d = plan_dense_mfma(m->dense_storage, m->planes.k, m->planes.n, rows,
                                                     ctx->dense_tuning.shape);
            std::snprintf(buf, sizeof buf, "dense_mfma_kernel<%s> tile_n=%u waves=%u depth=%u launches=%u (dense %s %s)",
                          t, d.tile_n, d.waves, d.depth,
                          static_cast<unsigned>(ceil_div(rows, dense_mfma_rows(m->dense_storage))), t,
                          m->type == kQ6_K ? "super-block rows" : "rows");
            break;
        }
        std::snprintf(buf, sizeof buf, m->type == kQ6_K ? "%s (dense %s super-block rows)" : "%s (dense %s rows)",
                      rows <= 64u ? "dense_rows_kernel" : "dense_gemm_kernel tile=64x64", t);
        break;
    }
    case Route::prefill: {
        const PrefillShape s = plan_prefill(m->planes, rows, ctx->prefill_tuning);
        if (s.hybrid) {
            std::snprintf(buf, sizeof buf, "prefill_hyb_kernel<%s> tile_m=%u tile_n=%u stages=%u m_tiles=%u groups=%u "
                          "splits=%u", fmt, s.tile_m, s.tile_n, s.hybrid, s.m_tiles, s.groups, s.splits);
        } else if (s.lds_stages) {
            std::snprintf(buf, sizeof buf, "prefill_lds_kernel<%s> tile_m=%u tile_n=%u stages=%u m_tiles=%u groups=%u "
                          "splits=%u", fmt, s.tile_m, s.tile_n, s.lds_stages, s.m_tiles, s.groups, s.splits);
        } else {
            std::snprintf(buf, sizeof buf, "prefill_gemm_kernel<%s> tile_m=%u tile_n=%u prefetch=%u m_tiles=%u "
                          "groups=%u splits=%u", fmt, s.tile_m, s.tile_n, s.prefetch, s.m_tiles, s.groups, s.splits);
        }
        if (s.rem_groups) {
            const std::size_t used = std::strlen(buf);
            std::snprintf(buf + used, sizeof buf - used, " + remainder tile_m=4 tile_n=2 m_tiles=%u groups=%u splits=%u",
                          s.rem_m_tiles, s.rem_groups, s.rem_splits);
        }
        break;
    }
    case Route::gemv: {
        const GemvShape g = plan_decode_gemv(m->planes, ctx->tuning);
        std::snprintf(buf, sizeof buf, "decode_gemv_kernel<%s> rows_per_wave=%u depth=%u units_per_chunk=%u "
                      "waves=%u groups=%u%s", fmt, g.rows_per_wave, g.depth, g.units_per_chunk, g.waves_per_group,
                      static_cast<unsigned>(ceil_div(m->planes.nt, g.rows_per_wave)),
                      g.pair_split ? " pair_split" : "");
        break;
    }
    case Route::fused: {
        const FusedShape f = plan_decode_fused(m->planes, rows, ctx->tuning);
        std::snprintf(buf, sizeof buf, "decode_fused_kernel<%s> rows_per_wave=%u waves=%u k_splits=%u groups=%u", fmt,
                      f.rows_per_wave, f.waves_per_group, f.k_splits, f.groups);
        break;
    }
    case Route::skinny_x:
    case Route::skinny_loaded: {
        const bool loaded = route_linear(ctx, m, rows, tactic) == Route::skinny_loaded;
        const SkinnyShape k = plan_skinny(m->planes, rows, ctx->skinny_tile_n, ctx->skinny_splits, ctx->skinny_lds_stages,
                                          ctx->skinny_waves);
        const bool lds = loaded && k.lds_stages >= 2u;
        char stages[32] = "";
        if (lds) std::snprintf(stages, sizeof stages, " lds_stages=%u%s", k.lds_stages, k.waves == 8u ? " waves=8" : "");
        std::snprintf(buf, sizeof buf, "%s%s<%s%s> mt=%u tile_n=%u groups=%u splits=%u%s%s",
                      loaded ? "split_rows_kernel + " : "", lds ? "skinny_lds_kernel" : "skinny_kernel", fmt,
                      loaded ? "" : ", f32 input", k.mt, k.tile_n, k.groups, k.splits, stages,
                      split_tail(ctx, k.splits, rows, m->planes.n));
        break;
    }
    case Route::decode_linear:
        std::snprintf(buf, sizeof buf, "split_activations_kernel + decode_linear_kernel<%s>", fmt);
        break;
    case Route::wsplit: {
        const WsplitShape w = plan_wsplit(m->planes, rows, ctx->wsplit_tuning);
        std::snprintf(buf, sizeof buf, "%swsplit_kernel<%s%s> mt=%u tile_n=%u waves=%u depth=%u groups=%u splits=%u%s",
                      w.split_x ? "split_rows_kernel + " : "", fmt, w.split_x ? "" : ", f32 input", w.mt, w.tile_n,
                      w.waves, w.depth, w.groups, w.splits, split_tail(ctx, w.splits, rows, m->planes.n));
        break;
    }
    }
    return buf;
}

} // namespace

extern "C" {

int air_hip_linear(air_hip_context* ctx, const air_hip_matrix* m, const float* x, float* y,
                   const float* bias, uint32_t rows, int tactic) {
    const LinearRange range(rows);
    return linear_rows(ctx, m, x, y, bias, rows, tactic, nullptr, nullptr);
}

int air_hip_linear_noalloc(air_hip_context* ctx, const air_hip_matrix* m, const float* x, float* y, const float* bias,
                           uint32_t rows, int tactic) {
    if (!ctx || !m || !x || !y) return fail(AIR_HIP_INVALID_ARGUMENT, "context, matrix, x and y must not be null");
    forget_loaded_source(ctx);
    if (static_cast<const void*>(x) == static_cast<const void*>(y)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "y must not alias x");
    }
    if (tactic != AIR_HIP_LINEAR_AUTO && tactic != AIR_HIP_LINEAR_DECODE) {
        return fail(tactic == AIR_HIP_LINEAR_PREFILL ? AIR_HIP_UNSUPPORTED : AIR_HIP_INVALID_ARGUMENT,
                    "the no-allocation linear runs the decode tactic only (tactic %d)", tactic);
    }
    if (rows == 0) return fail(AIR_HIP_INVALID_ARGUMENT, "linear batch width must be non-zero");
    if (rows > AIR_HIP_MAX_DECODE_ROWS) {
        return fail(AIR_HIP_UNSUPPORTED, "the no-allocation linear covers decode widths up to %u, not %u",
                    AIR_HIP_MAX_DECODE_ROWS, rows);
    }
    if (m->owner->device != ctx->device) return fail(AIR_HIP_INVALID_ARGUMENT, "matrix belongs to another device");
    if (reinterpret_cast<std::uintptr_t>(x) % 16u != 0) return fail(AIR_HIP_INVALID_ARGUMENT, "x must be 16-byte aligned");
    if (m->dense) {   // no scratch: the same launch as air_hip_linear
        DeviceScope scope(ctx->device);
        if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
        const hipError_t err = launch_dense_linear(m->dense, m->dense_storage, m->planes.k, m->planes.n, x, bias, y, rows,
                                                     ctx->stream, ctx->dense_tuning);
        if (err != hipSuccess) return hip_fail(err, "dense_rows_kernel / dense_gemm_kernel");
        ctx->decode_linear_calls.fetch_add(1, std::memory_order_relaxed);
        ctx->decode_rows.fetch_add(rows, std::memory_order_relaxed);
        return AIR_HIP_OK;
    }
    if (!ctx->noalloc_scratch) return fail(AIR_HIP_INTERNAL_ERROR, "the device scratch array is not mapped");
    // Same route, plans and kernels as air_hip_linear with this context's
    // settings, so the results are bit-identical; only the buffers differ:
    // the split activations at the start of the scratch array, the K-split
    // partials after them (256-byte aligned).  Each launch writes every
    // scratch byte it later reads, so nothing needs clearing between calls.
    const Route route = route_linear(ctx, m, rows, tactic);
    const TilePlanes& p = m->planes;
    const std::uint64_t kp = ceil_div(p.k, kSplitK) * kSplitK;
    std::uint64_t ws_bytes = 0, partial_bytes = 0;
    SkinnyShape shape{};
    WsplitShape wshape{};
    if (route == Route::skinny_x || route == Route::skinny_loaded) {
        shape = plan_skinny(p, rows, ctx->skinny_tile_n, ctx->skinny_splits, ctx->skinny_lds_stages,
                                          ctx->skinny_waves);
        partial_bytes = skinny_partials_bytes(shape, rows, p.n);
    }
    if (route == Route::wsplit) {
        wshape = plan_wsplit(p, rows, ctx->wsplit_tuning);
        partial_bytes = wsplit_partials_bytes(wshape, rows, p.n);
    }
    if (route == Route::skinny_loaded || route == Route::decode_linear || (route == Route::wsplit && wshape.split_x)) {
        ws_bytes = ceil_div(split_workspace_bytes(kp, rows), 256u) * 256u;
    }
    if (route == Route::fused && plan_decode_fused(p, rows, ctx->tuning).k_splits > 1u) {
        return fail(AIR_HIP_UNSUPPORTED, "the no-allocation linear does not run the fused kernel's cross-workgroup "
                    "K split (a context tuning override)");
    }
    if (ws_bytes + partial_bytes > kNoAllocScratchBytes) {
        return fail(AIR_HIP_UNSUPPORTED, "this linear needs %llu bytes of scratch; the no-allocation array holds %llu",
                    static_cast<unsigned long long>(ws_bytes + partial_bytes),
                    static_cast<unsigned long long>(kNoAllocScratchBytes));
    }
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    auto* base = static_cast<unsigned char*>(ctx->noalloc_scratch);
    float* partials = reinterpret_cast<float*>(base + ws_bytes);
    const SplitWorkspace ws = carve_split_workspace(base, kp, rows);
    hipError_t err = hipSuccess;
    switch (route) {
    case Route::gemv:
        err = launch_decode_gemv(p, x, bias, y, plan_decode_gemv(p, ctx->tuning), ctx->noalloc_pairs, ctx->stream);
        break;
    case Route::fused:
        err = launch_decode_fused(p, x, bias, y, rows, plan_decode_fused(p, rows, ctx->tuning), nullptr, nullptr,
                                  ctx->stream);
        break;
    case Route::skinny_x:
        err = launch_skinny_linear_x(p, x, bias, y, rows, shape, partials, ctx->stream);
        break;
    case Route::skinny_loaded:
        err = launch_split_activations_rows(x, rows, p.k, kp, ws, ctx->stream);
        if (err == hipSuccess) err = launch_skinny_linear(p, ws, bias, y, rows, shape, partials, ctx->stream);
        break;
    case Route::wsplit:
        if (wshape.split_x) err = launch_split_activations_rows(x, rows, p.k, kp, ws, ctx->stream);
        if (err == hipSuccess) {
            err = launch_wsplit_linear(p, x, wshape.split_x ? &ws : nullptr, bias, y, rows, wshape, partials,
                                       ctx->stream);
        }
        break;
    case Route::decode_linear:
        err = launch_split_activations(x, rows, p.k, kp, ws, ctx->stream);
        if (err == hipSuccess) err = launch_decode_linear(p, ws, bias, y, rows, ctx->tuning, ctx->stream);
        break;
    case Route::prefill:
    case Route::dense:
        return fail(AIR_HIP_UNSUPPORTED, "the no-allocation linear runs the decode tactic only");
    }
    if (err != hipSuccess) return hip_fail(err, "no-allocation decode linear");
    ctx->decode_linear_calls.fetch_add(1, std::memory_order_relaxed);
    ctx->decode_rows.fetch_add(rows, std::memory_order_relaxed);
    return AIR_HIP_OK;
}

int air_hip_linear_plan(const air_hip_context* ctx, const air_hip_matrix* m, uint32_t rows, int tactic, char* text,
                        uint64_t capacity) {
    if (!ctx || !m || !text || capacity == 0) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "context, matrix and text must not be null, capacity non-zero");
    }
    if (tactic != AIR_HIP_LINEAR_AUTO && tactic != AIR_HIP_LINEAR_DECODE && tactic != AIR_HIP_LINEAR_PREFILL) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "unknown linear tactic %d", tactic);
    }
    if (rows == 0) return fail(AIR_HIP_INVALID_ARGUMENT, "linear batch width must be non-zero");
    const std::string d = describe_linear(ctx, m, rows, tactic);
    const std::size_t n = std::min<std::size_t>(d.size(), capacity - 1u);
    std::memcpy(text, d.data(), n);
    text[n] = '\0';
    return AIR_HIP_OK;
}

int air_hip_linear_epilogue(air_hip_context* ctx, const air_hip_matrix* m, const float* x, uint32_t rows, float* out,
                            const float* bias, int epilogue, const float* norm_weight, float* norm_out, double eps,
                            int tactic) {
    const LinearRange range(rows);
    if (!ctx || !m || !x || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "context, matrix, x and out must not be null");
    if (epilogue != AIR_HIP_EPILOGUE_RESIDUAL && epilogue != AIR_HIP_EPILOGUE_SWIGLU &&
        epilogue != AIR_HIP_EPILOGUE_RESIDUAL_LOAD && epilogue != AIR_HIP_EPILOGUE_RESIDUAL_PREFILL) {
        return fail(AIR_HIP_INVALID_ARGUMENT,
                    "epilogue must be RESIDUAL, SWIGLU, RESIDUAL_LOAD or RESIDUAL_PREFILL, not %d", epilogue);
    }
    const bool load = epilogue == AIR_HIP_EPILOGUE_RESIDUAL_LOAD;
    const bool prefill_out = epilogue == AIR_HIP_EPILOGUE_RESIDUAL_PREFILL;
    if (load && (!norm_weight || m->planes.n % 32u != 0u)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "RESIDUAL_LOAD needs a norm and an output width that is a multiple of 32");
    }
    if (prefill_out && !norm_weight) return fail(AIR_HIP_INVALID_ARGUMENT, "RESIDUAL_PREFILL needs a norm");
    if (static_cast<const void*>(x) == static_cast<const void*>(out)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "out must not alias x");
    }
    if (epilogue == AIR_HIP_EPILOGUE_SWIGLU && (norm_weight || m->planes.n % 2u != 0u)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "SWIGLU takes a fused gate|up matrix (even n) and no norm");
    }
    if (norm_weight && (!norm_out || norm_out == out || !(eps >= 0.0))) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "a norm needs its own output and a non-negative eps");
    }
    if (rows == 0) return fail(AIR_HIP_INVALID_ARGUMENT, "linear batch width must be non-zero");
    if (m->owner->device != ctx->device) return fail(AIR_HIP_INVALID_ARGUMENT, "matrix belongs to another device");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    // The linear's own output, for the routes whose reduction cannot carry
    // the epilogue; allocated up front so a captured step never allocates.
    const std::uint64_t n = m->planes.n;
    int rc = grow_buffer(ctx, &ctx->epilogue_rows, &ctx->epilogue_rows_bytes,
                         static_cast<std::uint64_t>(rows) * n * sizeof(float), "epilogue rows");
    if (rc != AIR_HIP_OK) return rc;
    float* y = static_cast<float*>(ctx->epilogue_rows);
    SplitEpilogue e{epilogue == AIR_HIP_EPILOGUE_SWIGLU ? kEpilogueSwiglu : kEpilogueResidual, out, norm_weight,
                    norm_out, eps};
    // RESIDUAL_LOAD: the workspace holds the split of norm_out afterwards.
    // Reserved first for this linear's own activations too, so the linear
    // cannot move it after the epilogue's pointers are taken.
    SplitWorkspace ws{};
    const std::uint64_t kp_out = ceil_div(n, kSplitK) * kSplitK;
    if (load) {
        const std::uint64_t kp_in = ceil_div(m->planes.k, kSplitK) * kSplitK;
        rc = ensure_workspace(ctx, std::max(split_workspace_bytes(kp_out, rows), split_workspace_bytes(kp_in, rows)));
        if (rc != AIR_HIP_OK) return rc;
        ws = carve_split_workspace(ctx->workspace, kp_out, rows);
        if (rows <= AIR_HIP_MAX_DECODE_ROWS && ctx->decode_path != 1u) {
            e.load = &ws;
            e.load_blocks = static_cast<std::uint32_t>(kp_out / 32u);
        }
    }
    // RESIDUAL_PREFILL: the prefill workspace holds norm_out's f16 operand
    // afterwards.  Reserved first for this linear too (so it cannot move after
    // the pointers are taken); carried by a prefill reduction only when that
    // operand ends before the partials it reads.
    PrefillOperandArgs pf_args{};
    const std::uint64_t pf_ldx = prefill_ldx(n);
    const std::uint64_t pf_mp = prefill_rows_padded(rows);
    const std::uint64_t pf_xh_bytes = ceil_div(pf_mp * pf_ldx * 2u, 256u) * 256u;
    const std::uint64_t pf_bytes = pf_xh_bytes + ceil_div(pf_mp * 4u, 256u) * 256u;
    const bool prefill_route = route_linear(ctx, m, rows, tactic) == Route::prefill;
    if (prefill_out && prefill_route && prefill_norm_fits(n, pf_ldx) && rows <= kMaxRows) {
        const PrefillShape shape = plan_prefill(m->planes, rows, ctx->prefill_tuning);
        rc = ensure_prefill_workspace(
            ctx, std::max(prefill_workspace_bytes(m->planes.k, rows, shape, m->planes.n), pf_bytes),
            ctx->prefill_source != nullptr);
        if (rc != AIR_HIP_OK) return rc;
        if (pf_bytes <= prefill_partials_offset(m->planes.k, rows)) {
            auto* base = static_cast<std::uint8_t*>(ctx->prefill_workspace);
            pf_args = PrefillOperandArgs{reinterpret_cast<_Float16*>(base), reinterpret_cast<float*>(base + pf_xh_bytes),
                                         static_cast<std::uint32_t>(pf_mp), pf_ldx};
            e.prefill = &pf_args;
        }
    }
    bool applied = false;
    rc = linear_rows(ctx, m, x, y, bias, rows, tactic, &e, &applied);
    if (rc != AIR_HIP_OK) return rc;
    if (prefill_out) {
        if (applied) {
            remember_prefill(ctx, norm_out, n, rows);
            return AIR_HIP_OK;
        }
        // The linear wrote y: the residual add and the norm with the operand.
        PrefillOperand op{};
        hipError_t err = hipErrorInvalidValue;
        if (prefill_norm_fits(n, pf_ldx) && rows <= kMaxRows) {
            rc = prefill_operand(ctx, n, rows, &op);
            if (rc != AIR_HIP_OK) return rc;
            err = launch_rms_norm_prefill(out, y, norm_weight, norm_out, rows, n, eps, op.xh, op.row_inv, op.mp, op.ldx,
                                          ctx->stream);
            if (err == hipSuccess) {
                remember_prefill(ctx, norm_out, n, rows);
                return AIR_HIP_OK;
            }
            if (err != hipErrorInvalidValue) return hip_fail(err, "rms_norm_vec_kernel");
        }
        err = launch_add_rms_norm(out, y, norm_weight, norm_out, rows, n, eps, ctx->stream);
        return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "linear epilogue");
    }
    if (!applied) {
        hipError_t err;
        if (epilogue == AIR_HIP_EPILOGUE_SWIGLU) {
            err = launch_silu_mul(y, out, rows, n / 2u, ctx->stream);
        } else if (norm_weight) {
            err = launch_add_rms_norm(out, y, norm_weight, norm_out, rows, n, eps, ctx->stream);
        } else {
            err = launch_add(out, y, static_cast<std::uint64_t>(rows) * n, ctx->stream);
        }
        if (err != hipSuccess) return hip_fail(err, "linear epilogue");
        if (load && (rc = air_hip_activations_load(ctx, norm_out, n, rows)) != AIR_HIP_OK) return rc;
    } else if (load && e.load) {
        ctx->loaded_k = n;
        ctx->loaded_rows = rows;
        ctx->loaded_row_scaled = true;
    } else if (load && (rc = air_hip_activations_load(ctx, norm_out, n, rows)) != AIR_HIP_OK) {
        return rc;   // a prefill reduction applied the norm without the split
    }
    if (load) ctx->loaded_source = norm_out;
    return AIR_HIP_OK;
}


// ---- the Qwen2 step around the linears ------------------------------------

int air_hip_matrix_rows(air_hip_context* ctx, const air_hip_matrix* m, const int32_t* rows, uint32_t count,
                        float* out) {
    if (!ctx || !m || !rows || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (m->owner->device != ctx->device) return fail(AIR_HIP_INVALID_ARGUMENT, "matrix belongs to another device");
    if (count == 0) return AIR_HIP_OK;
    if (count > 65535u) return fail(AIR_HIP_UNSUPPORTED, "at most 65535 rows per call");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = m->dense ? launch_dense_rows(m->dense, m->dense_storage, m->planes.k, m->planes.n, rows,
                                                        count, out, ctx->stream)
                                    : launch_matrix_rows(m->planes, rows, count, out, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "matrix_rows_kernel");
}

int air_hip_rms_norm(air_hip_context* ctx, const float* x, const float* weight, float* out, uint32_t m, uint64_t n,
                     double eps) {
    if (!ctx || !x || !weight || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (n == 0 || !(eps >= 0.0)) return fail(AIR_HIP_INVALID_ARGUMENT, "width must be non-zero and eps non-negative");
    if (m == 0) return AIR_HIP_OK;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = launch_rms_norm(x, weight, out, m, n, eps, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "rms_norm_kernel");
}

int air_hip_add_rms_norm(air_hip_context* ctx, float* x, const float* y, const float* weight, float* out, uint32_t m,
                         uint64_t n, double eps) {
    if (!ctx || !x || !y || !weight || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (n == 0 || !(eps >= 0.0)) return fail(AIR_HIP_INVALID_ARGUMENT, "width must be non-zero and eps non-negative");
    if (out == x || out == y) return fail(AIR_HIP_INVALID_ARGUMENT, "out must not alias x or y");
    if (m == 0) return AIR_HIP_OK;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = launch_add_rms_norm(x, y, weight, out, m, n, eps, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "rms_norm_vec_kernel");
}

int air_hip_rms_norm_prefill(air_hip_context* ctx, float* x, const float* y, const float* weight, float* out,
                             uint32_t m, uint64_t n, double eps) {
    if (!ctx || !x || !weight || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (n == 0 || !(eps >= 0.0)) return fail(AIR_HIP_INVALID_ARGUMENT, "width must be non-zero and eps non-negative");
    if (y && (out == x || out == y)) return fail(AIR_HIP_INVALID_ARGUMENT, "out must not alias x or y");
    if (m == 0) return AIR_HIP_OK;
    if (m > kMaxRows) return fail(AIR_HIP_UNSUPPORTED, "batch width %u exceeds %u", m, kMaxRows);
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    PrefillOperand op{};
    if (prefill_norm_fits(n, prefill_ldx(n))) {
        int rc = prefill_operand(ctx, n, m, &op);
        if (rc != AIR_HIP_OK) return rc;
        const hipError_t err = launch_rms_norm_prefill(x, y, weight, out, m, n, eps, op.xh, op.row_inv, op.mp, op.ldx,
                                                       ctx->stream);
        if (err == hipSuccess) {
            remember_prefill(ctx, out, n, m);
            return AIR_HIP_OK;
        }
        if (err != hipErrorInvalidValue) return hip_fail(err, "rms_norm_vec_kernel");
    }
    // Rows the fused kernel does not take: the plain norm (the linear then converts).
    const hipError_t err = y ? launch_add_rms_norm(x, y, weight, out, m, n, eps, ctx->stream)
                             : launch_rms_norm(x, weight, out, m, n, eps, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "rms_norm_kernel");
}

int air_hip_silu_mul_prefill(air_hip_context* ctx, const float* gate_up, float* out, uint32_t m, uint64_t ffn) {
    if (!ctx || !gate_up || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (m == 0 || ffn == 0) return AIR_HIP_OK;
    if (m > kMaxRows) return fail(AIR_HIP_UNSUPPORTED, "batch width %u exceeds %u", m, kMaxRows);
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    if (silu_prefill_fits(ffn, prefill_ldx(ffn))) {
        PrefillOperand op{};
        int rc = prefill_operand(ctx, ffn, m, &op);
        if (rc != AIR_HIP_OK) return rc;
        const hipError_t err = launch_silu_mul_prefill(gate_up, out, m, ffn, op.xh, op.row_inv, op.mp, op.ldx,
                                                       ctx->stream);
        if (err == hipSuccess) {
            remember_prefill(ctx, out, ffn, m);
            return AIR_HIP_OK;
        }
        if (err != hipErrorInvalidValue) return hip_fail(err, "silu_rows_prefill_kernel");
    }
    const hipError_t err = launch_silu_mul(gate_up, out, m, ffn, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "silu_mul_kernel");
}

int air_hip_rope(air_hip_context* ctx, float* qkv, uint64_t row_stride, uint32_t m, const int32_t* positions,
                 uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t rope_dims, const float* table,
                 uint64_t table_positions) {
    if (!ctx || !qkv || !positions || !table) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (rope_dims == 0 || rope_dims % 2u != 0 || rope_dims > head_dim || table_positions == 0) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "RoPE needs an even rope_dims <= head_dim and a table");
    }
    if (row_stride < static_cast<uint64_t>(q_heads + kv_heads) * head_dim) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "row stride is shorter than the q and k heads");
    }
    if (m == 0) return AIR_HIP_OK;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = launch_rope(qkv, row_stride, m, positions, q_heads, kv_heads, head_dim, rope_dims, table,
                                       table_positions, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "rope_kernel");
}

} // extern "C"

namespace {
int check_kv(const air_hip_kv_layout* kv) {
    if (!kv || (!kv->pool && !kv->chunks)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "KV layout and its pool (or chunk table) must not be null");
    }
    if (kv->page_tokens == 0 || kv->kv_width == 0 || kv->layers == 0 || kv->max_pages == 0 || kv->pool_pages == 0) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "KV layout has a zero dimension");
    }
    if (kv->pool_pages > static_cast<uint32_t>(INT32_MAX)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "KV pool pages must fit int32 page ids");
    }
    if (kv->chunks && (kv->chunk_shift > 30u || kv->pool_pages % (1u << kv->chunk_shift) != 0u)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "chunked KV pool: pool_pages must be a whole number of 2^chunk_shift chunks");
    }
    return AIR_HIP_OK;
}
KvLayout kv_layout_of(const air_hip_kv_layout* kv) {
    // A chunk table takes precedence: the kernels then never read `pool`.
    return KvLayout{kv->chunks ? nullptr : kv->pool, kv->page_tokens, kv->kv_width, kv->layers, kv->max_pages,
                    kv->pool_pages, kv->chunks, kv->chunks ? kv->chunk_shift : 0u};
}
int check_heads(const air_hip_kv_layout* kv, uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                uint64_t max_tokens) {
    if (q_heads == 0 || kv_heads == 0 || q_heads % kv_heads != 0 || head_dim == 0 || head_dim > 512u ||
        static_cast<uint64_t>(kv_heads) * head_dim != kv->kv_width) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "head geometry does not match the KV layout");
    }
    if (max_tokens == 0 || max_tokens > static_cast<uint64_t>(kv->max_pages) * kv->page_tokens) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "max_tokens must be in [1, max_pages * page_tokens]");
    }
    return AIR_HIP_OK;
}
// Grows the attention scratch to at least `bytes` (geometrically, so a decode
// loop whose key count grows by one per step reallocates rarely).
int ensure_attention_scratch(air_hip_context* ctx, uint64_t bytes) {
    return grow_buffer(ctx, &ctx->attention_scratch, &ctx->attention_scratch_bytes, bytes, "attention scratch");
}
static_assert(sizeof(AttentionTile) == sizeof(air_hip_attention_tile), "tile layouts agree");
} // namespace

extern "C" {

int air_hip_kv_append(air_hip_context* ctx, const air_hip_kv_layout* kv, const float* qkv, uint64_t row_stride,
                      uint64_t q_width, uint32_t m, const int32_t* positions, const int32_t* page_tables,
                      uint32_t layer) {
    if (!ctx || !qkv || !positions || !page_tables) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (int rc = check_kv(kv); rc != AIR_HIP_OK) return rc;
    if (layer >= kv->layers) return fail(AIR_HIP_INVALID_ARGUMENT, "layer %u is out of range", layer);
    if (row_stride < q_width + 2u * static_cast<uint64_t>(kv->kv_width)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "row stride is shorter than q|k|v");
    }
    if (m == 0) return AIR_HIP_OK;
    if (m > 65535u) return fail(AIR_HIP_UNSUPPORTED, "at most 65535 rows per call");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = launch_kv_append(kv_layout_of(kv), qkv, row_stride, q_width, m, positions, page_tables,
                                            layer, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "kv_append_kernel");
}

int air_hip_rope_kv_append(air_hip_context* ctx, const air_hip_kv_layout* kv, float* qkv, uint64_t row_stride,
                           uint32_t m, const int32_t* positions, const int32_t* page_tables, uint32_t layer,
                           uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim, uint32_t rope_dims,
                           const float* table, uint64_t table_positions) {
    if (!ctx || !qkv || !positions || !page_tables || !table) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    }
    forget_loaded_source(ctx);
    if (int rc = check_kv(kv); rc != AIR_HIP_OK) return rc;
    if (layer >= kv->layers) return fail(AIR_HIP_INVALID_ARGUMENT, "layer %u is out of range", layer);
    if (rope_dims == 0 || rope_dims % 2u != 0 || rope_dims > head_dim || table_positions == 0) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "RoPE needs an even rope_dims <= head_dim and a table");
    }
    if (static_cast<uint64_t>(kv_heads) * head_dim != kv->kv_width) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "kv_heads * head_dim must equal the KV width");
    }
    const uint64_t q_width = static_cast<uint64_t>(q_heads) * head_dim;
    if (row_stride < q_width + 2u * static_cast<uint64_t>(kv->kv_width)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "row stride is shorter than q|k|v");
    }
    if (m == 0) return AIR_HIP_OK;
    if (m > 65535u) return fail(AIR_HIP_UNSUPPORTED, "at most 65535 rows per call");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = launch_rope_kv_append(kv_layout_of(kv), qkv, row_stride, q_width, m, positions, page_tables,
                                                 layer, q_heads, kv_heads, head_dim, rope_dims, table,
                                                 table_positions, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "rope_kv_append_kernel");
}

int air_hip_linear_rope_kv(air_hip_context* ctx, const air_hip_matrix* m, const float* x, uint32_t rows, float* qkv,
                           const float* bias, const air_hip_kv_layout* kv, const int32_t* positions,
                           const int32_t* page_tables, uint32_t layer, uint32_t q_heads, uint32_t kv_heads,
                           uint32_t head_dim, uint32_t rope_dims, const float* table, uint64_t table_positions,
                           int tactic) {
    const LinearRange range(rows);
    if (!ctx || !m || !x || !qkv || !positions || !page_tables || !table) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    }
    if (static_cast<const void*>(x) == static_cast<const void*>(qkv)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "qkv must not alias x");
    }
    if (int rc = check_kv(kv); rc != AIR_HIP_OK) return rc;
    if (layer >= kv->layers) return fail(AIR_HIP_INVALID_ARGUMENT, "layer %u is out of range", layer);
    if (rope_dims == 0 || rope_dims % 2u != 0 || rope_dims > head_dim || table_positions == 0) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "RoPE needs an even rope_dims <= head_dim and a table");
    }
    if (static_cast<uint64_t>(kv_heads) * head_dim != kv->kv_width) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "kv_heads * head_dim must equal the KV width");
    }
    const uint64_t q_width = static_cast<uint64_t>(q_heads) * head_dim;
    if (m->planes.n != q_width + 2u * static_cast<uint64_t>(kv->kv_width)) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "the matrix's %llu outputs are not q|k|v of these heads",
                    static_cast<unsigned long long>(m->planes.n));
    }
    if (rows == 0) return fail(AIR_HIP_INVALID_ARGUMENT, "linear batch width must be non-zero");
    if (rows > 65535u) return fail(AIR_HIP_UNSUPPORTED, "at most 65535 rows per call");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const RopeKvArgs args{kv_layout_of(kv), positions, page_tables, layer, q_heads, kv_heads, head_dim, rope_dims,
                          table, table_positions};
    const SplitEpilogue e{kEpilogueRopeKv, qkv, nullptr, nullptr, 0.0, &args};
    bool applied = false;
    int rc = linear_rows(ctx, m, x, qkv, bias, rows, tactic, &e, &applied);
    if (rc != AIR_HIP_OK || applied) return rc;
    const hipError_t err = launch_rope_kv_append(args.kv, qkv, m->planes.n, q_width, rows, positions, page_tables, layer,
                                                 q_heads, kv_heads, head_dim, rope_dims, table, table_positions,
                                                 ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "rope_kv_append_kernel");
}

int air_hip_attention(air_hip_context* ctx, const air_hip_kv_layout* kv, const float* qkv, uint64_t row_stride,
                      uint32_t m, const int32_t* positions, const int32_t* page_tables, uint32_t layer,
                      uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim, uint64_t max_tokens, float* out) {
    if (!ctx || !qkv || !positions || !page_tables || !out) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    }
    forget_loaded_source(ctx);
    if (int rc = check_kv(kv); rc != AIR_HIP_OK) return rc;
    if (layer >= kv->layers) return fail(AIR_HIP_INVALID_ARGUMENT, "layer %u is out of range", layer);
    if (int rc = check_heads(kv, q_heads, kv_heads, head_dim, max_tokens); rc != AIR_HIP_OK) return rc;
    if (m == 0) return AIR_HIP_OK;
    const uint64_t blocks = static_cast<uint64_t>(m) * q_heads;
    if (blocks > 0x7fffffffu) return fail(AIR_HIP_UNSUPPORTED, "too many (row, head) pairs");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    if (int rc = ensure_attention_scratch(ctx, blocks * max_tokens * sizeof(double)); rc != AIR_HIP_OK) return rc;
    const hipError_t err = launch_attention(kv_layout_of(kv), qkv, row_stride, m, positions, page_tables, layer,
                                            q_heads, kv_heads, head_dim, static_cast<double*>(ctx->attention_scratch),
                                            max_tokens, out, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "attention_kernel");
}

int air_hip_attention_make_tiles(const uint32_t* run_rows, uint32_t runs, uint32_t q_heads, uint32_t kv_heads,
                                 air_hip_attention_tile* tiles, uint32_t capacity, uint32_t* count) {
    if (!run_rows || !count) return fail(AIR_HIP_INVALID_ARGUMENT, "run_rows and count must not be null");
    if (q_heads == 0 || kv_heads == 0 || q_heads % kv_heads != 0) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "q heads must be a non-zero multiple of the KV heads");
    }
    for (uint32_t i = 0; i < runs; ++i) {
        if (run_rows[i] == 0) return fail(AIR_HIP_INVALID_ARGUMENT, "run %u has no rows", i);
    }
    *count = make_attention_tiles(run_rows, runs, q_heads, kv_heads, reinterpret_cast<AttentionTile*>(tiles),
                                  tiles ? capacity : 0u);
    if (tiles && *count > capacity) return fail(AIR_HIP_INVALID_ARGUMENT, "%u tiles exceed capacity %u", *count, capacity);
    return AIR_HIP_OK;
}

int air_hip_attention_online(air_hip_context* ctx, const air_hip_kv_layout* kv, const float* qkv, uint64_t row_stride,
                             uint32_t m, const int32_t* positions, const int32_t* page_tables, uint32_t layer,
                             uint32_t q_heads, uint32_t kv_heads, uint32_t head_dim,
                             const air_hip_attention_tile* tiles, uint32_t tile_count, uint64_t max_tokens,
                             float* out) {
    if (!ctx || !qkv || !positions || !page_tables || !tiles || !out) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    }
    forget_loaded_source(ctx);
    if (int rc = check_kv(kv); rc != AIR_HIP_OK) return rc;
    if (layer >= kv->layers) return fail(AIR_HIP_INVALID_ARGUMENT, "layer %u is out of range", layer);
    if (int rc = check_heads(kv, q_heads, kv_heads, head_dim, max_tokens); rc != AIR_HIP_OK) return rc;
    if (head_dim != 64u && head_dim != 128u) {
        return fail(AIR_HIP_UNSUPPORTED, "online attention supports head widths 64 and 128, not %u", head_dim);
    }
    const uint64_t qkv_width = static_cast<uint64_t>(q_heads) * head_dim + 2u * static_cast<uint64_t>(kv->kv_width);
    if (row_stride < qkv_width || row_stride % 4u != 0 || reinterpret_cast<std::uintptr_t>(qkv) % 16u != 0 ||
        reinterpret_cast<std::uintptr_t>(out) % 16u != 0 || reinterpret_cast<std::uintptr_t>(kv->pool) % 16u != 0) {
        return fail(AIR_HIP_INVALID_ARGUMENT, "q|k|v rows, output and pool must be 16-byte aligned, stride >= q|k|v");
    }
    if (m == 0 || tile_count == 0) return AIR_HIP_OK;
    if (tile_count > 0x7fffffffu) return fail(AIR_HIP_UNSUPPORTED, "too many tiles");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const uint32_t splits = attention_splits(tile_count, max_tokens, m);
    if (int rc = ensure_attention_scratch(ctx, attention_partials_bytes(tile_count, splits, head_dim));
        rc != AIR_HIP_OK) {
        return rc;
    }
    const hipError_t err = launch_attention_tiles(kv_layout_of(kv), qkv, row_stride, m, positions, page_tables, layer,
                                                  q_heads, kv_heads, head_dim,
                                                  reinterpret_cast<const AttentionTile*>(tiles), tile_count, splits,
                                                  static_cast<float*>(ctx->attention_scratch), out, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "attention_mfma_kernel");
}

int air_hip_silu_mul(air_hip_context* ctx, const float* gate_up, float* out, uint32_t m, uint64_t ffn) {
    if (!ctx || !gate_up || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (m == 0 || ffn == 0) return AIR_HIP_OK;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = launch_silu_mul(gate_up, out, m, ffn, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "silu_mul_kernel");
}

int air_hip_add(air_hip_context* ctx, float* x, const float* y, uint64_t count) {
    if (!ctx || !x || !y) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (count == 0) return AIR_HIP_OK;
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    const hipError_t err = launch_add(x, y, count, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "add_kernel");
}

int air_hip_argmax(air_hip_context* ctx, const float* logits, uint32_t m, uint64_t n, int32_t* out) {
    if (!ctx || !logits || !out) return fail(AIR_HIP_INVALID_ARGUMENT, "arguments must not be null");
    forget_loaded_source(ctx);
    if (n == 0 || n > 0x7fffffffu) return fail(AIR_HIP_INVALID_ARGUMENT, "row width must be in [1, 2^31)");
    if (m == 0) return AIR_HIP_OK;
    if (m > 65535u) return fail(AIR_HIP_UNSUPPORTED, "at most 65535 rows per call");
    DeviceScope scope(ctx->device);
    if (scope.status() != hipSuccess) return hip_fail(scope.status(), "hipSetDevice");
    if (int rc = grow_buffer(ctx, &ctx->argmax_partials, &ctx->argmax_partials_bytes, argmax_scratch_bytes(m, n),
                             "argmax partials");
        rc != AIR_HIP_OK) {
        return rc;
    }
    const hipError_t err = launch_argmax(logits, m, n, out, ctx->argmax_partials, ctx->stream);
    return err == hipSuccess ? AIR_HIP_OK : hip_fail(err, "argmax_slice_kernel");
}

} // extern "C"

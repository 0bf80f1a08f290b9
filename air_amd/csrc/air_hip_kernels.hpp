// air_hip_kernels.hpp -- host-side launchers of the HIP kernels (internal).
#pragma once

#include <hip/hip_runtime.h>
#include <cstdint>

namespace air_hip {

// Resident planes of one matrix in the wavefront tile layout.
struct TilePlanes {
    int type{0};
    std::uint64_t k{0}, n{0};
    std::uint32_t nt{0};   // 16-row tiles
    std::uint32_t kt{0};   // k tiles
    std::uint64_t kp{0};   // padded k = kt * tile_k
    void* codes{nullptr};
    void* scales{nullptr};
};

// Canonical GGUF bytes (device) -> tile planes.
hipError_t launch_repack(const TilePlanes& planes, const std::uint8_t* canonical, hipStream_t stream);
// Tile planes -> f32 [n][k] (device), bit-exact decode.
hipError_t launch_dequantize_tiles(const TilePlanes& planes, float* out, hipStream_t stream);
// Canonical GGUF bytes (device) -> f32, bit-exact decode.
hipError_t launch_dequantize_canonical(int type, const std::uint8_t* canonical,
                                       std::uint64_t elements, float* out, hipStream_t stream);

// Workspace of the split activations for `m` rows of width kp (padded).
struct SplitWorkspace {
    void* xs{nullptr};       // [kp/32][mp/16][2][64][8] f16  (hi, lo)
    float* block_sums{nullptr}; // [kp/32][mp] f32  (sum of scaled x per 32-block)
    float* inv_scale{nullptr};  // [mp] f32
};
std::uint64_t split_workspace_bytes(std::uint64_t kp, std::uint32_t m);
SplitWorkspace carve_split_workspace(void* base, std::uint64_t kp, std::uint32_t m);

// Activation split: x [m][k] f32 -> per-row power-of-two scaled f16 hi/lo
// tiles, scaled 32-block sums and inverse scales.  Rows m..mp-1 are zeroed.
hipError_t launch_split_activations(const float* x, std::uint32_t m, std::uint64_t k,
                                    std::uint64_t kp, const SplitWorkspace& ws, hipStream_t stream);

// Decode linear over the split activations: y[m][n] (+ bias[n]).
hipError_t launch_decode_linear(const TilePlanes& planes, const SplitWorkspace& ws,
                                const float* bias, float* y, std::uint32_t m, hipStream_t stream);

} // namespace air_hip

// stream.hip -- a read-only streaming pass over device bytes.
//
// The floor any M = 1 linear launch is measured against: reading a buffer of
// the matrix's size once, in one launch, with nothing else to do.  Each
// workgroup reads one contiguous chunk, its eight waves taking 8 KiB steps
// (one 16-byte non-temporal load per lane per KiB, the decode GEMV's access
// pattern); the data are folded into an XOR checksum so no load can be
// dropped: the workgroup's waves meet in LDS and the workgroup stores its
// chunk's XOR in its own word of the sink.  The checksum is the XOR of the
// sink's words (XOR is associative and commutative: it does not depend on
// the order of the reads).  One plain store per workgroup: an atomic XOR per
// workgroup into a shared word cost 2 us of gate|up's 22 us (measured).
#include "air_hip_device.hpp"
#include "air_hip_kernels.hpp"

namespace air_hip {
namespace {


// kStreamWaves waves per workgroup, kStreamStep KiB per wave per step.
template <unsigned kStreamWaves, unsigned kStreamStep>
__global__ __launch_bounds__(64 * kStreamWaves) void stream_read_kernel(const u32x4* __restrict__ data,
                                                                       std::uint64_t vecs, std::uint64_t chunk_vecs,
                                                                       unsigned* __restrict__ sink) {
    const unsigned lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const std::uint64_t begin = static_cast<std::uint64_t>(blockIdx.x) * chunk_vecs;
    const std::uint64_t end = begin + chunk_vecs < vecs ? begin + chunk_vecs : vecs;
    unsigned acc = 0;
    for (std::uint64_t base = begin + static_cast<std::uint64_t>(wave) * 64u * kStreamStep; base < end;
         base += 64u * kStreamStep * kStreamWaves) {
        u32x4 v[kStreamStep];
#pragma unroll
        for (unsigned t = 0; t < kStreamStep; ++t) {
            const std::uint64_t i = base + 64u * t + lane;
            v[t] = i < end ? __builtin_nontemporal_load(data + i) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (unsigned t = 0; t < kStreamStep; ++t) acc ^= v[t].x ^ v[t].y ^ v[t].z ^ v[t].w;
    }
    for (int off = 32; off > 0; off >>= 1) acc ^= static_cast<unsigned>(__shfl_xor(static_cast<int>(acc), off));
    __shared__ unsigned waves_acc[kStreamWaves];
    if (lane == 0u) waves_acc[wave] = acc;
    __syncthreads();
    if (threadIdx.x == 0u) {
        unsigned total = 0;
#pragma unroll
        for (unsigned w = 0; w < kStreamWaves; ++w) total ^= waves_acc[w];
        sink[blockIdx.x] = total;
    }
}

} // namespace

hipError_t launch_stream_read(const void* data, std::uint64_t bytes, unsigned* sink, std::uint64_t sink_words,
                              hipStream_t stream) {
    if (bytes % 16u != 0u) return hipErrorInvalidValue;
    const std::uint64_t vecs = bytes / 16u;
    if (vecs == 0u) return hipSuccess;
    // Large buffers: chunks of 56 KiB (a 7B gate|up row tile) read by eight
    // waves in 8 KiB steps, halved while fewer than 512 workgroups would
    // share the buffer.  Below 32 MiB: 4 KiB chunks, one 1 KiB load per wave
    // of four (thousands of small workgroups ramp up fastest: measured with a
    // grid-stride reader of that shape, q|k|v-sized 17.5 MB 4.1 us against
    // 4.8 in 56 KiB chunks, o-sized 13.6 MB 3.6 against 4.1).  Either way
    // doubled while the sink holds fewer words than chunks.
    const bool small = bytes < (32ull << 20);
    std::uint64_t chunk = small ? 4u * 64u : 56u * 64u;   // 16-byte vectors
    while (!small && chunk > 64u * 8u && ceil_div(vecs, chunk) < 512u) chunk /= 2u;
    while (ceil_div(vecs, chunk) > sink_words) chunk *= 2u;
    const std::uint64_t groups = ceil_div(vecs, chunk);
    if (groups > 0x7fffffffu) return hipErrorInvalidValue;
    if (small) {
        hipLaunchKernelGGL((stream_read_kernel<4, 1>), dim3(static_cast<unsigned>(groups)), dim3(256), 0, stream,
                           static_cast<const u32x4*>(data), vecs, chunk, sink);
    } else {
        hipLaunchKernelGGL((stream_read_kernel<8, 8>), dim3(static_cast<unsigned>(groups)), dim3(512), 0, stream,
                           static_cast<const u32x4*>(data), vecs, chunk, sink);
    }
    return hipGetLastError();
}

} // namespace air_hip

// profile.hpp -- named ranges for rocprofv3 --marker-trace.
//
// The reference wraps every executor stage in an NVTX range
// (ScopedProfileRange, src/cuda/cuda_backend.cu:32-48: air.decode.step,
// air.decode.layer, air.cuda.matmul, ...); the HIP executor marks the same
// stages with ROCTX ranges of the same names (air.hip.* for the device
// operations), so a kernel trace can be read stage by stage.  Without a
// profiler attached a range costs one library call on each side.
#pragma once

#include <rocprofiler-sdk-roctx/roctx.h>

namespace air {

class ScopedRange final {
public:
    explicit ScopedRange(const char* name) noexcept { roctxRangePushA(name); }
    ~ScopedRange() { roctxRangePop(); }
    ScopedRange(const ScopedRange&) = delete;
    ScopedRange& operator=(const ScopedRange&) = delete;
};

} // namespace air

// SwiGLU launch helpers (kernels in swiglu.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace esep {

hipError_t launch_swiglu_fwd(const void* g, const void* u, void* h, int64_t n, int dt,
                             hipStream_t s, bool* supported);
hipError_t launch_swiglu_bwd(const void* dh, const void* g, const void* u, void* dg, void* du,
                             int64_t n, int dt, hipStream_t s, bool* supported);

}  // namespace esep

// LoRA-dropout launch helpers (kernels in dropout.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace esep {

hipError_t launch_dropout_fwd(const void* x, const int64_t* key, void* xd, int64_t n, float p,
                              int dt, hipStream_t s, bool* supported);
hipError_t launch_dropout_bwd(const void* x, const void* g, const int64_t* key, void* xd, void* dx,
                              int64_t n, float p, int accumulate, int dt, hipStream_t s,
                              bool* supported);

}  // namespace esep

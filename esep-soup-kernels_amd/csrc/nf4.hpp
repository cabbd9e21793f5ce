// NF4 dequantization launch helper (kernel in nf4.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace esep {

struct Nf4Args {
  const void* packed;      // uint8 [n_blocks * 32]
  const uint8_t* absmax;   // uint8 [n_blocks]
  const float* absmax2;    // fp32 [ceil(n_blocks / 256)]
  const float* code2;      // fp32 [256]
  const float* offset;     // fp32 scalar (device)
  const float* nf4;        // fp32 [16]
  void* out;               // [n_blocks * 64] of the output dtype
  int64_t n_blocks;
};

hipError_t launch_nf4_dequant(const Nf4Args& a, int out_dt, hipStream_t s, bool* supported);

constexpr int kNf4MultiMax = 8;

// Up to kNf4MultiMax weights decoded by one launch; weight i covers the global 8-packed-byte
// units [q0[i], q0[i + 1]) (4 per 64-element scale block).
struct Nf4Multi {
  Nf4Args w[kNf4MultiMax];
  int64_t q0[kNf4MultiMax + 1];
  int n;
};

hipError_t launch_nf4_dequant_multi(const Nf4Multi& m, int out_dt, hipStream_t s, bool* supported);

}  // namespace esep

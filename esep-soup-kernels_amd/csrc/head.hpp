// LM-head row kernel launch helper (kernel in head.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace esep {

struct HeadArgs {
  void* z;                // [rows, ld] logits chunk (fp16 / bf16); rows with g get overwritten
  const int64_t* target;  // [rows] vocabulary id; outside [0, V) = no target
  const float* cew;       // [rows] CE weight: pass 2 runs on rows where it is != 0
  float* lse;             // [rows] log-sum-exp
  float* tlogit;          // [rows] target logit (0 without a target)
  float* ent;             // [rows] entropy of softmax(z)
  int32_t* amax;          // [rows] first index of the row maximum
  int64_t rows, ld, V;
  float g_scale;
  int write_g;
};

// vec: z is 16-byte aligned and ld and V are multiples of 8 (whole 16-byte chunks).
hipError_t launch_head_row(const HeadArgs& a, int dt, bool vec, hipStream_t s, bool* supported);

}  // namespace esep

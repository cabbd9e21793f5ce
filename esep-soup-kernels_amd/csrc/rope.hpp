// Argument block and launcher of the rotary-embedding kernel (rope.hip).
#pragma once

#include "common.hpp"

namespace esep {

struct RopeArgs {
  const void* q;
  const void* qd;
  const void* k;
  void* qo;
  void* ko;
  int64_t q_s[3], qd_s[3], k_s[3], qo_s[3], ko_s[3];  // (b, s, h) strides in elements
  int64_t B, S;
  int HQ, HK;
  const void* pos;
  int pos_i64;
  int64_t pos_s[2];
  const int32_t* cu;
  int n_seq;
  const float* inv_freq;
  float sign;
  int vec;
};

hipError_t launch_rope(const RopeArgs& a, int dt, int half, hipStream_t s, bool* supported);

}  // namespace esep

// Rotary embedding (forward and backward) on q and k for gfx950 (MI355X).
//
// Mapping. One wavefront per token. The token's D/2 angles are computed once: lane j takes
// angle j (and j + 64 for D = 256), calls the accurate sincosf (full range reduction, so
// positions in the tens of thousands stay exact to fp32 rounding) and parks cos / sin in a
// per-wave LDS slot. Each lane then owns 8 consecutive frequencies of a head half, reads their
// cos / sin back as two 16-byte LDS loads, and reuses them for every head of the token:
// HALF/8 lanes cover one head (both halves: x1 = [8c, 8c+8), x2 = [HALF+8c, HALF+8c+8)), so a
// wavefront instruction moves 64/(HALF/8) heads and every global access is 16 bytes.
// Up to four passes of heads are loaded before any is rotated and stored, so a lane keeps
// eight 16-byte loads in flight.
//
// Numerics follow the reference's _rope_kernel (solution/body/norm_rope.py:330-369):
// angle = float(pos) * inv_freq[j] as one fp32 multiply; q + q_delta is formed in the storage
// dtype (one rounding) before the rotation; the rotation runs in fp32 with one rounding at the
// store; backward is the same kernel with the sine negated.
#include "rope.hpp"

namespace esep {

constexpr int kRopeWaves = 4;
constexpr int kRopePasses = 4;

template <bool VEC, typename T>
__device__ __forceinline__ void ld_half(const T* p, float (&v)[8]) {
  if constexpr (VEC) {
    Chunk<T>::load(p, v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = Elt<T>::to_f(p[e]);
  }
}
template <bool VEC, typename T>
__device__ __forceinline__ void st_half(T* p, const float (&v)[8]) {
  if constexpr (VEC) {
    Chunk<T>::store(p, v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = Elt<T>::from_f(v[e]);
  }
}

template <bool VEC, typename T, int HALF>
__device__ __forceinline__ void rope_token(const RopeArgs& a, int64_t b, int64_t s, int lane,
                                           const float (&cv)[8], const float (&sv)[8]) {
  constexpr int LPH = HALF / 8;
  constexpr int HPP = kWave / LPH;
  const int c = lane % LPH;
  const int hs = lane / LPH;
  const int nh = a.HQ + a.HK;
  const T* __restrict__ q = static_cast<const T*>(a.q);
  const T* __restrict__ qd = static_cast<const T*>(a.qd);
  const T* __restrict__ k = static_cast<const T*>(a.k);
  T* __restrict__ qo = static_cast<T*>(a.qo);
  T* __restrict__ ko = static_cast<T*>(a.ko);

  for (int h0 = 0; h0 < nh; h0 += kRopePasses * HPP) {
    float x1[kRopePasses][8], x2[kRopePasses][8];
#pragma unroll
    for (int i = 0; i < kRopePasses; ++i) {
      const int h = h0 + i * HPP + hs;
      if (h < nh) {
        const T* src = h < a.HQ
            ? q + b * a.q_s[0] + s * a.q_s[1] + (int64_t)h * a.q_s[2]
            : k + b * a.k_s[0] + s * a.k_s[1] + (int64_t)(h - a.HQ) * a.k_s[2];
        ld_half<VEC>(src + 8 * c, x1[i]);
        ld_half<VEC>(src + HALF + 8 * c, x2[i]);
      }
    }
    if (qd != nullptr) {
#pragma unroll
      for (int i = 0; i < kRopePasses; ++i) {
        const int h = h0 + i * HPP + hs;
        if (h < a.HQ) {
          const T* src = qd + b * a.qd_s[0] + s * a.qd_s[1] + (int64_t)h * a.qd_s[2];
          float d1[8], d2[8];
          ld_half<VEC>(src + 8 * c, d1);
          ld_half<VEC>(src + HALF + 8 * c, d2);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            x1[i][e] = Elt<T>::round(x1[i][e] + d1[e]);
            x2[i][e] = Elt<T>::round(x2[i][e] + d2[e]);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < kRopePasses; ++i) {
      const int h = h0 + i * HPP + hs;
      if (h < nh) {
        float o1[8], o2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o1[e] = x1[i][e] * cv[e] - x2[i][e] * sv[e];
          o2[e] = x2[i][e] * cv[e] + x1[i][e] * sv[e];
        }
        T* dst = h < a.HQ
            ? qo + b * a.qo_s[0] + s * a.qo_s[1] + (int64_t)h * a.qo_s[2]
            : ko + b * a.ko_s[0] + s * a.ko_s[1] + (int64_t)(h - a.HQ) * a.ko_s[2];
        st_half<VEC>(dst + 8 * c, o1);
        st_half<VEC>(dst + HALF + 8 * c, o2);
      }
    }
  }
}

template <typename T, int HALF>
__global__ __launch_bounds__(kRopeWaves * kWave) void k_rope(const RopeArgs a) {
  __shared__ float cs[kRopeWaves][2][HALF];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t t = (int64_t)blockIdx.x * kRopeWaves + wave;
  if (t >= a.B * a.S) return;  // whole wavefront leaves; nothing below waits on other waves
  const int64_t b = t / a.S;
  const int64_t s = t - b * a.S;

  int64_t pos;
  if (a.pos != nullptr) {
    const int64_t off = b * a.pos_s[0] + s * a.pos_s[1];
    pos = a.pos_i64 ? static_cast<const int64_t*>(a.pos)[off]
                    : (int64_t) static_cast<const int32_t*>(a.pos)[off];
  } else if (a.cu != nullptr) {
    // Sequence of token s: the number of starts cu[1..n_seq-1] that are <= s (cu is
    // non-decreasing; empty sequences are skipped over), counted 64 starts at a time.
    int idx = 0;
    for (int base = 1; base < a.n_seq; base += kWave) {
      const int j = base + lane;
      const bool le = j < a.n_seq && (int64_t)a.cu[j] <= s;
      idx += __popcll(__ballot(le));
      if (base + kWave >= a.n_seq || (int64_t)a.cu[base + kWave - 1] > s) break;
    }
    pos = s - (int64_t)a.cu[idx];
  } else {
    pos = s;
  }

  const float p = (float)pos;
  for (int j = lane; j < HALF; j += kWave) {
    const float ang = p * a.inv_freq[j];
    float sn, cn;
    sincosf(ang, &sn, &cn);
    cs[wave][0][j] = cn;
    cs[wave][1][j] = sn * a.sign;
  }
  wave_lds_sync();
  constexpr int LPH = HALF / 8;
  const int c = lane % LPH;
  float cv[8], sv[8];
  {
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(&cs[wave][0][8 * c]);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(&cs[wave][0][8 * c + 4]);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(&cs[wave][1][8 * c]);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(&cs[wave][1][8 * c + 4]);
    cv[0] = c0.x; cv[1] = c0.y; cv[2] = c0.z; cv[3] = c0.w;
    cv[4] = c1.x; cv[5] = c1.y; cv[6] = c1.z; cv[7] = c1.w;
    sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w;
    sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
  }
  if (a.vec)
    rope_token<true, T, HALF>(a, b, s, lane, cv, sv);
  else
    rope_token<false, T, HALF>(a, b, s, lane, cv, sv);
}

template <typename T>
static hipError_t rope_half(const RopeArgs& a, int half, dim3 g, dim3 b, hipStream_t s, bool* sup) {
  *sup = true;
  switch (half) {
    case 32: hipLaunchKernelGGL((k_rope<T, 32>), g, b, 0, s, a); break;
    case 64: hipLaunchKernelGGL((k_rope<T, 64>), g, b, 0, s, a); break;
    case 128: hipLaunchKernelGGL((k_rope<T, 128>), g, b, 0, s, a); break;
    default: *sup = false; return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rope(const RopeArgs& a, int dt, int half, hipStream_t s, bool* sup) {
  const int64_t tokens = a.B * a.S;
  const dim3 grid((unsigned)((tokens + kRopeWaves - 1) / kRopeWaves)), block(kRopeWaves * kWave);
  if (dt == 0) return rope_half<float>(a, half, grid, block, s, sup);
  if (dt == 1) return rope_half<_Float16>(a, half, grid, block, s, sup);
  if (dt == 2) return rope_half<__bf16>(a, half, grid, block, s, sup);
  *sup = false;
  return hipErrorInvalidValue;
}

}  // namespace esep

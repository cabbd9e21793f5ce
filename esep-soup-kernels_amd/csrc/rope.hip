// Rotary embedding (forward and backward) on q and k for gfx950 (MI355X).
//
// Mapping. One wavefront per token (two on the vector path, processed together). The token's D/2 angles are computed once: lane j takes
// angle j (and j + 64 for D = 256), calls the accurate sincosf (full range reduction, so
// positions in the tens of thousands stay exact to fp32 rounding) and parks cos / sin in a
// per-wave LDS slot. Each lane then owns 8 consecutive frequencies of a head half, reads their
// cos / sin back as two 16-byte LDS loads, and reuses them for every head of the token:
// HALF/8 lanes cover one head (both halves: x1 = [8c, 8c+8), x2 = [HALF+8c, HALF+8c+8)), so a
// wavefront instruction moves 64/(HALF/8) heads and every global access is 16 bytes.
// Up to four passes of heads are loaded (raw, still packed, non-temporal) before any is
// rotated and stored, so a lane keeps eight 16-byte loads in flight in few registers.
//
// Numerics follow the reference's _rope_kernel (solution/body/norm_rope.py:330-369):
// angle = float(pos) * inv_freq[j] as one fp32 multiply; q + q_delta is formed in the storage
// dtype (one rounding) before the rotation; the rotation runs in fp32 with one rounding at the
// store; backward is the same kernel with the sine negated.
#include "rope.hpp"

namespace esep {

// Wavefronts per block: 4 with two tokens per wavefront, 2 with one. Measured per launch (us,
// fwd / bwd): config 4 (two tokens) 2 waves 10.62 / 10.66, 4 waves 10.57 / 10.56, 8 waves
// 10.59 / 10.64; config 5 (one token) 2 waves 184.4 / 182.6, 4 waves 189.2 / 187.9, 8 waves
// 188.3 / 187.4.
constexpr int rope_waves(int tpw) { return tpw == 2 ? 4 : 2; }
constexpr int kRopePasses = 4;

// One head half (8 elements) of one lane: VEC as a single raw 16-byte (two for fp32)
// non-temporal load, kept packed until it is rotated; !VEC element by element.
template <bool VEC, typename T>
__device__ __forceinline__ Raw<T> ld_raw(const T* p) {
  Raw<T> r;
  if constexpr (VEC) {
    r.a = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    if constexpr (sizeof(T) == 4) r.b = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + 1);
  } else {
    typedef T v8 __attribute__((ext_vector_type(8)));
    v8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = p[e];
    if constexpr (sizeof(T) == 4) {
      r.a = u32x4{__float_as_uint(h[0]), __float_as_uint(h[1]), __float_as_uint(h[2]), __float_as_uint(h[3])};
      r.b = u32x4{__float_as_uint(h[4]), __float_as_uint(h[5]), __float_as_uint(h[6]), __float_as_uint(h[7])};
    } else {
      r.a = __builtin_bit_cast(u32x4, h);
    }
  }
  return r;
}

template <bool VEC, typename T>
__device__ __forceinline__ void st_half(T* p, const float (&v)[8]) {
  typedef T v8 __attribute__((ext_vector_type(8)));
  v8 h;
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = Elt<T>::from_f(v[e]);
  if constexpr (VEC) {
    if constexpr (sizeof(T) == 4) {
      __builtin_nontemporal_store(u32x4{__float_as_uint(h[0]), __float_as_uint(h[1]),
                                        __float_as_uint(h[2]), __float_as_uint(h[3])},
                                  reinterpret_cast<u32x4*>(p));
      __builtin_nontemporal_store(u32x4{__float_as_uint(h[4]), __float_as_uint(h[5]),
                                        __float_as_uint(h[6]), __float_as_uint(h[7])},
                                  reinterpret_cast<u32x4*>(p) + 1);
    } else {
      __builtin_nontemporal_store(__builtin_bit_cast(u32x4, h), reinterpret_cast<u32x4*>(p));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) p[e] = h[e];
  }
}

// Position of token (b, s): explicit, from cu_seqlens, or s itself.
__device__ __forceinline__ int64_t token_pos(const RopeArgs& a, int64_t b, int64_t s, int lane) {
  if (a.pos != nullptr) {
    const int64_t off = b * a.pos_s[0] + s * a.pos_s[1];
    return a.pos_i64 ? static_cast<const int64_t*>(a.pos)[off]
                     : (int64_t) static_cast<const int32_t*>(a.pos)[off];
  }
  if (a.cu != nullptr) {
    // Sequence of token s: the number of starts cu[1..n_seq-1] that are <= s (cu is
    // non-decreasing; empty sequences are skipped over), counted 64 starts at a time.
    int idx = 0;
    for (int base = 1; base < a.n_seq; base += kWave) {
      const int j = base + lane;
      const bool le = j < a.n_seq && (int64_t)a.cu[j] <= s;
      idx += __popcll(__ballot(le));
      if (base + kWave >= a.n_seq || (int64_t)a.cu[base + kWave - 1] > s) break;
    }
    return s - (int64_t)a.cu[idx];
  }
  return s;
}

// The raw (still packed) halves of one group of heads of the TPW tokens of a wavefront: heads
// go in groups of PG passes per token (TPW * PG = 4 passes in total).
template <typename T, int TPW, int PG>
struct RopeGroup {
  Raw<T> x1[TPW][PG], x2[TPW][PG], d1[TPW][PG], d2[TPW][PG];
};

// Issue every load of the head group starting at head h0 (all tokens, all passes) before any
// is used.
template <bool VEC, bool QD, typename T, int HALF, int TPW>
__device__ __forceinline__ void rope_load(const RopeArgs& a, const int64_t (&bb)[TPW],
                                          const int64_t (&ss)[TPW], const bool (&live)[TPW],
                                          int lane, int h0,
                                          RopeGroup<T, TPW, kRopePasses / TPW>& g) {
  constexpr int LPH = HALF / 8;
  constexpr int HPP = kWave / LPH;
  constexpr int PG = kRopePasses / TPW;
  const int c = lane % LPH;
  const int hs = lane / LPH;
  const int nh = a.HQ + a.HK;
  const T* __restrict__ q = static_cast<const T*>(a.q);
  const T* __restrict__ qd = static_cast<const T*>(a.qd);
  const T* __restrict__ k = static_cast<const T*>(a.k);
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
#pragma unroll
    for (int i = 0; i < PG; ++i) {
      const int h = h0 + i * HPP + hs;
      if (live[t] && h < nh) {
        const T* src = h < a.HQ
            ? q + bb[t] * a.q_s[0] + ss[t] * a.q_s[1] + (int64_t)h * a.q_s[2]
            : k + bb[t] * a.k_s[0] + ss[t] * a.k_s[1] + (int64_t)(h - a.HQ) * a.k_s[2];
        g.x1[t][i] = ld_raw<VEC>(src + 8 * c);
        g.x2[t][i] = ld_raw<VEC>(src + HALF + 8 * c);
        if (QD && h < a.HQ) {
          const T* dsrc = qd + bb[t] * a.qd_s[0] + ss[t] * a.qd_s[1] + (int64_t)h * a.qd_s[2];
          g.d1[t][i] = ld_raw<VEC>(dsrc + 8 * c);
          g.d2[t][i] = ld_raw<VEC>(dsrc + HALF + 8 * c);
        }
      }
    }
  }
}

// Rotate and store the head group starting at h0.
template <bool VEC, bool QD, typename T, int HALF, int TPW>
__device__ __forceinline__ void rope_store(const RopeArgs& a, const int64_t (&bb)[TPW],
                                           const int64_t (&ss)[TPW], const bool (&live)[TPW],
                                           int lane, int h0,
                                           const RopeGroup<T, TPW, kRopePasses / TPW>& g,
                                           const float (&cv)[TPW][8], const float (&sv)[TPW][8]) {
  constexpr int LPH = HALF / 8;
  constexpr int HPP = kWave / LPH;
  constexpr int PG = kRopePasses / TPW;
  const int c = lane % LPH;
  const int hs = lane / LPH;
  const int nh = a.HQ + a.HK;
  T* __restrict__ qo = static_cast<T*>(a.qo);
  T* __restrict__ ko = static_cast<T*>(a.ko);
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
#pragma unroll
    for (int i = 0; i < PG; ++i) {
      const int h = h0 + i * HPP + hs;
      if (live[t] && h < nh) {
        float u1[8], u2[8];
        Buf<T>::unpack(g.x1[t][i], u1);
        Buf<T>::unpack(g.x2[t][i], u2);
        if (QD && h < a.HQ) {
          // q + q_delta in the storage dtype (one rounding), as the unfused model adds them
          float e1[8], e2[8];
          Buf<T>::unpack(g.d1[t][i], e1);
          Buf<T>::unpack(g.d2[t][i], e2);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            u1[e] = Elt<T>::round(u1[e] + e1[e]);
            u2[e] = Elt<T>::round(u2[e] + e2[e]);
          }
        }
        float o1[8], o2[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          o1[e] = u1[e] * cv[t][e] - u2[e] * sv[t][e];
          o2[e] = u2[e] * cv[t][e] + u1[e] * sv[t][e];
        }
        T* dst = h < a.HQ
            ? qo + bb[t] * a.qo_s[0] + ss[t] * a.qo_s[1] + (int64_t)h * a.qo_s[2]
            : ko + bb[t] * a.ko_s[0] + ss[t] * a.ko_s[1] + (int64_t)(h - a.HQ) * a.ko_s[2];
        st_half<VEC>(dst + 8 * c, o1);
        st_half<VEC>(dst + HALF + 8 * c, o2);
      }
    }
  }
}

template <typename T, int HALF, bool VEC, bool QD, int TPW>
__global__ __launch_bounds__(rope_waves(TPW) * kWave) void k_rope(const RopeArgs a) {
  constexpr int NW = rope_waves(TPW);
  __shared__ float cs[NW][TPW][2][HALF];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t tokens = a.B * a.S;
  const int64_t t0 = ((int64_t)blockIdx.x * NW + wave) * TPW;
  if (t0 >= tokens) return;  // whole wavefront leaves; nothing below waits on other waves
  int64_t bb[TPW], ss[TPW];
  bool live[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    live[t] = t0 + t < tokens;
    const int64_t tt = live[t] ? t0 + t : t0;
    bb[t] = tt / a.S;
    ss[t] = tt - bb[t] * a.S;
  }
  // With two tokens per wavefront (few heads: the launch is short and latency-bound) the first
  // head group's loads go out before the angles are worked out (an inv_freq and position read,
  // sincosf, the LDS round), which then overlap the data's memory round trip: config 4
  // 11.6 -> 10.6 us per launch. With one token per wavefront (many heads, a long launch at the
  // bandwidth limit) the loads follow the angles: issued first they made config 5 5% slower.
  constexpr int PG = kRopePasses / TPW;
  constexpr int HPP = kWave / (HALF / 8);
  constexpr bool kLoadFirst = TPW == 2;
  RopeGroup<T, TPW, PG> g;
  if constexpr (kLoadFirst) rope_load<VEC, QD, T, HALF, TPW>(a, bb, ss, live, lane, 0, g);
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const float p = (float)token_pos(a, bb[t], ss[t], lane);
    for (int j = lane; j < HALF; j += kWave) {
      const float ang = p * a.inv_freq[j];
      float sn, cn;
      sincosf(ang, &sn, &cn);
      cs[wave][t][0][j] = cn;
      cs[wave][t][1][j] = sn * a.sign;
    }
  }
  wave_lds_sync();
  constexpr int LPH = HALF / 8;
  const int c = lane % LPH;
  float cv[TPW][8], sv[TPW][8];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(&cs[wave][t][0][8 * c]);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(&cs[wave][t][0][8 * c + 4]);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(&cs[wave][t][1][8 * c]);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(&cs[wave][t][1][8 * c + 4]);
    cv[t][0] = c0.x; cv[t][1] = c0.y; cv[t][2] = c0.z; cv[t][3] = c0.w;
    cv[t][4] = c1.x; cv[t][5] = c1.y; cv[t][6] = c1.z; cv[t][7] = c1.w;
    sv[t][0] = s0.x; sv[t][1] = s0.y; sv[t][2] = s0.z; sv[t][3] = s0.w;
    sv[t][4] = s1.x; sv[t][5] = s1.y; sv[t][6] = s1.z; sv[t][7] = s1.w;
  }
  if constexpr (!kLoadFirst) rope_load<VEC, QD, T, HALF, TPW>(a, bb, ss, live, lane, 0, g);
  rope_store<VEC, QD, T, HALF, TPW>(a, bb, ss, live, lane, 0, g, cv, sv);
  for (int h0 = PG * HPP; h0 < a.HQ + a.HK; h0 += PG * HPP) {
    rope_load<VEC, QD, T, HALF, TPW>(a, bb, ss, live, lane, h0, g);
    rope_store<VEC, QD, T, HALF, TPW>(a, bb, ss, live, lane, h0, g, cv, sv);
  }
}

// Tokens per wavefront: two when a token's heads fit in at most two passes (each lane then
// keeps both tokens' loads in flight at once), else one (its four passes already do).
template <typename T, int HALF>
static void rope_variant(const RopeArgs& a, hipStream_t s) {
  constexpr int HPP = kWave / (HALF / 8);
  const bool qd = a.qd != nullptr;
  const int64_t tokens = a.B * a.S;
  const int passes = (a.HQ + a.HK + HPP - 1) / HPP;
  const int tpw = (a.vec && passes <= 2) ? 2 : 1;
  const int nw = rope_waves(tpw);
  const dim3 b(nw * kWave);
  const dim3 g((unsigned)((tokens + nw * tpw - 1) / (nw * tpw)));
  if (a.vec) {
    if (tpw == 2 && !qd) hipLaunchKernelGGL((k_rope<T, HALF, true, false, 2>), g, b, 0, s, a);
    else if (tpw == 2) hipLaunchKernelGGL((k_rope<T, HALF, true, true, 2>), g, b, 0, s, a);
    else if (!qd) hipLaunchKernelGGL((k_rope<T, HALF, true, false, 1>), g, b, 0, s, a);
    else hipLaunchKernelGGL((k_rope<T, HALF, true, true, 1>), g, b, 0, s, a);
  } else if (!qd) {
    hipLaunchKernelGGL((k_rope<T, HALF, false, false, 1>), g, b, 0, s, a);
  } else {
    hipLaunchKernelGGL((k_rope<T, HALF, false, true, 1>), g, b, 0, s, a);
  }
}

template <typename T>
static hipError_t rope_half(const RopeArgs& a, int half, hipStream_t s, bool* sup) {
  *sup = true;
  switch (half) {
    case 32: rope_variant<T, 32>(a, s); break;
    case 64: rope_variant<T, 64>(a, s); break;
    case 128: rope_variant<T, 128>(a, s); break;
    default: *sup = false; return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_rope(const RopeArgs& a, int dt, int half, hipStream_t s, bool* sup) {
  if (dt == 0) return rope_half<float>(a, half, s, sup);
  if (dt == 1) return rope_half<_Float16>(a, half, s, sup);
  if (dt == 2) return rope_half<__bf16>(a, half, s, sup);
  *sup = false;
  return hipErrorInvalidValue;
}

}  // namespace esep

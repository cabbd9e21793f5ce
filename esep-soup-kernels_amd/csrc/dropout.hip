// Dropout on the LoRA input with the mask regenerated from a key, forward and backward, for
// gfx950. Restates the reference's Triton kernels (solution/body/lora.py:67-137,
// lora_dropout_fwd_kernel / lora_dropout_bwd_kernel):
//   forward   xd = x * keep / (1 - p)
//   backward  xd = x * keep / (1 - p)        (the forward's input of lora_A, regenerated)
//             dx = [dx +] g * keep / (1 - p) (g = dxa @ A; dx may alias g)
// keep(e) = uniform(e) >= p with a mask that is a pure function of (key, e), so the backward
// stores nothing between the passes. The key is one int64 in device memory (drawn by torch's
// CUDA generator; no host sync).
//
// Generator: Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel Random Numbers: As Easy as
// 1, 2, 3", SC 2011), written from the paper. Element e uses word e % 4 of the evaluation at
// counter e / 4 (64-bit, in the first two counter words), key = the two halves of the int64;
// uniform(e) = (word >> 8) * 2^-24. The reference's bit layout is tied to its Triton block and
// is not part of its contract (its docstring: only the law and the regeneration are); this one
// matches oracle/lora_ref.py bit for bit.
//
// Mapping: 8 consecutive elements per thread per step (two Philox evaluations, 16-byte
// accesses for 16-bit types), grid-strided, non-temporal; the n % 8 tail element-wise.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "dropout.hpp"

namespace esep {
namespace {

constexpr int kDropThreads = 256;

struct U4 {
  uint32_t w[4];
};

__device__ __forceinline__ U4 philox4x32_10(uint64_t ctr, uint32_t k0, uint32_t k1) {
  uint32_t c0 = (uint32_t)ctr, c1 = (uint32_t)(ctr >> 32), c2 = 0u, c3 = 0u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r) {
      k0 += 0x9E3779B9u;
      k1 += 0xBB67AE85u;
    }
    // one 32 x 32 -> 64-bit product per multiplier (v_mad_u64_u32) instead of a low and a
    // high half (v_mul_lo_u32 + v_mul_hi_u32, each quarter rate)
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t lo0 = (uint32_t)p0, hi0 = (uint32_t)(p0 >> 32);
    const uint32_t lo1 = (uint32_t)p1, hi1 = (uint32_t)(p1 >> 32);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return U4{{c0, c1, c2, c3}};
}

__device__ __forceinline__ bool keep_of(uint32_t word, float p) {
  return (float)(word >> 8) * 5.9604644775390625e-8f >= p;  // 2^-24
}

template <typename T>
__device__ __forceinline__ void ld8(const T* q, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    typedef T v8t __attribute__((ext_vector_type(8)));
    const v8t r = __builtin_bit_cast(v8t, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(q)));
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Elt<T>::to_f(r[i]);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 r = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(q) + h);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[4 * h + i] = r[i];
    }
  }
}

template <typename T>
__device__ __forceinline__ void st8(T* q, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    typedef T v8t __attribute__((ext_vector_type(8)));
    v8t e;
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = Elt<T>::from_f(v[i]);
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, e), reinterpret_cast<u32x4*>(q));
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 r = {v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
      __builtin_nontemporal_store(r, reinterpret_cast<f32x4*>(q) + h);
    }
  }
}

// keep flags of elements 8c .. 8c + 7 (counters 2c and 2c + 1)
__device__ __forceinline__ void keep8(int64_t c, uint32_t k0, uint32_t k1, float p, bool (&k)[8]) {
  const U4 a = philox4x32_10((uint64_t)(2 * c), k0, k1);
  const U4 b = philox4x32_10((uint64_t)(2 * c + 1), k0, k1);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    k[i] = keep_of(a.w[i], p);
    k[4 + i] = keep_of(b.w[i], p);
  }
}

__device__ __forceinline__ bool keep1(int64_t e, uint32_t k0, uint32_t k1, float p) {
  return keep_of(philox4x32_10((uint64_t)(e / 4), k0, k1).w[e % 4], p);
}

template <typename T>
__global__ __launch_bounds__(kDropThreads) void k_dropout_fwd(const T* x, const int64_t* key,
                                                              T* xd, int64_t n, float p,
                                                              float inv_keep) {
  const uint64_t kk = (uint64_t)*key;
  const uint32_t k0 = (uint32_t)kk, k1 = (uint32_t)(kk >> 32);
  const int64_t chunks = n / 8;
  const int64_t stride = (int64_t)gridDim.x * kDropThreads;
  for (int64_t c = (int64_t)blockIdx.x * kDropThreads + threadIdx.x; c < chunks; c += stride) {
    float v[8];
    bool k[8];
    ld8(x + 8 * c, v);
    keep8(c, k0, k1, p, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = k[i] ? v[i] * inv_keep : 0.f;
    st8(xd + 8 * c, v);
  }
  const int64_t e = 8 * chunks + (int64_t)blockIdx.x * kDropThreads + threadIdx.x;
  if (blockIdx.x == 0 && e < n)
    xd[e] = Elt<T>::from_f(keep1(e, k0, k1, p) ? Elt<T>::to_f(x[e]) * inv_keep : 0.f);
}

template <typename T>
__global__ __launch_bounds__(kDropThreads) void k_dropout_bwd(const T* x, const T* g,
                                                              const int64_t* key, T* xd, T* dx,
                                                              int64_t n, float p, float inv_keep,
                                                              int accumulate) {
  const uint64_t kk = (uint64_t)*key;
  const uint32_t k0 = (uint32_t)kk, k1 = (uint32_t)(kk >> 32);
  const int64_t chunks = n / 8;
  const int64_t stride = (int64_t)gridDim.x * kDropThreads;
  for (int64_t c = (int64_t)blockIdx.x * kDropThreads + threadIdx.x; c < chunks; c += stride) {
    float v[8], gv[8], d[8];
    bool k[8];
    ld8(x + 8 * c, v);
    ld8(g + 8 * c, gv);
    if (accumulate) ld8(dx + 8 * c, d);
    keep8(c, k0, k1, p, k);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[i] = k[i] ? v[i] * inv_keep : 0.f;
      const float t = k[i] ? gv[i] * inv_keep : 0.f;
      d[i] = accumulate ? d[i] + t : t;
    }
    st8(xd + 8 * c, v);
    st8(dx + 8 * c, d);
  }
  const int64_t e = 8 * chunks + (int64_t)blockIdx.x * kDropThreads + threadIdx.x;
  if (blockIdx.x == 0 && e < n) {
    const bool kp = keep1(e, k0, k1, p);
    const float t = kp ? Elt<T>::to_f(g[e]) * inv_keep : 0.f;
    const float d = accumulate ? Elt<T>::to_f(dx[e]) + t : t;
    xd[e] = Elt<T>::from_f(kp ? Elt<T>::to_f(x[e]) * inv_keep : 0.f);
    dx[e] = Elt<T>::from_f(d);
  }
}

unsigned drop_blocks(int64_t n) {
  int64_t b = (n / 8 + kDropThreads - 1) / kDropThreads;
  if (b > 256 * 16) b = 256 * 16;
  return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace

hipError_t launch_dropout_fwd(const void* x, const int64_t* key, void* xd, int64_t n, float p,
                              int dt, hipStream_t s, bool* sup) {
  *sup = true;
  const float inv = 1.f / (1.f - p);
  const dim3 grid(drop_blocks(n)), block(kDropThreads);
  if (dt == 0)
    hipLaunchKernelGGL(k_dropout_fwd<float>, grid, block, 0, s, static_cast<const float*>(x), key,
                       static_cast<float*>(xd), n, p, inv);
  else if (dt == 1)
    hipLaunchKernelGGL(k_dropout_fwd<_Float16>, grid, block, 0, s, static_cast<const _Float16*>(x),
                       key, static_cast<_Float16*>(xd), n, p, inv);
  else if (dt == 2)
    hipLaunchKernelGGL(k_dropout_fwd<__bf16>, grid, block, 0, s, static_cast<const __bf16*>(x), key,
                       static_cast<__bf16*>(xd), n, p, inv);
  else {
    *sup = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dropout_bwd(const void* x, const void* g, const int64_t* key, void* xd, void* dx,
                              int64_t n, float p, int accumulate, int dt, hipStream_t s,
                              bool* sup) {
  *sup = true;
  const float inv = 1.f / (1.f - p);
  const dim3 grid(drop_blocks(n)), block(kDropThreads);
  if (dt == 0)
    hipLaunchKernelGGL(k_dropout_bwd<float>, grid, block, 0, s, static_cast<const float*>(x),
                       static_cast<const float*>(g), key, static_cast<float*>(xd),
                       static_cast<float*>(dx), n, p, inv, accumulate);
  else if (dt == 1)
    hipLaunchKernelGGL(k_dropout_bwd<_Float16>, grid, block, 0, s, static_cast<const _Float16*>(x),
                       static_cast<const _Float16*>(g), key, static_cast<_Float16*>(xd),
                       static_cast<_Float16*>(dx), n, p, inv, accumulate);
  else if (dt == 2)
    hipLaunchKernelGGL(k_dropout_bwd<__bf16>, grid, block, 0, s, static_cast<const __bf16*>(x),
                       static_cast<const __bf16*>(g), key, static_cast<__bf16*>(xd),
                       static_cast<__bf16*>(dx), n, p, inv, accumulate);
  else {
    *sup = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esep

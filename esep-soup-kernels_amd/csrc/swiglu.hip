// SwiGLU for the Qwen2 MLP, h = silu(g) * u, forward and backward, HBM-bound element-wise
// kernels for gfx950. Restates the example kernels the reference decoder calls
// (solution/swiglu.py:15-37, used by packed.py:527-559 and its recompute MLP):
//   s = sigmoid(g) = 1 / (1 + exp(-g))                  in fp32
//   h = g * s * u
//   du = dh * g * s,   dg = dh * u * s * (1 + g * (1 - s))
// One rounding at each store. Every element is read before it is written by the same thread,
// so the outputs may alias the inputs (h into g; dg into g and du into u), as the recompute
// MLP does to save a [T, I] buffer each way.
//
// Mapping: each thread takes 8 consecutive elements (16-byte accesses for 16-bit types) in a
// grid-strided loop over whole 8-element chunks; the n % 8 tail is done element-wise by the
// first threads. Streamed non-temporally (every byte is touched once).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "common.hpp"
#include "swiglu.hpp"

namespace esep {
namespace {

constexpr int kSwThreads = 256;

// sigmoid on the hardware's v_exp_f32 and v_rcp_f32 (each ~1 ulp; no denormal-range or
// division fix-ups: the kernels are memory-bound and keep their VALU work small)
__device__ __forceinline__ float sigmoid_f(float g) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    typedef T v8t __attribute__((ext_vector_type(8)));
    const v8t r = __builtin_bit_cast(v8t, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = Elt<T>::to_f(r[i]);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 r = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p) + h);
#pragma unroll
      for (int i = 0; i < 4; ++i) v[4 * h + i] = r[i];
    }
  }
}

template <typename T>
__device__ __forceinline__ void st8(T* p, const float (&v)[8]) {
  if constexpr (sizeof(T) == 2) {
    typedef T v8t __attribute__((ext_vector_type(8)));
    v8t e;
#pragma unroll
    for (int i = 0; i < 8; ++i) e[i] = Elt<T>::from_f(v[i]);
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4, e), reinterpret_cast<u32x4*>(p));
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const f32x4 r = {v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
      __builtin_nontemporal_store(r, reinterpret_cast<f32x4*>(p) + h);
    }
  }
}

template <typename T>
__global__ __launch_bounds__(kSwThreads) void k_swiglu_fwd(const T* g, const T* u, T* h,
                                                           int64_t n) {
  const int64_t chunks = n / 8;
  const int64_t stride = (int64_t)gridDim.x * kSwThreads;
  for (int64_t c = (int64_t)blockIdx.x * kSwThreads + threadIdx.x; c < chunks; c += stride) {
    float gv[8], uv[8], hv[8];
    ld8(g + 8 * c, gv);
    ld8(u + 8 * c, uv);
#pragma unroll
    for (int i = 0; i < 8; ++i) hv[i] = gv[i] * sigmoid_f(gv[i]) * uv[i];
    st8(h + 8 * c, hv);
  }
  const int64_t t = 8 * chunks + (int64_t)blockIdx.x * kSwThreads + threadIdx.x;
  if (blockIdx.x == 0 && t < n) {
    const float gf = Elt<T>::to_f(g[t]);
    h[t] = Elt<T>::from_f(gf * sigmoid_f(gf) * Elt<T>::to_f(u[t]));
  }
}

template <typename T>
__device__ __forceinline__ void swiglu_grad(float d, float g, float u, float* dg, float* du) {
  const float s = sigmoid_f(g);
  *du = d * g * s;
  *dg = d * u * s * (1.f + g * (1.f - s));
}

template <typename T>
__global__ __launch_bounds__(kSwThreads) void k_swiglu_bwd(const T* dh, const T* g, const T* u,
                                                           T* dg, T* du, int64_t n) {
  const int64_t chunks = n / 8;
  const int64_t stride = (int64_t)gridDim.x * kSwThreads;
  for (int64_t c = (int64_t)blockIdx.x * kSwThreads + threadIdx.x; c < chunks; c += stride) {
    float dv[8], gv[8], uv[8], dgv[8], duv[8];
    ld8(dh + 8 * c, dv);
    ld8(g + 8 * c, gv);
    ld8(u + 8 * c, uv);
#pragma unroll
    for (int i = 0; i < 8; ++i) swiglu_grad<T>(dv[i], gv[i], uv[i], &dgv[i], &duv[i]);
    st8(dg + 8 * c, dgv);
    st8(du + 8 * c, duv);
  }
  const int64_t t = 8 * chunks + (int64_t)blockIdx.x * kSwThreads + threadIdx.x;
  if (blockIdx.x == 0 && t < n) {
    float a, b;
    swiglu_grad<T>(Elt<T>::to_f(dh[t]), Elt<T>::to_f(g[t]), Elt<T>::to_f(u[t]), &a, &b);
    dg[t] = Elt<T>::from_f(a);
    du[t] = Elt<T>::from_f(b);
  }
}

// Enough blocks to fill the GPU several times over, at most one per 8-element chunk.
unsigned sw_blocks(int64_t n) {
  const int64_t chunks = n / 8;
  int64_t b = (chunks + kSwThreads - 1) / kSwThreads;
  if (b > 256 * 16) b = 256 * 16;
  return (unsigned)(b < 1 ? 1 : b);
}

}  // namespace

hipError_t launch_swiglu_fwd(const void* g, const void* u, void* h, int64_t n, int dt,
                             hipStream_t s, bool* sup) {
  *sup = true;
  const dim3 grid(sw_blocks(n)), block(kSwThreads);
  if (dt == 0)
    hipLaunchKernelGGL(k_swiglu_fwd<float>, grid, block, 0, s, static_cast<const float*>(g),
                       static_cast<const float*>(u), static_cast<float*>(h), n);
  else if (dt == 1)
    hipLaunchKernelGGL(k_swiglu_fwd<_Float16>, grid, block, 0, s, static_cast<const _Float16*>(g),
                       static_cast<const _Float16*>(u), static_cast<_Float16*>(h), n);
  else if (dt == 2)
    hipLaunchKernelGGL(k_swiglu_fwd<__bf16>, grid, block, 0, s, static_cast<const __bf16*>(g),
                       static_cast<const __bf16*>(u), static_cast<__bf16*>(h), n);
  else {
    *sup = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_swiglu_bwd(const void* dh, const void* g, const void* u, void* dg, void* du,
                             int64_t n, int dt, hipStream_t s, bool* sup) {
  *sup = true;
  const dim3 grid(sw_blocks(n)), block(kSwThreads);
  if (dt == 0)
    hipLaunchKernelGGL(k_swiglu_bwd<float>, grid, block, 0, s, static_cast<const float*>(dh),
                       static_cast<const float*>(g), static_cast<const float*>(u),
                       static_cast<float*>(dg), static_cast<float*>(du), n);
  else if (dt == 1)
    hipLaunchKernelGGL(k_swiglu_bwd<_Float16>, grid, block, 0, s, static_cast<const _Float16*>(dh),
                       static_cast<const _Float16*>(g), static_cast<const _Float16*>(u),
                       static_cast<_Float16*>(dg), static_cast<_Float16*>(du), n);
  else if (dt == 2)
    hipLaunchKernelGGL(k_swiglu_bwd<__bf16>, grid, block, 0, s, static_cast<const __bf16*>(dh),
                       static_cast<const __bf16*>(g), static_cast<const __bf16*>(u),
                       static_cast<__bf16*>(dg), static_cast<__bf16*>(du), n);
  else {
    *sup = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esep

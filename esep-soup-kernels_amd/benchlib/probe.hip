// Streaming probes for bench.py (not part of libesep_body.so): out = a (+ b) over 16-byte chunks,
// the rate one streaming launch of a given size reaches on the box. bench.py times every variant
// at each path kernel's own byte counts and launch pattern and keeps the fastest as that
// kernel's streaming ceiling.
//
// Variants (U = 16-byte chunks per stream per lane, NT = threads per block):
//   one-shot  the grid covers the data once: each lane issues all U chunks of every stream
//             before its first store (U in flight per stream per lane, nothing waits);
//   strided   a fixed grid walks the data in steps of grid * NT * U chunks; the next step's U
//             chunks per stream are issued before this step's stores (2U in flight).
// Loads and stores are non-temporal buffer accesses with one descriptor per stream (the
// instructions the path kernels use). Sizes up to 4 GiB - 16 per stream.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "probe.h"

// Named (not anonymous) so that the kernels carry "esep" in their symbol names, as the library's
// do (the profiles select kernels by that).
namespace esep_probe {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int kNT = 2;  // non-temporal

__device__ __forceinline__ rsrc_t rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 ld(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNT);
}
__device__ __forceinline__ void st(rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kNT);
}

template <int NS, int U, int NT>
__global__ __launch_bounds__(NT) void k_oneshot(const void* a, const void* b, void* o, uint32_t bytes) {
  const rsrc_t ra = rsrc(a, bytes), rb = rsrc(b, bytes), ro = rsrc(o, bytes);
  const uint32_t base = (blockIdx.x * (uint32_t)(U * NT) + threadIdx.x) * 16u;
  u32x4 va[U], vb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    va[u] = ld(ra, base + u * NT * 16);
    if (NS == 2) vb[u] = ld(rb, base + u * NT * 16);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) st(ro, base + u * NT * 16, NS == 2 ? va[u] + vb[u] : va[u]);
}

template <int NS, int U, int NT>
__global__ __launch_bounds__(NT) void k_strided(const void* a, const void* b, void* o, uint32_t bytes) {
  const rsrc_t ra = rsrc(a, bytes), rb = rsrc(b, bytes), ro = rsrc(o, bytes);
  const uint32_t stepb = gridDim.x * (uint32_t)(U * NT) * 16u;
  uint32_t off = (blockIdx.x * (uint32_t)(U * NT) + threadIdx.x) * 16u;
  const uint32_t steps = (bytes + stepb - 1) / stepb;
  u32x4 va[U], vb[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    va[u] = ld(ra, off + u * NT * 16);
    if (NS == 2) vb[u] = ld(rb, off + u * NT * 16);
  }
  for (uint32_t s = 0; s < steps; ++s) {
    u32x4 r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) r[u] = NS == 2 ? va[u] + vb[u] : va[u];
    const uint32_t nx = off + stepb;
    if (s + 1 < steps) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        va[u] = ld(ra, nx + u * NT * 16);
        if (NS == 2) vb[u] = ld(rb, nx + u * NT * 16);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) st(ro, off + u * NT * 16, r[u]);
    off = nx;
  }
}

typedef void (*kern_t)(const void*, const void*, void*, uint32_t);

template <int NS, int NT>
kern_t pick(int mode, int u) {
  if (mode == ESEP_PROBE_ONESHOT) {
    switch (u) {
      case 1: return k_oneshot<NS, 1, NT>;
      case 2: return k_oneshot<NS, 2, NT>;
      case 4: return k_oneshot<NS, 4, NT>;
      case 8: return k_oneshot<NS, 8, NT>;
    }
  } else {
    switch (u) {
      case 1: return k_strided<NS, 1, NT>;
      case 2: return k_strided<NS, 2, NT>;
      case 4: return k_strided<NS, 4, NT>;
      case 8: return k_strided<NS, 8, NT>;
    }
  }
  return nullptr;
}

}  // namespace esep_probe

using esep_probe::kern_t;
using esep_probe::pick;

extern "C" {

int esep_probe_grid(int mode, int u, int threads, int64_t bytes, int blocks) {
  if (mode == ESEP_PROBE_ONESHOT) {
    const int64_t per_block = (int64_t)u * threads * 16;
    return (int)((bytes + per_block - 1) / per_block);
  }
  return blocks;
}

int esep_probe_stream(int mode, int u, int threads, int blocks, const void* a, const void* b,
                      void* out, int64_t bytes, void* stream) {
  if (a == nullptr || out == nullptr) return -1;
  if (bytes < 0 || bytes > (int64_t{1} << 32) - 16 || (bytes & 15) != 0) return -2;
  if ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
       reinterpret_cast<uintptr_t>(out)) & 15)
    return -3;
  if (mode != ESEP_PROBE_ONESHOT && mode != ESEP_PROBE_STRIDED) return -4;
  if (threads != 256 && threads != 512) return -4;
  if (bytes == 0) return 0;
  const int grid = esep_probe_grid(mode, u, threads, bytes, blocks);
  if (grid < 1) return -2;
  kern_t k = nullptr;
  if (b != nullptr)
    k = threads == 256 ? pick<2, 256>(mode, u) : pick<2, 512>(mode, u);
  else
    k = threads == 256 ? pick<1, 256>(mode, u) : pick<1, 512>(mode, u);
  if (k == nullptr) return -4;
  hipLaunchKernelGGL(k, dim3(grid), dim3(threads), 0, static_cast<hipStream_t>(stream), a, b, out,
                     (uint32_t)bytes);
  return (int)hipGetLastError();
}

}  // extern "C"

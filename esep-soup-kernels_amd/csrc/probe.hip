// Streaming ceiling for measurement: out = a (+ b), 32-bit lanes, over `bytes` bytes. It is not
// part of the decoder path. bench.py times it beside each path kernel at that kernel's own byte
// counts (one or two streams read, one written) and launch pattern (one launch per layer in a
// graph over distinct buffers), as the rate one streaming launch of that size reaches on the
// box. Grid-strided over 16-byte chunks, one chunk per stream per thread per step, non-temporal
// loads and stores, the next step's loads issued before this step's stores.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 512;

template <bool TWO>
__global__ __launch_bounds__(kThreads) void k_stream(const u32x4* __restrict__ a,
                                                     const u32x4* __restrict__ b,
                                                     u32x4* __restrict__ out, int64_t n16) {
  const int64_t step = (int64_t)gridDim.x * kThreads;
  int64_t i = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  u32x4 va = {0u, 0u, 0u, 0u}, vb = {0u, 0u, 0u, 0u};
  if (i < n16) {
    va = __builtin_nontemporal_load(a + i);
    if (TWO) vb = __builtin_nontemporal_load(b + i);
  }
  for (; i < n16; i += step) {
    const u32x4 r = TWO ? va + vb : va;
    const int64_t j = i + step;
    if (j < n16) {
      va = __builtin_nontemporal_load(a + j);
      if (TWO) vb = __builtin_nontemporal_load(b + j);
    }
    __builtin_nontemporal_store(r, out + i);
  }
}

}  // namespace

namespace esep {

hipError_t launch_stream_probe(const void* a, const void* b, void* out, int64_t bytes, int blocks,
                               hipStream_t s) {
  const int64_t n16 = bytes / 16;
  const u32x4* pa = static_cast<const u32x4*>(a);
  const u32x4* pb = static_cast<const u32x4*>(b);
  u32x4* po = static_cast<u32x4*>(out);
  if (b != nullptr)
    hipLaunchKernelGGL(k_stream<true>, dim3(blocks), dim3(kThreads), 0, s, pa, pb, po, n16);
  else
    hipLaunchKernelGGL(k_stream<false>, dim3(blocks), dim3(kThreads), 0, s, pa, pb, po, n16);
  return hipGetLastError();
}

}  // namespace esep

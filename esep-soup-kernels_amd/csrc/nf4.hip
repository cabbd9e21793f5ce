// NF4 (double-quant) weight dequantization for gfx950. Restates the reference's kernel
// (solution/nf4/dequant.py:35-57, nf4_dequant_kernel; the QLoRA / bitsandbytes Linear4bit format
// of its docstring, dequant.py:1-22):
//   scale[b] = fp32(fp32(code2[absmax[b]] * absmax2[b / 256]) + offset)
//   W[e]     = round(fp32(nf4[nibble(e)] * scale[e / 64]))     element 2i: high nibble of byte i
// Every step is rounded separately (contraction into fused multiply-adds is switched off in the
// kernel), which is what makes the result bit-exact with the format's reference decoder.
//
// Mapping: a thread decodes 8 packed bytes (16 elements, a quarter of one 64-element scale
// block) per step, grid-strided: 8-byte loads, two 16-byte (fp16 / bf16) or four 16-byte (fp32)
// stores. The 16-entry NF4 table sits in LDS; each thread rebuilds its block's scale from the
// two small tables in registers.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "nf4.hpp"

namespace esep {
namespace {

constexpr int kNf4Threads = 256;

template <typename TO>
__global__ __launch_bounds__(kNf4Threads) void k_nf4_dequant(const uint8_t* __restrict__ packed,
                                                             const uint8_t* __restrict__ absmax,
                                                             const float* __restrict__ absmax2,
                                                             const float* __restrict__ code2,
                                                             const float* __restrict__ offset,
                                                             const float* __restrict__ nf4,
                                                             TO* __restrict__ out,
                                                             int64_t n_blocks) {
  // Two roundings for the scale: without this the compiler contracts the multiply and the add
  // into one fused multiply-add (one rounding), which differs from the format's decoder. (HIP's
  // __fmul_rn is a plain multiply in a header, outside this pragma, so it does not prevent it.)
#pragma clang fp contract(off)
  __shared__ float tab[16];
  if (threadIdx.x < 16) tab[threadIdx.x] = nf4[threadIdx.x];
  __syncthreads();
  const float off = *offset;
  const int64_t quarters = 4 * n_blocks;
  const int64_t stride = (int64_t)gridDim.x * kNf4Threads;
  for (int64_t i = (int64_t)blockIdx.x * kNf4Threads + threadIdx.x; i < quarters; i += stride) {
    const int64_t b = i >> 2;
    const float prod = code2[absmax[b]] * absmax2[b >> 8];
    const float scale = prod + off;
    const uint2 raw = *reinterpret_cast<const uint2*>(packed + 8 * i);
    float v[16];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t byte = ((j < 4 ? raw.x : raw.y) >> (8 * (j & 3))) & 0xffu;
      v[2 * j] = tab[byte >> 4] * scale;
      v[2 * j + 1] = tab[byte & 15u] * scale;
    }
    TO* o = out + 16 * i;
    if constexpr (sizeof(TO) == 2) {
      typedef TO v8t __attribute__((ext_vector_type(8)));
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        v8t e;
#pragma unroll
        for (int k = 0; k < 8; ++k) e[k] = Elt<TO>::from_f(v[8 * h + k]);
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, e), reinterpret_cast<u32x4*>(o) + h);
      }
    } else {
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const f32x4 e = {v[4 * h], v[4 * h + 1], v[4 * h + 2], v[4 * h + 3]};
        __builtin_nontemporal_store(e, reinterpret_cast<f32x4*>(o) + h);
      }
    }
  }
}

}  // namespace

hipError_t launch_nf4_dequant(const Nf4Args& a, int out_dt, hipStream_t s, bool* sup) {
  *sup = true;
  int64_t blocks = (4 * a.n_blocks + kNf4Threads - 1) / kNf4Threads;
  if (blocks > 256 * 16) blocks = 256 * 16;
  if (blocks < 1) blocks = 1;
  const dim3 grid((unsigned)blocks), block(kNf4Threads);
  const uint8_t* pk = static_cast<const uint8_t*>(a.packed);
  if (out_dt == 0)
    hipLaunchKernelGGL(k_nf4_dequant<float>, grid, block, 0, s, pk, a.absmax, a.absmax2, a.code2,
                       a.offset, a.nf4, static_cast<float*>(a.out), a.n_blocks);
  else if (out_dt == 1)
    hipLaunchKernelGGL(k_nf4_dequant<_Float16>, grid, block, 0, s, pk, a.absmax, a.absmax2, a.code2,
                       a.offset, a.nf4, static_cast<_Float16*>(a.out), a.n_blocks);
  else if (out_dt == 2)
    hipLaunchKernelGGL(k_nf4_dequant<__bf16>, grid, block, 0, s, pk, a.absmax, a.absmax2, a.code2,
                       a.offset, a.nf4, static_cast<__bf16*>(a.out), a.n_blocks);
  else {
    *sup = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esep

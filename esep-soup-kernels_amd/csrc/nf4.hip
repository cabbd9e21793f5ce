// NF4 (double-quant) weight dequantization for gfx950. Restates the reference's kernel
// (solution/nf4/dequant.py:35-57, nf4_dequant_kernel; the QLoRA / bitsandbytes Linear4bit format
// of its docstring, dequant.py:1-22):
//   scale[b] = fp32(fp32(code2[absmax[b]] * absmax2[b / 256]) + offset)
//   W[e]     = round(fp32(nf4[nibble(e)] * scale[e / 64]))     element 2i: high nibble of byte i
// Every step is rounded separately (contraction into fused multiply-adds is switched off in the
// kernel), which is what makes the result bit-exact with the format's reference decoder.
//
// Mapping: a thread decodes 8 packed bytes (16 elements, a quarter of one 64-element scale
// block) per step (k_nf4_dequant: grid-strided; k_nf4_dequant_multi: one quarter per thread over
// several weights laid end to end, the reference's multi-weight kernel, dequant.py:129-166):
// 8-byte loads, two 16-byte (fp16 / bf16) or four 16-byte (fp32) stores. The 16-entry NF4 tables
// sit in LDS. (8 elements per thread, for wavefront-contiguous 16-byte stores, measured slower:
// 32 vs 28.6 us for one layer's seven weights.)
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "nf4.hpp"

namespace esep {
namespace {

constexpr int kNf4Threads = 256;

// Decode quarter i (8 packed bytes, 16 elements) of one weight with its block scale; tab = the
// weight's NF4 table (LDS).
template <typename TO>
__device__ __forceinline__ void nf4_decode(uint2 raw, float scale, const float* tab,
                                           TO* __restrict__ out, int64_t i) {
#pragma clang fp contract(off)
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

// Scale of block b: two roundings (without the pragma the compiler contracts the multiply and
// the add into one fused multiply-add, one rounding, which differs from the format's decoder;
// HIP's __fmul_rn is a plain multiply in a header, outside this pragma, and does not prevent
// it).
__device__ __forceinline__ float nf4_scale(const uint8_t* __restrict__ absmax,
                                           const float* __restrict__ absmax2,
                                           const float* __restrict__ code2, float off, int64_t b) {
#pragma clang fp contract(off)
  const float prod = code2[absmax[b]] * absmax2[b >> 8];
  return prod + off;
}

template <typename TO>
__global__ __launch_bounds__(kNf4Threads) void k_nf4_dequant(const uint8_t* __restrict__ packed,
                                                             const uint8_t* __restrict__ absmax,
                                                             const float* __restrict__ absmax2,
                                                             const float* __restrict__ code2,
                                                             const float* __restrict__ offset,
                                                             const float* __restrict__ nf4,
                                                             TO* __restrict__ out,
                                                             int64_t n_blocks) {
  __shared__ float tab[16];
  if (threadIdx.x < 16) tab[threadIdx.x] = nf4[threadIdx.x];
  __syncthreads();
  const float off = *offset;
  const int64_t quarters = 4 * n_blocks;
  const int64_t stride = (int64_t)gridDim.x * kNf4Threads;
  for (int64_t i = (int64_t)blockIdx.x * kNf4Threads + threadIdx.x; i < quarters; i += stride) {
    const uint2 raw = *reinterpret_cast<const uint2*>(packed + 8 * i);
    nf4_decode<TO>(raw, nf4_scale(absmax, absmax2, code2, off, i >> 2), tab, out, i);
  }
}

// Several weights, one quarter per thread over their concatenation (a weight is whole scale
// blocks, so the 4 quarters of a scale block share a weight). The packed bytes are requested
// first; meanwhile 64 threads resolve the block's 64 scales (absmax -> code2 is a dependent pair
// of loads) into LDS, so only a quarter of the threads wait on that chain. The NF4 tables of
// every weight sit in LDS.
template <typename TO>
__global__ __launch_bounds__(kNf4Threads) void k_nf4_dequant_multi(const Nf4Multi m) {
  __shared__ float tab[kNf4MultiMax][16];
  __shared__ float scl[kNf4Threads / 4];
  const int tid = threadIdx.x;
  const int64_t g0 = (int64_t)blockIdx.x * kNf4Threads;
  const int64_t total = m.q0[m.n];
  auto weight_of = [&](int64_t q) {
    int wi = 0;
#pragma unroll
    for (int k = 1; k < kNf4MultiMax; ++k)
      if (k < m.n && q >= m.q0[k]) wi = k;
    return wi;
  };
  const int64_t g = g0 + tid;
  const bool live = g < total;
  const int wi = live ? weight_of(g) : 0;
  const int64_t i = g - m.q0[wi];  // quarter within the weight
  uint2 raw = make_uint2(0, 0);
  if (live) raw = *reinterpret_cast<const uint2*>(static_cast<const uint8_t*>(m.w[wi].packed) + 8 * i);
  if (tid < 16 * m.n) tab[tid >> 4][tid & 15] = m.w[tid >> 4].nf4[tid & 15];
  if (tid < kNf4Threads / 4) {
    const int64_t gs = g0 + 4 * tid;  // first quarter of this scale block
    if (gs < total) {
      const int ws = weight_of(gs);
      const Nf4Args& w = m.w[ws];
      scl[tid] = nf4_scale(w.absmax, w.absmax2, w.code2, *w.offset, (gs - m.q0[ws]) >> 2);
    }
  }
  __syncthreads();
  if (live) nf4_decode<TO>(raw, scl[tid >> 2], tab[wi], static_cast<TO*>(m.w[wi].out), i);
}

}  // namespace

hipError_t launch_nf4_dequant_multi(const Nf4Multi& m, int out_dt, hipStream_t s, bool* sup) {
  *sup = true;
  const int64_t blocks = (m.q0[m.n] + kNf4Threads - 1) / kNf4Threads;
  if (blocks == 0) return hipSuccess;
  const dim3 grid((unsigned)blocks), block(kNf4Threads);
  if (out_dt == 0)
    hipLaunchKernelGGL(k_nf4_dequant_multi<float>, grid, block, 0, s, m);
  else if (out_dt == 1)
    hipLaunchKernelGGL(k_nf4_dequant_multi<_Float16>, grid, block, 0, s, m);
  else if (out_dt == 2)
    hipLaunchKernelGGL(k_nf4_dequant_multi<__bf16>, grid, block, 0, s, m);
  else {
    *sup = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

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

// RMSNorm forward / backward kernels for gfx950 (MI355X).
//
// Mapping. A row of n columns is cut into n/8 chunks of 8 elements. A "row group" of
// G = 64 * wpr lanes (wpr wavefronts, 1..11) owns one row at a time; lane tg of the group owns
// chunks tg, tg + G, tg + 2G (NV <= 3 of them), so every load and store is a 16-byte access
// and a wavefront instruction covers 1 KiB of contiguous 16-bit data. wpr is the smallest
// count that keeps NV <= 3 (n = 1536: 1 wave, 3 chunks; n = 3584: 3 waves), so a whole row
// stays in registers between the reduction and the output pass (HBM sees each input once) and
// the backward's three row arrays (dy, x, dw accumulators) fit the 128 VGPRs that 16
// wavefronts per CU leave.
//
// Reductions: a wavefront sums on DPP (common.hpp, fixed order); groups of several
// wavefronts add their wave sums through LDS in wave order. Everything is reproducible run
// to run.
//
// Weight gradient (backward): a grid of P blocks (P depends on (rows, n) only,
// esep_rmsnorm_partials) deals the rows out grid-strided: row group g of block b takes rows
// (b + i * P) * gpb + g for i = 0, 1, ..., so the rows in flight at any moment are one
// contiguous stretch of memory (contiguous per-block ranges put P streams a fixed stride apart,
// which measured 8% slower on HBM). Each lane accumulates dy * xhat of its chunks in fp32 over
// the rows of its group, the groups of a block are combined in a fixed order, and the block
// writes one fp32 row of the [P, n] partials. A second kernel sums the partials over P in a
// fixed order. No atomics anywhere: the result depends on (rows, n) and the data only.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace esep {

struct FwdArgs {
  const void* x;
  const void* delta;
  const float* w;
  void* r_out;
  void* y;
  float* rstd;
  const int32_t* slot;
  float* xs;
  int64_t ld_x, ld_d, ld_r, ld_y;
  int64_t rows;
  int n;
  int n_special;
  float eps;
  int wpr;  // wavefronts per row
  int gpb;  // row groups per block (blockDim.x / (64 * wpr))
  int vec;  // 1: every chunk is a whole 16-byte aligned vector
};

struct BwdArgs {
  const void* dy[5];
  int n_dy;
  int64_t ld_dy;
  const float* dr_out;
  const void* x;
  int64_t ld_x;
  int from_y;
  const float* rstd;  // nullptr: recompute from x
  const float* w;
  const int32_t* slot;
  const float* xs;
  int n_special;
  float* dr;    // fp32 [rows, n] or nullptr
  void* dx;     // low-precision copy or nullptr
  int64_t ld_out;
  float* part;  // [P, n] weight-gradient partials or nullptr
  int64_t rows;
  int n;
  float eps;
  int wpr;
  int gpb;  // row groups per block (blockDim.x / (64 * wpr))
  int vec;
  int fast;  // set by the entry point with the launch shape: 0 the general or API kernel,
             // 1 the pipelined kernel (rows of one wavefront), 2 the wide fast kernel
};

constexpr int kFwdMaxThreads = 1024;
constexpr int kMaxNV = 3;
constexpr int kBwdThreads = 1024;  // largest backward block (the launch picks its size)
constexpr int kMaxDy = 5;

// Sum of x over the wavefronts of this row group. `red` holds one float per wavefront.
__device__ __forceinline__ float row_sum(float x, int wpr, float* red) {
  x = wave_sum(x);
  if (wpr == 1) return x;
  const int wave = wave_id();
  if ((threadIdx.x & 63) == 0) red[wave] = x;
  __syncthreads();
  const int g0 = (wave / wpr) * wpr;
  float s = red[g0];
  for (int i = 1; i < wpr; ++i) s += red[g0 + i];
  __syncthreads();
  return s;
}

__device__ __forceinline__ float inv_rms(float ss, int n, float eps) {
  // mean of squares, then 1 / sqrt(ms + eps): correctly rounded fp32 sqrt and divide.
  return 1.0f / sqrtf(ss / (float)n + eps);
}

// Streamed row data (read or written once) is accessed non-temporally; the weight vector and
// the slot table (read by every row) through the caches.
template <bool VEC, typename T, int POL = kStream>
__device__ __forceinline__ void bload(const Span& s, uint32_t off, float (&v)[8]) {
  Buf<T>::template load<VEC, POL>(s, off, v);
}
template <bool VEC, typename T, int POL = kStream>
__device__ __forceinline__ void bstore(const Span& s, uint32_t off, const float (&v)[8]) {
  Buf<T>::template store<VEC, POL>(s, off, v);
}

// Span of row `row` of a [rows, n] tensor with leading dimension ld (elements); a row that
// does not exist gets 0 bytes, so its loads read 0 and its stores vanish.
template <typename T>
__device__ __forceinline__ Span row_rsrc(const void* base, int64_t row, int64_t ld, int n,
                                         bool ok) {
  return make_span(static_cast<const T*>(base) + (ok ? row : 0) * ld,
                   ok ? (uint32_t)n * (uint32_t)sizeof(T) : 0u);
}

// ---------------------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------------------
template <int NV, bool VEC, typename TX, typename TD, typename TY>
__device__ __forceinline__ void fwd_rows(const FwdArgs& a, float* red) {
  const int G = kWave * a.wpr;
  const int gpb = a.gpb;  // blockDim.x would cost a vector load of the hidden kernel arguments
  const int grp = wave_id() / a.wpr;
  const int tg = (int)threadIdx.x - grp * G;
  const int64_t row = (int64_t)blockIdx.x * gpb + grp;
  const bool ok = row < a.rows;
  const int n = a.n;

  float v[NV][8];
  const Span rx = row_rsrc<TX>(a.x, row, a.ld_x, n, ok);
#pragma unroll
  for (int k = 0; k < NV; ++k) bload<VEC, TX>(rx, (tg + k * G) * 8 * sizeof(TX), v[k]);

  if constexpr (!std::is_void_v<TD>) {
    const Span rd = row_rsrc<TD>(a.delta, row, a.ld_d, n, ok);
    float d[NV][8];
#pragma unroll
    for (int k = 0; k < NV; ++k) bload<VEC, TD>(rd, (tg + k * G) * 8 * sizeof(TD), d[k]);
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) v[k][e] = Elt<TX>::round(v[k][e] + d[k][e]);
    if (a.r_out != nullptr) {
      const Span rr = row_rsrc<TX>(a.r_out, row, a.ld_r, n, ok);
#pragma unroll
      for (int k = 0; k < NV; ++k) bstore<VEC, TX>(rr, (tg + k * G) * 8 * sizeof(TX), v[k]);
    }
  }

  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(v[k][e], v[k][e], ss);
  ss = row_sum(ss, a.wpr, red);
  const float inv = inv_rms(ss, n, a.eps);

  // every weight chunk is loaded before the first y store, so no weight load waits behind a
  // store in the one in-order counter of loads and stores (config 5: 163.2 -> 162.3 us)
  const Span rw = make_span(a.w, (uint32_t)n * 4u);
  const Span ry = row_rsrc<TY>(a.y, row, a.ld_y, n, ok);
  float w8[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k) bload<VEC, float, kCached>(rw, (tg + k * G) * 32, w8[k]);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = w8[k][e] * (v[k][e] * inv);
    bstore<VEC, TY>(ry, (tg + k * G) * 8 * sizeof(TY), o);
  }
  if (a.rstd != nullptr && ok && tg == 0) a.rstd[row] = inv;

  if (a.n_special > 0 && ok) {
    const Span rs = make_span(a.slot, (uint32_t)n * 4u);
    float* xsr = a.xs + row * (int64_t)a.n_special;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      const int col = 8 * (tg + k * G);
      int s8[8];
      buf_load8_i32<VEC>(rs, col * 4, s8);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (col + e < n && s8[e] >= 0) xsr[s8[e]] = v[k][e] * inv;
    }
  }
}

// The forward without exact channels (plain, or residual add with a delta) with RPW rows per
// row group: every row's x (and delta) is loaded (raw, still packed) before any row is reduced.
// Launched for rows of one wavefront (wpr = 1) in blocks of 256 threads only. The weight vector
// goes into LDS (wl, NV * 512 floats) once per block, behind the row loads, and every row reads
// it from there: read from global memory per row, each row's weight loads sat behind the previous
// row's y stores in the one in-order counter of loads and stores, so every row waited for the
// previous row's stores (config 4 step: 2.010 -> 1.998 ms; weight loads issued ahead of the row
// loads instead: 2.018 ms).
template <int NV, typename TX, typename TD, typename TY, int RPW>
__device__ __forceinline__ void fwd_rows_multi(const FwdArgs& a, float* red, float* wl) {
  const int G = kWave * a.wpr;
  const int gpb = a.gpb;
  const int grp = wave_id() / a.wpr;
  const int tg = (int)threadIdx.x - grp * G;
  const int n = a.n;
  const int64_t row0 = ((int64_t)blockIdx.x * gpb + grp) * RPW;
  constexpr bool kDelta = !std::is_void_v<TD>;
  using TDR = std::conditional_t<kDelta, TD, TX>;  // a type for the unused delta registers
  Raw<TX> rx[RPW][NV];
  Raw<TDR> rd[kDelta ? RPW : 1][NV];
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    const Span sx = row_rsrc<TX>(a.x, row, a.ld_x, n, row < a.rows);
#pragma unroll
    for (int k = 0; k < NV; ++k)
      rx[r][k] = Buf<TX>::template load_raw<kStream>(sx, (tg + k * G) * 8 * sizeof(TX));
    if constexpr (kDelta) {
      const Span sd = row_rsrc<TD>(a.delta, row, a.ld_d, n, row < a.rows);
#pragma unroll
      for (int k = 0; k < NV; ++k)
        rd[r][k] = Buf<TD>::template load_raw<kStream>(sd, (tg + k * G) * 8 * sizeof(TD));
    }
  }
  {  // threads 0 .. NV * 64 - 1 copy 8 weights each (past n: 0)
    const Span rw = make_span(a.w, (uint32_t)n * 4u);
    const int c = (int)threadIdx.x;
    if (c < NV * kWave) {
      float w8[8];
      bload<true, float, kCached>(rw, c * 32, w8);
      Chunk<float>::store(wl + 8 * c, w8);
    }
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const int64_t row = row0 + r;
    const bool ok = row < a.rows;
    float v[NV][8];
#pragma unroll
    for (int k = 0; k < NV; ++k) Buf<TX>::unpack(rx[r][k], v[k]);
    if constexpr (kDelta) {
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        float d[8];
        Buf<TD>::unpack(rd[r][k], d);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] = Elt<TX>::round(v[k][e] + d[e]);
      }
      if (a.r_out != nullptr) {
        const Span rr = row_rsrc<TX>(a.r_out, row, a.ld_r, n, ok);
#pragma unroll
        for (int k = 0; k < NV; ++k) bstore<true, TX>(rr, (tg + k * G) * 8 * sizeof(TX), v[k]);
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[k][e], v[k][e], ss);
    const float inv = inv_rms(row_sum(ss, a.wpr, red), n, a.eps);
    const Span ry = row_rsrc<TY>(a.y, row, a.ld_y, n, ok);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float w8[8], o[8];
      Chunk<float>::load(wl + 8 * (tg + k * G), w8);
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = w8[e] * (v[k][e] * inv);
      bstore<true, TY>(ry, (tg + k * G) * 8 * sizeof(TY), o);
    }
    if (a.rstd != nullptr && ok && tg == 0) a.rstd[row] = inv;
  }
}

template <int NV, typename TX, typename TD, typename TY, int RPW>
__global__ __launch_bounds__(kFwdMaxThreads) void k_rmsnorm_fwd_multi(const FwdArgs a) {
  __shared__ float red[kFwdMaxThreads / kWave];
  __shared__ __align__(16) float wl[NV * kWave * 8];
  fwd_rows_multi<NV, TX, TD, TY, RPW>(a, red, wl);
}

// VEC kernels are instantiated for NV = 2, 3; the element-wise (!VEC) kernel only for
// NV = 3, which serves every row width (surplus chunks lie past the row and read 0).
template <int NV, bool VEC, typename TX, typename TD, typename TY>
__global__ __launch_bounds__(kFwdMaxThreads) void k_rmsnorm_fwd(const FwdArgs a) {
  __shared__ float red[kFwdMaxThreads / kWave];
  fwd_rows<NV, VEC, TX, TD, TY>(a, red);
}

// Weight-gradient partial of one block: a fixed tree over the gpb row groups (at each level
// the groups [half, 2 half) park their accumulators in LDS and the groups below add them; the
// LDS slot stride NV * G * 8 floats keeps chunks past the row end inside their slot), then
// group 0 writes the block sum as row blockIdx.x of the [P, n] partials.
template <int NV, bool VEC>
__device__ __forceinline__ void dw_block_partial(const BwdArgs& a, float (&acc)[NV][8],
                                                 float* lds, int grp, int gpb, int tg, int G) {
  const int n = a.n;
  const int stride = NV * G * 8;
  int top = 1;
  while (top < gpb) top <<= 1;
  for (int half = top >> 1; half >= 1; half >>= 1) {
    if (grp >= half && grp < 2 * half && grp < gpb) {
      float* dst = lds + (grp - half) * stride;
#pragma unroll
      for (int k = 0; k < NV; ++k) Chunk<float>::store(dst + 8 * (tg + k * G), acc[k]);
    }
    __syncthreads();
    if (grp < half && grp + half < gpb) {
      const float* src = lds + grp * stride;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        float t[8];
        Chunk<float>::load(src + 8 * (tg + k * G), t);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[k][e] += t[e];
      }
    }
    __syncthreads();
  }
  if (grp == 0) {
    const Span rp = make_span(a.part + (int64_t)blockIdx.x * n, (uint32_t)n * 4u);
#pragma unroll
    for (int k = 0; k < NV; ++k) bstore<VEC, float, kCached>(rp, (tg + k * G) * 32, acc[k]);
  }
}

// ---------------------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------------------
template <int NV, bool VEC, typename TX, typename TDY, typename TO>
__device__ __forceinline__ void bwd_rows(const BwdArgs& a, float* red, float* lds) {
  const int G = kWave * a.wpr;
  const int gpb = a.gpb;  // blockDim.x would cost a vector load of the hidden kernel arguments
  const int grp = wave_id() / a.wpr;
  const int tg = (int)threadIdx.x - grp * G;
  const int n = a.n;
  const int64_t step = (int64_t)gridDim.x * gpb;  // grid-strided rows
  const int64_t first = (int64_t)blockIdx.x * gpb + grp;
  const int iters = (int)((a.rows + step - 1) / step);
  const bool want_dw = a.part != nullptr;
  const Span rw = make_span(a.w, (uint32_t)n * 4u);

  float acc[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[k][e] = 0.f;

  for (int it = 0; it < iters; ++it) {
    const int64_t row = first + (int64_t)it * step;
    const bool ok = row < a.rows;
    float dr[NV][8];

    if (a.n_dy > 0) {
      // Everything is updated in place so that three row-sized register arrays are live at
      // most (acc, dy -> g -> dr, x -> xhat).
      float dy[NV][8], x[NV][8];
      {
        const Span r0 = row_rsrc<TDY>(a.dy[0], row, a.ld_dy, n, ok);
        const Span rx = row_rsrc<TX>(a.x, row, a.ld_x, n, ok);
#pragma unroll
        for (int k = 0; k < NV; ++k) bload<VEC, TDY>(r0, (tg + k * G) * 8 * sizeof(TDY), dy[k]);
#pragma unroll
        for (int k = 0; k < NV; ++k) bload<VEC, TX>(rx, (tg + k * G) * 8 * sizeof(TX), x[k]);
      }
      // Further consumers' gradients, summed in fp32 (constant indices: no private copy of
      // the pointer array; one gradient at a time keeps the registers of the common path).
#pragma unroll 1
      for (int i = 1; i < kMaxDy; ++i) {
        if (i < a.n_dy) {
          const Span ri = row_rsrc<TDY>(a.dy[i], row, a.ld_dy, n, ok);
#pragma unroll
          for (int k = 0; k < NV; ++k) {
            float t[8];
            bload<VEC, TDY>(ri, (tg + k * G) * 8 * sizeof(TDY), t);
#pragma unroll
            for (int e = 0; e < 8; ++e) dy[k][e] += t[e];
          }
        }
      }

      // rstd: saved, or recomputed from x exactly as the forward computed it.
      float inv;
      if (a.rstd == nullptr) {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < NV; ++k)
#pragma unroll
          for (int e = 0; e < 8; ++e) ss = fmaf(x[k][e], x[k][e], ss);
        inv = inv_rms(row_sum(ss, a.wpr, red), n, a.eps);
      } else {
        inv = ok ? a.rstd[row] : 1.f;
      }

      // x -> xhat
      if (a.from_y) {
        // xhat = y / w for the columns of the row (0 beyond it: no 0 / 0), as y times the
        // hardware reciprocal of w (v_rcp_f32, about 1 ulp; the reference's Triton division
        // is itself approximate, and y carries 16-bit rounding): the correctly rounded
        // division costs ~10 instructions per element and made this call compute-bound. The
        // exact channels (w tiny, huge or not finite) come from xs.
#pragma unroll
        for (int k = 0; k < NV; ++k) {
          const int col = 8 * (tg + k * G);
          float w8[8];
          bload<VEC, float, kCached>(rw, col * 4, w8);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            x[k][e] = x[k][e] * __builtin_amdgcn_rcpf(col + e < n ? w8[e] : 1.f);
        }
        if (a.n_special > 0 && ok) {
          const Span rs = make_span(a.slot, (uint32_t)n * 4u);
          const float* xsr = a.xs + row * (int64_t)a.n_special;
#pragma unroll
          for (int k = 0; k < NV; ++k) {
            const int col = 8 * (tg + k * G);
            int s8[8];
            buf_load8_i32<VEC>(rs, col * 4, s8);
#pragma unroll
            for (int e = 0; e < 8; ++e)
              if (col + e < n && s8[e] >= 0) x[k][e] = xsr[s8[e]];
          }
        }
      } else {
#pragma unroll
        for (int k = 0; k < NV; ++k)
#pragma unroll
          for (int e = 0; e < 8; ++e) x[k][e] *= inv;
      }

      if (want_dw && ok) {
#pragma unroll
        for (int k = 0; k < NV; ++k)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[k][e] = fmaf(dy[k][e], x[k][e], acc[k][e]);
      }

      // dy -> g = dy * w; proj = sum g * xhat / n
      float p = 0.f;
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        float w8[8];
        bload<VEC, float, kCached>(rw, (tg + k * G) * 32, w8);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dy[k][e] *= w8[e];
          p = fmaf(dy[k][e], x[k][e], p);
        }
      }
      const float proj = row_sum(p, a.wpr, red) / (float)n;

      // g -> dr = rstd * (g - xhat * proj)
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) dr[k][e] = inv * (dy[k][e] - x[k][e] * proj);
    } else {
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) dr[k][e] = 0.f;
    }

    if (a.dr_out != nullptr) {
      const Span ro = row_rsrc<float>(a.dr_out, row, a.ld_out, n, ok);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        float t[8];
        bload<VEC, float>(ro, (tg + k * G) * 32, t);
#pragma unroll
        for (int e = 0; e < 8; ++e) dr[k][e] += t[e];
      }
    }
    if (a.dr != nullptr) {
      const Span ro = row_rsrc<float>(a.dr, row, a.ld_out, n, ok);
#pragma unroll
      for (int k = 0; k < NV; ++k) bstore<VEC, float>(ro, (tg + k * G) * 32, dr[k]);
    }
    if (a.dx != nullptr) {
      const Span ro = row_rsrc<TO>(a.dx, row, a.ld_out, n, ok);
#pragma unroll
      for (int k = 0; k < NV; ++k) bstore<VEC, TO>(ro, (tg + k * G) * 8 * sizeof(TO), dr[k]);
    }
  }

  if (want_dw) dw_block_partial<NV, VEC>(a, acc, lds, grp, gpb, tg, G);
}

// The pipelined backward runs blocks of 4 wavefronts (one row group each), one block per CU at
// config-4 sizes, so each wavefront may hold up to 512 registers without lowering occupancy.
constexpr int kBwdPipeThreads = 256;

// Fast backward for the common call (one gradient of y, xhat from x, not from y, no dr_out,
// 16-byte-aligned whole chunks) on rows of one wavefront (n <= 1536). Rows are grid-strided (row
// group g of block b takes rows (b + i * P) * gpb + g, so the rows in flight at any moment are
// one contiguous stretch of memory).
//
// Schedule. Two register sets with fixed roles hold the raw (still packed) dy and x of two
// rows: row i is computed from set i % 2, then row i + 2's loads are issued into the same set,
// then row i's dx is stored. Scheduling barriers pin that order (the compiler otherwise sinks
// the next row's loads into the middle of the current row's arithmetic, which leaves about one
// row in flight). The loads of row i + 1 are thus always in flight while row i is computed,
// and the stores are issued after the loads they follow, so no wait for a row's data ever
// waits for a store (gfx9's vmcnt counts loads and stores in one in-order counter). Row 0 is
// peeled off and the last row is kept out of the loop, so the loop is entered with the same
// outstanding operations as it loops back with and its waits stay exact. Each lane owns the same
// columns of every row, so its weight chunks (NV * 8 floats) are loaded once into registers.
// The saved rstd of the group's rows comes in one vector load and is read per row with readlane;
// the entry point sends inputs of more than 64 rows per group to the wide kernel.
//
// Weight gradient: each lane sums dy * xhat of its chunks in registers over its group's rows;
// after the last row the groups park their sums in one LDS slot each (NV * G * 8 floats, indexed
// by column) and, after one barrier, every thread adds the slots of column pairs 2t, 2t + 2 *
// threads, ... in group order and stores them as the block's row of the [P, n] partials. These
// stores are cached, unlike the streamed rows: stage 2 re-reads the partials (right after the
// launch in the per-call schedule, at the end of the pass in the deferred one), and cached they
// can still be in the Infinity Cache then. Against non-temporal partial stores, config 4 per
// call 2.243 -> 2.199 ms, deferred 1.997-2.004 -> 1.987-2.005 ms over four paired runs (the
// launch alone 0.1 us slower); the same bits.
//
// Measured at config 4 (8192 x 1536 bf16, 256 blocks of 4 wavefronts, graphs of 57 launches):
// 15.19 us with the compiler's placement (a full wait at the loop head, one row in flight),
// 14.9 us pinned. Ablations of the pinned kernel: no arithmetic (a raw copy of the same rows)
// 13.7 us, arithmetic without the partials' store 14.3 us.
//
// FIX fixes the call's optional parts at compile time: 1 = saved rstd, dx only, with the weight
// gradient; 2 = the same without it; 3 = rstd recomputed from x, dx only, with the weight
// gradient; 0 reads them from the arguments.
template <int NV, typename TX, typename TDY, typename TO, int FIX>
__device__ __forceinline__ void bwd_rows_pipe(const BwdArgs& a, float* lds) {
  constexpr int G = kWave;  // one wavefront per row: every row reduction is a DPP wave sum
  constexpr int gpb = kBwdPipeThreads / kWave;  // the launch is checked to match
  const int grp = wave_id();
  const int tg = (int)threadIdx.x & (kWave - 1);
  const int lane = tg;
  const int n = a.n;
  // 32-bit scalar row indices (the entry point sends rows < 2^30 here)
  const int rows = (int)a.rows;
  const int step = (int)gridDim.x * gpb;  // grid-strided rows
  const int first = (int)blockIdx.x * gpb + grp;
  const int iters = (rows - first + step - 1) / step;  // rows of this group
  // rows of the block's groups (block-uniform: the groups of a block differ by at most one row;
  // a group's surplus rows read 0 and store nothing), at least 1
  const int iters_blk = (rows - (int)blockIdx.x * gpb + step - 1) / step;
  const bool want_dw = (FIX == 1 || FIX == 3) ? true : FIX == 2 ? false : a.part != nullptr;
  const bool has_rstd = (FIX == 1 || FIX == 2) ? true : FIX == 3 ? false : a.rstd != nullptr;
  const bool has_dr = FIX == 0 && a.dr != nullptr;
  const bool has_dx = FIX != 0 || a.dx != nullptr;
  const float inv_n = 1.0f / (float)n;

  float wr[NV][8];  // chunks past the row read 0
  {
    const Span rw = make_span(a.w, (uint32_t)n * 4u);
#pragma unroll
    for (int k = 0; k < NV; ++k) bload<true, float, kCached>(rw, (tg + k * G) * 32, wr[k]);
  }
  // Saved rstd of this group's rows (at most 64): lane l holds row first + l * step.
  float rstd64 = 1.f;
  auto load_rstd = [&](int it0) {
    if (has_rstd) {
      const int it = it0 + lane;
      rstd64 = it < iters ? a.rstd[first + (int64_t)it * step] : 1.f;
    }
  };

  Raw<TDY> rdy[2][NV];
  Raw<TX> rx[2][NV];
  // Loads of row `it` of this group into register set `set`; a row past the end gets 0-byte
  // buffers (its loads read 0 without touching memory).
  auto fetch = [&](int set, int it) {
    const int row = first + it * step;
    const bool ok = row < rows;
    const Span sd = row_rsrc<TDY>(a.dy[0], row, a.ld_dy, n, ok);
    const Span sx = row_rsrc<TX>(a.x, row, a.ld_x, n, ok);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      rdy[set][k] = Buf<TDY>::template load_raw<kStream>(sd, (tg + k * G) * 8 * sizeof(TDY));
      rx[set][k] = Buf<TX>::template load_raw<kStream>(sx, (tg + k * G) * 8 * sizeof(TX));
    }
  };

  float dwa[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) dwa[k][e] = 0.f;

  // Row `it` of this group from register set `set` into o:
  // dx = rstd * (g - xhat * mean(g * xhat)), g = dy * w.
  float o[NV][8];
  auto compute = [&](int set, int it) {
    float dy[NV][8], x[NV][8];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      Buf<TDY>::unpack(rdy[set][k], dy[k]);
      Buf<TX>::unpack(rx[set][k], x[k]);
    }
    float inv;
    if (has_rstd) {
      inv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rstd64), it & (kWave - 1)));
    } else {
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x[k][e], x[k][e], ss);
      inv = inv_rms(wave_sum(ss), n, a.eps);
    }
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[k][e] *= inv;
    if (want_dw) {
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) dwa[k][e] = fmaf(dy[k][e], x[k][e], dwa[k][e]);
    }
    float p = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dy[k][e] *= wr[k][e];
        p = fmaf(dy[k][e], x[k][e], p);
      }
    const float proj = wave_sum(p) * inv_n;
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[k][e] = inv * (dy[k][e] - x[k][e] * proj);
  };
  auto store = [&](int it) {
    const int row = first + it * step;
    const bool ok = row < rows;  // a row that does not exist has dy = x = 0: adds nothing
    if (has_dr) {
      const Span so = row_rsrc<float>(a.dr, row, a.ld_out, n, ok);
#pragma unroll
      for (int k = 0; k < NV; ++k) bstore<true, float>(so, (tg + k * G) * 32, o[k]);
    }
    if (has_dx) {
      const Span so = row_rsrc<TO>(a.dx, row, a.ld_out, n, ok);
#pragma unroll
      for (int k = 0; k < NV; ++k) bstore<true, TO>(so, (tg + k * G) * 8 * sizeof(TO), o[k]);
    }
  };
  // row `it` from `set`, then row it + 2 into the same set, then row it's stores
  auto finish = [&](int set, int it) {
    compute(set, it);
    __builtin_amdgcn_sched_barrier(0);
    fetch(set, it + 2);
    __builtin_amdgcn_sched_barrier(0);
    store(it);
  };

  // The two-set pipeline over this group's rows 0 .. iters_blk - 1 (at most 64, one saved-rstd
  // window: the entry point sends longer runs to the wide kernel).
  load_rstd(0);
  fetch(0, 0);
  fetch(1, 1);
  __builtin_amdgcn_sched_barrier(0);
  if (iters_blk == 1) {
    compute(0, 0);
    store(0);
  } else {
    finish(0, 0);
    int it = 1;  // rows it (set 1) and it + 1 (set 0) per pass; the last row after the loop
    for (; it + 2 < iters_blk; it += 2) {
      finish(1, it);
      finish(0, it + 1);
    }
    if (it + 1 < iters_blk) {
      finish(1, it);
      compute(0, it + 1);
      store(it + 1);
    } else {
      compute(1, it);
      store(it);
    }
  }

  if (want_dw) {
    const int stride = NV * G * 8;  // floats per slot (>= n; the tail past n stays 0)
    float* acc = lds + grp * stride;
#pragma unroll
    for (int k = 0; k < NV; ++k) Chunk<float>::store(acc + 8 * (tg + k * G), dwa[k]);
    __syncthreads();  // LDS only: on gfx950 this waits for LDS writes, not for the dx stores
    // block sum of column pairs 2t, 2t + 2 * threads, ..., groups added in group order
    const rsrc_t rp = make_rsrc(a.part + (int64_t)blockIdx.x * n, (uint32_t)n * 4u);
    constexpr int nthr = gpb * G;
#pragma unroll
    for (int j = 0; j < (NV * G * 8 + 2 * nthr - 1) / (2 * nthr); ++j) {  // every pair of the slot
      const int c = 2 * (int)threadIdx.x + 2 * nthr * j;
      if (c < n) {
        float2 t = *reinterpret_cast<const float2*>(lds + c);
#pragma unroll
        for (int g = 1; g < gpb; ++g) {
          const float2 u = *reinterpret_cast<const float2*>(lds + g * stride + c);
          t.x += u.x;
          t.y += u.y;
        }
        typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{__float_as_uint(t.x), __float_as_uint(t.y)},
                                              rp, (uint32_t)c * 4u, 0, kCached);
      }
    }
  }
}

template <int NV, typename TX, typename TDY, typename TO, int FIX>
__global__ __launch_bounds__(kBwdPipeThreads) void k_rmsnorm_bwd_pipe(const BwdArgs a) {
  extern __shared__ float lds[];
  bwd_rows_pipe<NV, TX, TDY, TO, FIX>(a, lds);
}

// Fast backward for rows of several wavefronts (n > 1536): the same call pattern as
// bwd_rows_pipe. LDS holds, per block, the weight vector (staged once, read by every row instead
// of through L2: at n = 3584 that is 14 KiB per row) and, with a weight gradient, one slot of
// NV * G * 8 floats per row group, indexed by column. Each lane keeps its dy * xhat sums in
// registers over the rows of its group, parks them in its group's slot at the end, and the
// block sums the slots in group order. Each row's dy and x are loaded at the top of its
// iteration: at n = 3584 (three wavefronts per row, a barrier in every row reduction) the
// pipelined form measured slower (config 5 backward 242 -> 262 us).
template <int NV, typename TX, typename TDY, typename TO>
__device__ __forceinline__ void bwd_rows_wide(const BwdArgs& a, float* red, float* lds) {
  const int G = kWave * a.wpr;
  const int gpb = a.gpb;  // blockDim.x would cost a vector load of the hidden kernel arguments
  const int grp = wave_id() / a.wpr;
  const int tg = (int)threadIdx.x - grp * G;
  const int n = a.n;
  const int64_t step = (int64_t)gridDim.x * gpb;  // grid-strided rows
  const int64_t first = (int64_t)blockIdx.x * gpb + grp;
  const int iters = (int)((a.rows + step - 1) / step);
  const bool want_dw = a.part != nullptr;
  const float inv_n = 1.0f / (float)n;
  const int stride = NV * G * 8;  // floats per slot (>= n; the tail past n stays 0)
  float* acc = lds + grp * stride;
  float* wl = lds + (want_dw ? gpb * stride : 0);
  for (int q = threadIdx.x; q < stride / 4; q += gpb * G) {
    f32x4 t = {0.f, 0.f, 0.f, 0.f};
    if (4 * q < n) t = *reinterpret_cast<const f32x4*>(a.w + 4 * q);
    *reinterpret_cast<f32x4*>(wl + 4 * q) = t;
  }
  float dwa[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k)
#pragma unroll
    for (int e = 0; e < 8; ++e) dwa[k][e] = 0.f;
  __syncthreads();

  for (int it = 0; it < iters; ++it) {
    const int64_t row = first + (int64_t)it * step;
    const bool ok = row < a.rows;  // a row that does not exist reads 0 and writes nothing
    Raw<TDY> rdy[NV];
    Raw<TX> rx[NV];
    {
      const Span sd = row_rsrc<TDY>(a.dy[0], row, a.ld_dy, n, ok);
      const Span sx = row_rsrc<TX>(a.x, row, a.ld_x, n, ok);
#pragma unroll
      for (int k = 0; k < NV; ++k) {
        rdy[k] = Buf<TDY>::template load_raw<kStream>(sd, (tg + k * G) * 8 * sizeof(TDY));
        rx[k] = Buf<TX>::template load_raw<kStream>(sx, (tg + k * G) * 8 * sizeof(TX));
      }
    }
    float inv = (a.rstd != nullptr && ok) ? a.rstd[row] : 1.f;

    float dy[NV][8], x[NV][8];
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      Buf<TDY>::unpack(rdy[k], dy[k]);
      Buf<TX>::unpack(rx[k], x[k]);
    }
    if (a.rstd == nullptr) {
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < NV; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) ss = fmaf(x[k][e], x[k][e], ss);
      inv = inv_rms(row_sum(ss, a.wpr, red), n, a.eps);
    }
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) x[k][e] *= inv;
    // (a row that does not exist has dy = x = 0 and adds nothing)
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) dwa[k][e] = fmaf(dy[k][e], x[k][e], dwa[k][e]);
    float p = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float w8[8];
      Chunk<float>::load(wl + 8 * (tg + k * G), w8);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        dy[k][e] *= w8[e];
        p = fmaf(dy[k][e], x[k][e], p);
      }
    }
    const float proj = row_sum(p, a.wpr, red) * inv_n;
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) dy[k][e] = inv * (dy[k][e] - x[k][e] * proj);
    if (a.dr != nullptr) {
      const Span so = row_rsrc<float>(a.dr, row, a.ld_out, n, ok);
#pragma unroll
      for (int k = 0; k < NV; ++k) bstore<true, float>(so, (tg + k * G) * 32, dy[k]);
    }
    if (a.dx != nullptr) {
      const Span so = row_rsrc<TO>(a.dx, row, a.ld_out, n, ok);
#pragma unroll
      for (int k = 0; k < NV; ++k) bstore<true, TO>(so, (tg + k * G) * 8 * sizeof(TO), dy[k]);
    }
  }
  if (want_dw) {
#pragma unroll
    for (int k = 0; k < NV; ++k) Chunk<float>::store(acc + 8 * (tg + k * G), dwa[k]);
    // block sum: column quads over all threads, groups added in group order
    __syncthreads();
    float* dst = a.part + (int64_t)blockIdx.x * n;
    for (int q = threadIdx.x; 4 * q < n; q += gpb * G) {
      f32x4 t = *reinterpret_cast<const f32x4*>(lds + 4 * q);
      for (int g = 1; g < gpb; ++g) t += *reinterpret_cast<const f32x4*>(lds + g * stride + 4 * q);
      *reinterpret_cast<f32x4*>(dst + 4 * q) = t;
    }
  }
}

template <int NV, typename TX, typename TDY, typename TO>
__global__ __launch_bounds__(kBwdThreads) void k_rmsnorm_bwd_wide(const BwdArgs a) {
  __shared__ float red[kBwdThreads / kWave];
  extern __shared__ float lds[];
  bwd_rows_wide<NV, TX, TDY, TO>(a, red, lds);
}

// Backward of the reference API's calls without a weight gradient or exact channels (up to 5
// gradients of y, dr_out, xhat from x or from y = w * xhat) in blocks of at most 256 threads:
// every load of a row (all dys, x, dr_out) is issued before any is used. The general kernel
// keeps within 128 registers by loading them one after another, a chain of dependent memory
// round trips per row. Inputs that are absent get 0-byte buffers: they read 0 and cost no
// memory access, and the absent gradients add +0 (the same sums as the general kernel).
constexpr int kBwdApiThreads = 256;
template <int NV, typename TX, typename TDY, typename TO>
__global__ __launch_bounds__(kBwdApiThreads) void k_rmsnorm_bwd_api(const BwdArgs a) {
  __shared__ float red[kBwdApiThreads / kWave];
  const int G = kWave * a.wpr;
  const int grp = wave_id() / a.wpr;
  const int tg = (int)threadIdx.x - grp * G;
  const int n = a.n;
  const int64_t row = (int64_t)blockIdx.x * a.gpb + grp;
  const bool ok = row < a.rows;
  Raw<TDY> rdy[kMaxDy][NV];
  Raw<TX> rx[NV];
  Raw<float> ro[NV];
#pragma unroll
  for (int i = 0; i < kMaxDy; ++i) {
    const Span sd = row_rsrc<TDY>(a.dy[i], row, a.ld_dy, n, ok && i < a.n_dy);
#pragma unroll
    for (int k = 0; k < NV; ++k)
      rdy[i][k] = Buf<TDY>::template load_raw<kStream>(sd, (tg + k * G) * 8 * sizeof(TDY));
  }
  {
    const Span sx = row_rsrc<TX>(a.x, row, a.ld_x, n, ok);
    const Span so = row_rsrc<float>(a.dr_out, row, a.ld_out, n, ok && a.dr_out != nullptr);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      rx[k] = Buf<TX>::template load_raw<kStream>(sx, (tg + k * G) * 8 * sizeof(TX));
      ro[k] = Buf<float>::template load_raw<kStream>(so, (tg + k * G) * 32);
    }
  }
  const float rstd_saved = (a.rstd != nullptr && ok) ? a.rstd[row] : 1.f;
  const Span rw = make_span(a.w, (uint32_t)n * 4u);

  float dy[NV][8], x[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    Buf<TDY>::unpack(rdy[0][k], dy[k]);
    Buf<TX>::unpack(rx[k], x[k]);
  }
#pragma unroll
  for (int i = 1; i < kMaxDy; ++i)
#pragma unroll
    for (int k = 0; k < NV; ++k) {
      float t[8];
      Buf<TDY>::unpack(rdy[i][k], t);
#pragma unroll
      for (int e = 0; e < 8; ++e) dy[k][e] += t[e];
    }
  float inv = rstd_saved;
  if (a.rstd == nullptr) {  // recomputed from x (from_y always has the saved rstd)
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k)
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(x[k][e], x[k][e], ss);
    inv = inv_rms(row_sum(ss, a.wpr, red), n, a.eps);
  }
  float p = 0.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float w8[8];
    bload<true, float, kCached>(rw, (tg + k * G) * 32, w8);
    const int col = 8 * (tg + k * G);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // xhat = x * rstd, or y times the hardware reciprocal of w (as the general kernel)
      x[k][e] = a.from_y ? x[k][e] * __builtin_amdgcn_rcpf(col + e < n ? w8[e] : 1.f)
                         : x[k][e] * inv;
      dy[k][e] *= w8[e];
      p = fmaf(dy[k][e], x[k][e], p);
    }
  }
  const float proj = row_sum(p, a.wpr, red) / (float)n;
  float dr[NV][8];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    float t[8];
    Buf<float>::unpack(ro[k], t);
#pragma unroll
    for (int e = 0; e < 8; ++e) dr[k][e] = inv * (dy[k][e] - x[k][e] * proj) + t[e];
  }
  if (a.dr != nullptr) {
    const Span so = row_rsrc<float>(a.dr, row, a.ld_out, n, ok);
#pragma unroll
    for (int k = 0; k < NV; ++k) bstore<true, float>(so, (tg + k * G) * 32, dr[k]);
  }
  if (a.dx != nullptr) {
    const Span so = row_rsrc<TO>(a.dx, row, a.ld_out, n, ok);
#pragma unroll
    for (int k = 0; k < NV; ++k) bstore<true, TO>(so, (tg + k * G) * 8 * sizeof(TO), dr[k]);
  }
}

// The general backward (every reference mode; vector or element-wise rows).
template <int NV, bool VEC, typename TX, typename TDY, typename TO>
__global__ __launch_bounds__(kBwdThreads) void k_rmsnorm_bwd(const BwdArgs a) {
  __shared__ float red[kBwdThreads / kWave];
  extern __shared__ float lds[];
  bwd_rows<NV, VEC, TX, TDY, TO>(a, red, lds);
}

// Stage 2 of the weight gradient: dw[j] = sum_p part[p, j]. A block of 256 threads owns
// kRedCols columns: thread (stripe r = tid / (kRedCols / 4), quad c = tid % (kRedCols / 4)) adds
// the 4 columns 4c..4c+3 of the block's span over rows p = r, r + kRedStripes, r + 2 kRedStripes,
// ... in ascending p, then a fixed tree of log2(kRedStripes) levels adds the kRedStripes stripe
// sums (stripe r + h into stripe r). n % 4 != 0 takes the same order one column at a time.
// Block shape kRedCols x kRedStripes, measured at config 4 (per call with its reduce / batched
// over 57 norms, us per norm): 8 x 128 19.9 / 17.1, 16 x 64 18.9 / 16.7, 32 x 32 18.8 / 16.4,
// 64 x 16 19.4 / 16.4.
constexpr int kRedCols = 32;
constexpr int kRedStripes = 1024 / kRedCols;

// Stage 2 for columns [blockIdx.x * kRedCols, + kRedCols) of one [P, n] partials array:
// kRedStripes stripes of rows summed per thread, then the fixed tree over the stripes. Shared
// by the single-norm and the batched kernel, so both give the same bits for the same partials.
// The partials are read as 16-byte vectors when n % 4 == 0 (the entry points require 16-byte
// aligned partials).
template <typename TW>
__device__ __forceinline__ void dgamma_reduce_cols(const float* __restrict__ part, int64_t P,
                                                   int n, TW* __restrict__ dw) {
  __shared__ f32x4 red[kRedStripes][kRedCols / 4];
  const int c = threadIdx.x % (kRedCols / 4);
  const int r = threadIdx.x / (kRedCols / 4);
  const int j = blockIdx.x * kRedCols + 4 * c;
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  if ((n & 3) == 0) {
    if (j < n) {
#pragma unroll 4
      for (int64_t p = r; p < P; p += kRedStripes)
        s += *reinterpret_cast<const f32x4*>(part + p * n + j);
    }
  } else {
    for (int64_t p = r; p < P; p += kRedStripes) {
      const float* row = part + p * n;
      if (j < n) s.x += row[j];
      if (j + 1 < n) s.y += row[j + 1];
      if (j + 2 < n) s.z += row[j + 2];
      if (j + 3 < n) s.w += row[j + 3];
    }
  }
  red[r][c] = s;
  __syncthreads();
#pragma unroll
  for (int h = kRedStripes / 2; h >= 1; h >>= 1) {
    if (r < h) red[r][c] += red[r + h][c];
    __syncthreads();
  }
  if (r == 0) {
    const f32x4 t = red[0][c];
    const float v[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (j + e < n) dw[j + e] = Elt<TW>::from_f(v[e]);
  }
}

template <typename TW>
__global__ __launch_bounds__(256) void k_dgamma_reduce(const float* __restrict__ part,
                                                          int64_t P, int n, TW* __restrict__ dw) {
  dgamma_reduce_cols<TW>(part, P, n, dw);
}

// Several norms' stage 2 in one launch: blockIdx.y selects the item.
constexpr int kDgammaBatchMax = 64;
struct DgammaBatch {
  const float* part[kDgammaBatchMax];
  int64_t P[kDgammaBatchMax];
  void* dw[kDgammaBatchMax];
};
template <typename TW>
__global__ __launch_bounds__(256) void k_dgamma_reduce_batch(const DgammaBatch b, int n) {
  const int i = blockIdx.y;
  dgamma_reduce_cols<TW>(b.part[i], b.P[i], n, static_cast<TW*>(b.dw[i]));
}

// Launch helpers implemented in the instantiating translation units.
hipError_t launch_rmsnorm_fwd(const FwdArgs& a, int x_dt, int d_dt, int y_dt, int nv, dim3 grid,
                              dim3 block, hipStream_t s, bool* supported);
hipError_t launch_rmsnorm_bwd(const BwdArgs& a, int x_dt, int dy_dt, int o_dt, int nv, dim3 grid,
                              dim3 block, size_t lds_bytes, hipStream_t s, bool* supported);
hipError_t launch_dgamma_reduce(const float* part, int64_t P, int n, void* dw, int dw_dt,
                                hipStream_t s, bool* supported);
hipError_t launch_dgamma_reduce_batch(const DgammaBatch& b, int count, int n, int dw_dt,
                                      hipStream_t s, bool* supported);

}  // namespace esep

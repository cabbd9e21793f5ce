// Row statistics and dlogits of the fused LM head, for gfx950. Restates the reference's row
// kernel (solution/head/kernels.py:38-93, head_row_softmax_kernel): for one row z of a logits
// chunk ([rows, V], fp16 / bf16, row stride ld),
//   pass 1 (reads the row once): online max M, S = sum exp(z - M), T = sum exp(z - M) (z - M)
//          and the first index of the maximum;
//          lse = M + log S, entropy = log S - T / S (no difference of two large numbers);
//   pass 2 (write_g, and only on rows whose CE weight is != 0): the row is overwritten in place
//          with g = (softmax(z) - onehot(target)) * g_scale, rounded to the row's dtype.
// A row whose target lies outside [0, V) gets target logit 0 and no onehot term.
//
// Mapping: one block of kHeadThreads threads per row. The row is cut into 16-byte chunks of 8
// elements; thread t owns chunks t, t + kHeadThreads, ... and loads kBatch of them per step
// before using any (kBatch x 16 bytes in flight per lane). Per step the thread takes the batch
// maximum, rescales its running sums once, and adds 2^d and 2^d d per element with
// d = (z - M) log2(e) (one fma, one v_exp_f32): exponentials are base 2, so T is kept in base-2
// units and converted once at the end. The argmax costs nothing per element: a thread records
// only the step in which its running maximum last grew; after the block has merged M, the
// threads whose maximum equals M re-read that one step's chunks and the first matching index
// is taken with an LDS min. The partial (M, S, T) states are merged by a fixed tree (lane
// exchanges within the wavefront, then the wavefronts in order), so the statistics do not
// depend on timing. Pass 2 evaluates p = 2^((z - M) log2(e) - log2 S): z - M is exact and
// log2 S is small where p is near 1, so p - 1 keeps its accuracy for confident rows.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"
#include "head.hpp"

namespace esep {
namespace {

constexpr int kHeadThreads = 1024;
constexpr int kHeadWaves = kHeadThreads / kWave;
constexpr int kBatch = 4;            // chunks of 8 elements per thread per step
constexpr float kNegBig = -1.0e30f;  // finite "minus infinity": 0 * (m_old - m_new) stays 0
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.69314718055994531f;

// 2^x on the hardware's v_exp_f32 (results below 2^-126 may flush to 0; they vanish next to
// S >= 1 and below every output's resolution).
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

struct RowState {
  float m;  // running maximum (logit units)
  float s;  // sum 2^d over the elements, d = (z - m) log2(e)
  float t;  // sum 2^d d (base-2 units)
};

// State of the union of two element sets.
__device__ __forceinline__ RowState merge(const RowState& a, const RowState& b) {
  const float M = fmaxf(a.m, b.m);
  const float da = (a.m - M) * kLog2e, db = (b.m - M) * kLog2e;
  const float ea = exp2f(da), eb = exp2f(db);
  RowState r;
  r.m = M;
  r.s = ea * a.s + eb * b.s;
  r.t = ea * fmaf(a.s, da, a.t) + eb * fmaf(b.s, db, b.t);
  return r;
}

// The kBatch chunks of step c0: whole 16-byte loads when the step is full for the whole
// wavefront (FULL), else chunk- and element-wise masking; masked elements read kNegBig.
template <typename T, bool VEC>
__device__ __forceinline__ void load_step(const Span& sp, int c0, int nch, int V, bool full,
                                          float (&zv)[kBatch][8]) {
  if (VEC && full) {
    Raw<T> r[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
      r[b] = Buf<T>::template load_raw<kCached>(sp, (uint32_t)(c0 + b * kHeadThreads) * 16u);
#pragma unroll
    for (int b = 0; b < kBatch; ++b) Buf<T>::unpack(r[b], zv[b]);
  } else {
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int c = c0 + b * kHeadThreads;
      if (c < nch) Buf<T>::template load<VEC>(sp, (uint32_t)c * 16u, zv[b]);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (c >= nch || (!VEC && 8 * c + e >= V)) zv[b][e] = kNegBig;
    }
  }
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kHeadThreads) void k_head_row(const HeadArgs a) {
  __shared__ RowState red[kHeadWaves];
  __shared__ float m_sh, log2s_sh;
  __shared__ int amin_sh;
  const int64_t row = blockIdx.x;
  const int V = (int)a.V;
  const int nch = (V + 7) >> 3;
  const T* zrow = static_cast<const T*>(a.z) + row * a.ld;
  const Span sp = make_span(zrow, (uint32_t)(V * (int)sizeof(T)));
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  constexpr int kStep = kBatch * kHeadThreads;
  if (tid == 0) amin_sh = 0x7fffffff;

  // ---- pass 1 ----
  RowState st{kNegBig, 0.f, 0.f};
  int arg_step = -1;  // step (first chunk c0) in which the running maximum last grew
  for (int c0 = tid; c0 < nch; c0 += kStep) {
    // wave-uniform: every chunk of this step lies inside the row for all 64 lanes
    const bool full = c0 - lane + (kWave - 1) + (kBatch - 1) * kHeadThreads < nch;
    float zv[kBatch][8];
    load_step<T, VEC>(sp, c0, nch, V, full, zv);
    float bm = zv[0][0];
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
#pragma unroll
      for (int e = 0; e < 8; ++e) bm = fmaxf(bm, zv[b][e]);
    if (bm > st.m) arg_step = c0;
    const float mn = fmaxf(st.m, bm);
    const float nm2 = -mn * kLog2e;
    float se = 0.f, sd = 0.f;
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // masked elements: d ~ -1.4e30, 2^d = 0 and 0 * d = 0 (mn is a real logit: chunk c0
        // always holds at least one element of the row)
        const float d = fmaf(zv[b][e], kLog2e, nm2);
        const float ex = exp2_fast(d);
        se += ex;
        sd = fmaf(ex, d, sd);
      }
    const float dm = (st.m - mn) * kLog2e;
    const float sc = exp2_fast(dm);
    st.t = fmaf(sc, fmaf(st.s, dm, st.t), sd);
    st.s = fmaf(sc, st.s, se);
    st.m = mn;
  }

  // ---- merge: wavefront tree, then the wavefronts in order ----
  const float my_m = st.m;  // the thread's own maximum, for the argmax
#pragma unroll
  for (int h = kWave / 2; h >= 1; h >>= 1) {
    RowState o;
    o.m = __shfl_down(st.m, h);
    o.s = __shfl_down(st.s, h);
    o.t = __shfl_down(st.t, h);
    if (lane < h) st = merge(st, o);
  }
  if (lane == 0) red[tid / kWave] = st;
  __syncthreads();
  if (tid == 0) {
    RowState r = red[0];
    for (int w = 1; w < kHeadWaves; ++w) r = merge(r, red[w]);
    const float log2s = log2f(r.s);
    a.lse[row] = fmaf(log2s, kLn2, r.m);
    a.ent[row] = (log2s - r.t / r.s) * kLn2;
    const int64_t tg = a.target[row];
    a.tlogit[row] = (tg >= 0 && tg < a.V) ? Elt<T>::to_f(zrow[tg]) : 0.f;
    m_sh = r.m;
    log2s_sh = log2s;
  }
  __syncthreads();
  const float M = m_sh;

  // ---- argmax: a thread whose maximum is M re-reads the step where it was reached (its
  // first occurrence among the thread's elements) and offers the first index holding M ----
  if (arg_step >= 0 && my_m == M) {
    float zv[kBatch][8];
    load_step<T, VEC>(sp, arg_step, nch, V, false, zv);
    int best = 0x7fffffff;
#pragma unroll
    for (int b = kBatch - 1; b >= 0; --b)
#pragma unroll
      for (int e = 7; e >= 0; --e)
        if (zv[b][e] == M) best = 8 * (arg_step + b * kHeadThreads) + e;
    atomicMin(&amin_sh, best);
  }
  __syncthreads();
  if (tid == 0) a.amax[row] = amin_sh;
  if (!a.write_g || a.cew[row] == 0.f) return;  // uniform over the block

  // ---- pass 2: g = (softmax - onehot) * g_scale, in place ----
  const float l2s = log2s_sh;
  const float gs = a.g_scale;
  const int64_t tg = a.target[row];
  const int tch = (tg >= 0 && tg < a.V) ? (int)(tg >> 3) : -1;
  for (int c0 = tid; c0 < nch; c0 += kStep) {
    const bool full = c0 - lane + (kWave - 1) + (kBatch - 1) * kHeadThreads < nch;
    float zv[kBatch][8];
    load_step<T, VEC>(sp, c0, nch, V, full, zv);
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int c = c0 + b * kHeadThreads;
      float gv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) gv[e] = exp2_fast(fmaf(zv[b][e] - M, kLog2e, -l2s)) * gs;
      if (c == tch) {  // the target element (one lane of the row): (p - 1) * g_scale
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (e == (int)(tg & 7)) gv[e] = (exp2_fast(fmaf(zv[b][e] - M, kLog2e, -l2s)) - 1.f) * gs;
      }
      if (c < nch) Buf<T>::template store<VEC, kStream>(sp, (uint32_t)c * 16u, gv);
    }
  }
}

template <typename T>
void launch_t(const HeadArgs& a, bool vec, hipStream_t s) {
  const dim3 grid((unsigned)a.rows), block(kHeadThreads);
  if (vec)
    hipLaunchKernelGGL((k_head_row<T, true>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((k_head_row<T, false>), grid, block, 0, s, a);
}

}  // namespace

hipError_t launch_head_row(const HeadArgs& a, int dt, bool vec, hipStream_t s, bool* supported) {
  *supported = true;
  if (a.rows == 0) return hipSuccess;
  if (dt == 1)
    launch_t<_Float16>(a, vec, s);
  else if (dt == 2)
    launch_t<__bf16>(a, vec, s);
  else {
    *supported = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esep

// Varlen causal attention forward (see attention.hpp for the layout and the MFMA mapping).
#include <cmath>
#include <type_traits>

#include "attention.hpp"

namespace esep {
namespace {

// One 32-key half of the online softmax for a wavefront's 32 queries: keys kh .. kh + 31, held
// in rows r0 .. r0 + 31 of the row-major LDS tiles ks / vs (pitch KP). Lane (lq, hi) gets the
// scores of its query qi against keys kh + 8 (i / 4) + 4 hi + i % 4, i < 16, from
// S^T = K Q^T (K rows from LDS as the A operand, the wave's Q^T in registers as B), then
// updates (m, l) and O^T += V^T P^T.
template <typename T, int D, int KP>
__device__ __forceinline__ void fwd_half(const T* ks, const T* vs, int r0, int kh, int qw0, int qi,
                                         int lane, float scale_log2,
                                         const typename Mfma<T>::v8 (&qb)[D / 16],
                                         f32x16 (&oacc)[D / 32], float& m, float& l) {
  using V8 = typename Mfma<T>::v8;
  const int lq = lane & 31, hi = lane >> 5;
  f32x16 acc = f32x16{};
  const T* krow = &ks[(r0 + lq) * KP + 8 * hi];
  // K operands read three ahead of the MFMA that uses them; the scheduling barriers keep the
  // compiler from sinking each read to just before its use (two ahead), which left an LDS
  // round trip exposed per pair of MFMAs (config 5 forward 2.03 -> 1.98 ms)
  constexpr int KA = 3;
  V8 kbuf[KA];
#pragma unroll
  for (int c = 0; c < KA; ++c) kbuf[c] = ld16<V8>(krow + 16 * c);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    acc = Mfma<T>::run(kbuf[c % KA], qb[c], acc);
    if (c + KA < D / 16) kbuf[c % KA] = ld16<V8>(krow + 16 * (c + KA));
    __builtin_amdgcn_sched_barrier(0);
  }
  // the first two V^T operands (PV order j = 2 md + c2) read before the softmax, whose VALU
  // work hides their LDS latency (1.98 -> 1.93 ms)
  constexpr int VA = 2;
  V8 vbuf[VA];
#pragma unroll
  for (int j = 0; j < VA; ++j) vbuf[j] = ld_tr<V8, KP>(vs, r0 + 16 * (j % 2), 32 * (j / 2), lane);
  __builtin_amdgcn_sched_barrier(0);
  // the causal mask only bites on the half-tiles that reach past the wave's first query
  if (kh + 31 > qw0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kj = kh + 8 * (i / 4) + 4 * hi + (i % 4);
      if (kj > qi) acc[i] = -INFINITY;
    }
  }
  float mx = acc[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) mx = fmaxf(mx, acc[i]);
  mx = pair_max(mx) * scale_log2;
  // Online softmax (base 2) with a lazy reference: the lane's m moves only when the half's
  // maximum exceeds it by more than 8, so p <= 2^8 (exact in bf16 / fp16 relative terms) and
  // O, l are rescaled only in the rare half-tiles where some lane's m moved.
  const bool grow = mx > m + 8.f;
  float alpha = 1.f;
  if (grow) {
    alpha = exp2_fast(m - mx);  // m = -inf on the first half: alpha = 0, O and l are 0
    m = mx;
  }
  const float nm = m == -INFINITY ? 0.f : -m;  // a lane with no visible key yet: p = 0
  float ps = 0.f;
  V8 pb[2];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float p = exp2_fast(fmaf(acc[i], scale_log2, nm));
    ps += p;
    pb[i / 8][i % 8] = (T)p;
  }
  ps = pair_sum(ps);
  l = fmaf(l, alpha, ps);
  if (__any(grow)) {
#pragma unroll
    for (int md = 0; md < D / 32; ++md) oacc[md] *= alpha;
  }
  // O^T += V^T P^T over the 32 keys, contraction in the permuted key order of pb (element e of
  // chunk c2 is key kh + 16 c2 + 8 (e / 4) + 4 hi + e % 4); V^T read transposed out of the
  // row-major V tile, two operands ahead of the MFMAs
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 2 * (D / 32); ++j) {
    oacc[j / 2] = Mfma<T>::run(vbuf[j % VA], pb[j % 2], oacc[j / 2]);
    if (j + VA < 2 * (D / 32))
      vbuf[j % VA] = ld_tr<V8, KP>(vs, r0 + 16 * ((j + VA) % 2), 32 * ((j + VA) / 2), lane);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The D = 64 forward: K / V staged through registers in 64-key tiles (rows of 128 bytes).
template <typename T, int D>
// 3 wavefronts per SIMD (<= 168 registers): without the bound the compiler parks the
// accumulators in AGPRs and stops at 2.
__global__ __launch_bounds__(kAttnThreads, 3) void k_attn_fwd(const AttnArgs a) {
  using V8 = typename Mfma<T>::v8;
  constexpr int BN = kAttnBN;
  constexpr int KP = D + kRowPad;  // row pitch of the K and V tiles in LDS (elements)
  __shared__ __align__(16) T ks[BN * KP];
  __shared__ __align__(16) T vs[BN * KP];

  const int seq = blockIdx.z, h = blockIdx.y;
  int start, end;  // clamped into [0, T]: malformed offsets stay in bounds
  seq_bounds(a.cu, seq, a.T, &start, &end);
  const int ntiles = (end - start + kAttnBM - 1) / kAttnBM;
  if ((int)blockIdx.x >= ntiles) return;
  const int q0 = start + (ntiles - 1 - (int)blockIdx.x) * kAttnBM;  // heaviest tiles first
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lq = lane & 31, hi = lane >> 5;
  const int kvh = h / (a.HQ / a.HK);
  const int qw0 = q0 + 32 * w;                  // this wavefront's first query
  const int qi = qw0 + lq;                      // this lane's query
  const bool wave_live = qw0 < end;
  const int wq_last = qw0 + 31 < end ? qw0 + 31 : end - 1;

  // Q^T as the B operand: lane (lq, hi) holds Q[qi][16c + 8hi .. 16c + 8hi + 7] for chunk c.
  V8 qb[D / 16];
  {
    const T* qrow = static_cast<const T*>(a.q) + (int64_t)qi * a.q_rs + (int64_t)h * D + 8 * hi;
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
      qb[c] = qi < end ? ld16<V8>(qrow + 16 * c) : V8{};
  }

  f32x16 oacc[D / 32];
#pragma unroll
  for (int md = 0; md < D / 32; ++md) oacc[md] = f32x16{};
  float m = -INFINITY, l = 0.f;
  const int kend = end < q0 + kAttnBM ? end : q0 + kAttnBM;
  const T* kbase = static_cast<const T*>(a.k) + (int64_t)kvh * D;
  const T* vbase = static_cast<const T*>(a.v) + (int64_t)kvh * D;

  for (int kt = start; kt < kend; kt += BN) {
    // K and V of the tile, row-major: every global read is issued before the barrier, one
    // memory round trip per tile; keys past kend read 0. (Reading the next tile during the
    // current one needs 32 more registers: 2 wavefronts per SIMD instead of 3, measured 15%
    // slower.)
    TileRows<T, D, BN> kr, vr;
    kr.load(kbase, a.k_rs, kt, kend, tid);
    vr.load(vbase, a.v_rs, kt, kend, tid);
    __syncthreads();  // the previous tile's LDS reads are done
    kr.template store<KP>(ks, tid);
    vr.template store<KP>(vs, tid);
    __syncthreads();
    if (!wave_live || kt > wq_last) continue;  // every key of the tile is after this wave's queries

    // One 32-key half at a time: keeping both halves' scores live needs ~250 registers,
    // 2 wavefronts per SIMD; one half at a time fits 3, which measured a third faster.
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
      fwd_half<T, D, KP>(ks, vs, 32 * sb, kt + 32 * sb, qw0, qi, lane, a.scale_log2, qb, oacc, m, l);
  }

  if (!wave_live || qi >= end) return;
  // O = O^T / l: lane (lq, hi) holds columns d = 32 md + 8 j + 4 hi + (0..3) of query qi.
  store_rows_t<T, D>(static_cast<T*>(a.o) + (int64_t)qi * a.o_rs + (int64_t)h * D, oacc, hi,
                     l > 0.f ? 1.f / l : 0.f);
  if (hi == 0 && a.lse != nullptr)
    a.lse[(int64_t)h * a.T + qi] = (m + log2f(l)) * 0.69314718055994531f;
}

// D = 128 forward on swizzled, unpadded LDS tiles (the layout, its DMA and its readers are in
// attention.hpp: swz, SwzFill, swz_row_base, SwzTr).
//
// One 32-key half (the whole 32-key tile) of the online softmax, as fwd_half, on swizzled tiles:
// the K operand of chunk pair c is read at byte (256 lq + 16 ((2c + hi) ^ f(lq))) of the K tile,
// the V^T operands of ld_tr's lane mapping at their rows' swizzled chunk positions.
template <typename T>
__device__ __forceinline__ void fwd_tile_swz(const char* ks, const char* vs, int kh, int qw0,
                                             int qi, int lane, float scale_log2,
                                             const typename Mfma<T>::v8 (&qb)[8],
                                             f32x16 (&oacc)[4], float& m, float& l) {
  using V8 = typename Mfma<T>::v8;
  const int lq = lane & 31, hi = lane >> 5;
  // The MFMA runs go at raised wave priority, the softmax between them at the normal one: with
  // several wavefronts per SIMD the arbiter then feeds the matrix core from a wavefront in its
  // MFMA run ahead of another's vector work (all three kernels; config 5: forward 1.44 -> 1.43
  // ms, backward 5.00 -> 4.91 ms).
  __builtin_amdgcn_s_setprio(1);
  f32x16 acc = f32x16{};
  const uint32_t k0 = swz_row_base(lane);
  constexpr int KA = 3;
  V8 kbuf[KA];
#pragma unroll
  for (int c = 0; c < KA; ++c) kbuf[c] = ld16<V8>(ks + (k0 ^ (32u * c)));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    acc = Mfma<T>::run(kbuf[c % KA], qb[c], acc);
    if (c + KA < 8) kbuf[c % KA] = ld16<V8>(ks + (k0 ^ (32u * (c + KA))));
    __builtin_amdgcn_sched_barrier(0);
  }
  // V^T operand j: rows 16 (j & 1) .., columns 32 (j >> 1) .. of the V tile
  const SwzTr vt(lane);
  auto ldv = [&](int j) { return vt.template read<V8>(vs, 16 * (j & 1), j >> 1); };
  constexpr int VA = 2;
  V8 vbuf[VA];
#pragma unroll
  for (int j = 0; j < VA; ++j) vbuf[j] = ldv(j);
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(0);
  if (kh + 31 > qw0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kj = kh + 8 * (i / 4) + 4 * hi + (i % 4);
      if (kj > qi) acc[i] = -INFINITY;
    }
  }
  float mx = acc[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) mx = fmaxf(mx, acc[i]);
  mx = pair_max(mx) * scale_log2;
  const bool grow = mx > m + 8.f;
  float alpha = 1.f;
  if (grow) {
    alpha = exp2_fast(m - mx);
    m = mx;
  }
  const float nm = m == -INFINITY ? 0.f : -m;
  float ps = 0.f;
  V8 pb[2];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float p = exp2_fast(fmaf(acc[i], scale_log2, nm));
    ps += p;
    pb[i / 8][i % 8] = (T)p;
  }
  ps = pair_sum(ps);
  l = fmaf(l, alpha, ps);
  if (__any(grow)) {
#pragma unroll
    for (int md = 0; md < 4; ++md) oacc[md] *= alpha;
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    oacc[j / 2] = Mfma<T>::run(vbuf[j % VA], pb[j % 2], oacc[j / 2]);
    if (j + VA < 8) vbuf[j % VA] = ldv(j + VA);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_setprio(0);
}

// The D = 128 forward kernel: blocks of 4 wavefronts own 128 queries of one (sequence, query
// head) with the online softmax in registers; the 32-key K / V tiles go through a ring of NBUF
// = 2 swizzled LDS buffers filled by LDS DMA (tile t + 1 in flight while tile t is consumed,
// one barrier per tile publishing it and freeing the buffer consumed before).
template <typename T, int NBUF>
__global__ __launch_bounds__(kAttnThreads, 3) void k_attn_fwd_swz(const AttnArgs a, int qtiles,
                                                                  int order) {
  constexpr int D = 128;
  constexpr int BN = 32;
  constexpr int TILE = BN * 256;  // bytes of one K or V tile
  using V8 = typename Mfma<T>::v8;
  __shared__ __align__(1024) char kv[NBUF][2][TILE];  // [buffer][K, V][swizzled rows]

  // XCD-aware order (xcd_order): the query tiles of one (sequence, head) run on one XCD.
  const int lin = block_order((int)blockIdx.x, qtiles, a.HQ * a.n_seq, order, a.HQ, a.cu, a.n_seq,
                              a.T);
  const int bx = lin % qtiles, rest = lin / qtiles;
  const int h = rest % a.HQ, seq = rest / a.HQ;
  if (seq >= a.n_seq) return;
  int start, end;
  seq_bounds(a.cu, seq, a.T, &start, &end);
  const int ntiles_q = (end - start + kAttnBM - 1) / kAttnBM;
  if (bx >= ntiles_q) return;
  const int q0 = start + (ntiles_q - 1 - bx) * kAttnBM;  // heaviest tiles first
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, hi = lane >> 5;
  const int kvh = h / (a.HQ / a.HK);
  const int qw0 = q0 + 32 * w;
  const int qi = qw0 + lq;
  const bool wave_live = qw0 < end;
  const int wq_last = qw0 + 31 < end ? qw0 + 31 : end - 1;

  V8 qb[D / 16];
  {
    const T* qrow = static_cast<const T*>(a.q) + (int64_t)qi * a.q_rs + (int64_t)h * D + 8 * hi;
#pragma unroll
    for (int c = 0; c < D / 16; ++c)
      qb[c] = qi < end ? ld16<V8>(qrow + 16 * c) : V8{};
  }

  f32x16 oacc[D / 32];
#pragma unroll
  for (int md = 0; md < D / 32; ++md) oacc[md] = f32x16{};
  float m = -INFINITY, l = 0.f;
  const int kend = end < q0 + kAttnBM ? end : q0 + kAttnBM;
  const char* kbase = reinterpret_cast<const char*>(static_cast<const T*>(a.k) + (int64_t)kvh * D);
  const char* vbase = reinterpret_cast<const char*>(static_cast<const T*>(a.v) + (int64_t)kvh * D);
  const int64_t krs = a.k_rs * (int64_t)sizeof(T), vrs = a.v_rs * (int64_t)sizeof(T);  // bytes
  const int ntiles = (kend - start + BN - 1) / BN;

  // Wavefront w fills row groups w and w + 4 of the K and V tiles (rows past kend repeat row
  // kend - 1: finite data, always masked). Tiles are issued in order, so whole ones step the
  // fillers' running addresses.
  SwzFill<BN, 4> fk(lane, w, krs), fv(lane, w, vrs);
  fk.seq_begin(kbase, start);
  fv.seq_begin(vbase, start);
  auto issue = [&](int buf, int kt) {
    if (kt + BN <= kend) {
      fk.seq_whole(kv[buf][0]);
      fv.seq_whole(kv[buf][1]);
    } else {
      swz_fill2(fk, kv[buf][0], kbase, fv, kv[buf][1], vbase, kt, kend);
    }
  };

  static_assert(NBUF == 2, "the tile loop is unrolled by the ring's two buffers");
  if (ntiles > 0) issue(0, start);
  // Tile t sits in buffer B = t % 2, and the loop is unrolled by two so that B is a constant:
  // the tiles' LDS addresses then fold into the reads' immediate offsets instead of costing a
  // VALU add per read (config-5-like forward 1.39 -> 1.34 ms, the same bits).
  auto tile = [&](int t, auto bc) {
    constexpr int B = decltype(bc)::value;
    // this wavefront's DMA of tile t has landed; the barrier publishes every wavefront's rows
    // and certifies that tile t - 1 is consumed, freeing its buffer for tile t + 1
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (t + 1 < ntiles) issue(B ^ 1, start + (t + 1) * BN);
    const int kt = start + t * BN;
    if (!wave_live || kt > wq_last) return;
    fwd_tile_swz<T>(kv[B][0], kv[B][1], kt, qw0, qi, lane, a.scale_log2, qb, oacc, m, l);
  };
  int t = 0;
  for (; t + 1 < ntiles; t += 2) {
    tile(t, std::integral_constant<int, 0>{});
    tile(t + 1, std::integral_constant<int, 1>{});
  }
  if (t < ntiles) tile(t, std::integral_constant<int, 0>{});

  if (!wave_live || qi >= end) return;
  store_rows_t<T, D>(static_cast<T*>(a.o) + (int64_t)qi * a.o_rs + (int64_t)h * D, oacc, hi,
                     l > 0.f ? 1.f / l : 0.f);
  if (hi == 0 && a.lse != nullptr)
    a.lse[(int64_t)h * a.T + qi] = (m + log2f(l)) * 0.69314718055994531f;
}

template <typename T>
hipError_t fwd_d(const AttnArgs& a, int D, dim3 grid, hipStream_t s, bool* sup) {
  *sup = true;
  if (D == 128) {
    const int64_t n = xcd_grid(grid.x, (int64_t)grid.y * grid.z);
    if (n > 0x7fffffff) return hipErrorInvalidValue;
    // 3 blocks resident per CU (launch bound)
    hipLaunchKernelGGL((k_attn_fwd_swz<T, 2>), dim3((unsigned)n), dim3(kAttnThreads), 0, s, a,
                       (int)grid.x, attn_order(n, 3, a.n_seq));
  }
  else if (D == 64)
    hipLaunchKernelGGL((k_attn_fwd<T, 64>), grid, dim3(kAttnThreads), 0, s, a);
  else {
    *sup = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_attn_fwd(const AttnArgs& a, int dt, int D, int max_seqlen, hipStream_t s,
                           bool* sup) {
  const dim3 grid((max_seqlen + kAttnBM - 1) / kAttnBM, a.HQ, a.n_seq);
  if (dt == 1) return fwd_d<_Float16>(a, D, grid, s, sup);
  if (dt == 2) return fwd_d<__bf16>(a, D, grid, s, sup);
  *sup = false;
  return hipErrorInvalidValue;
}

}  // namespace esep

// Varlen causal attention backward: two deterministic kernels, no atomics.
//
//   P = exp(scale q.k - lse)  (recomputed from the saved lse),   dP = dO V^T,
//   delta = rowsum(dO * O),   dS = P * (dP - delta),
//   dQ = scale dS K,   dK = scale dS^T Q,   dV = P^T dO
//
// k_attn_bwd_dq: one block per (128 queries, query head) as in the forward. It first computes
// delta for its queries (stored to the delta workspace), then walks the causal key tiles:
// S^T = K Q^T and dP^T = V dO^T with the wave's Q and dO held in registers as B operands, and
// dQ^T += K^T dS^T with K^T read transposed (ds_read_b64_tr_b16) out of the row-major K tile and
// dS^T fed from registers in the permuted key order (the forward's P V trick).
//
// k_attn_bwd_dkdv: one block per (128 keys; kv head; part of the kv
// head's query heads); wavefront w owns keys 32w..32w+31 and holds their K in registers as B
// operands (V's come from the block's V rows in LDS). It
// walks, for each of its query heads in turn and each query tile at or after its keys (at
// D = 128 the next tile's Q / dO / lse / delta moved by LDS DMA into the other buffer of a
// two-buffer ring during the current one; at D = 64 prefetched into registers), S = Q K^T and
// dP = dO V^T (Q and dO row-major in LDS as A operands), then dV^T += dO^T P and dK^T += Q^T dS (Q^T and dO^T
// read transposed out of the same tiles, P and dS from registers in the permuted query order). Each key's dK and
// dV are summed by one lane in a fixed order over heads and query tiles; with the heads split
// over several blocks (short inputs, to fill the GPU), each part writes fp32 partials and
// k_attn_dkdv_reduce adds them in part order, so the result is bitwise reproducible. Runs after
// k_attn_bwd_dq (it reads delta).
#include <cmath>
#include <type_traits>

#include "attention.hpp"

namespace esep {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

// One 32-key half of the dQ walk for a wavefront's 32 queries: keys kh .. kh + 31, held in rows
// r0 .. r0 + 31 of the row-major LDS tiles ks / vs (pitch KP). S^T = K Q^T and dP^T = V dO^T
// with the wave's Q and dO as B operands, dS^T = P^T * (dP^T - delta), then
// dQ^T += K^T dS^T with K^T read transposed out of ks and dS^T in the permuted key order.
template <typename T, int D, int KP>
__device__ __forceinline__ void dq_half(const T* ks, const T* vs, int r0, int kh, int qw0, int qi,
                                        int lane, float scale_log2, float lse2, float delta,
                                        const typename Mfma<T>::v8 (&qb)[D / 16],
                                        const typename Mfma<T>::v8 (&db)[D / 16],
                                        f32x16 (&dqa)[D / 32]) {
  using V8 = typename Mfma<T>::v8;
  const int lq = lane & 31, hi = lane >> 5;
  f32x16 s = f32x16{}, dp = f32x16{};
  const T* krow = &ks[(r0 + lq) * KP + 8 * hi];
  const T* vrow = &vs[(r0 + lq) * KP + 8 * hi];
  // K and V operands read three ahead of the MFMAs (the scheduling barriers keep the
  // compiler from sinking each read to just before its use; config 5 bwd 7.11 -> 6.97 ms
  // together with the K^T operands below)
  constexpr int KA = 3;
  V8 kbuf[KA], vbuf[KA];
#pragma unroll
  for (int c = 0; c < KA; ++c) {
    kbuf[c] = ld16<V8>(krow + 16 * c);
    vbuf[c] = ld16<V8>(vrow + 16 * c);
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    s = Mfma<T>::run(kbuf[c % KA], qb[c], s);
    dp = Mfma<T>::run(vbuf[c % KA], db[c], dp);
    if (c + KA < D / 16) {
      kbuf[c % KA] = ld16<V8>(krow + 16 * (c + KA));
      vbuf[c % KA] = ld16<V8>(vrow + 16 * (c + KA));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  // the first two K^T operands of dQ (order j = 2 md + c2) read before the exponentials
  constexpr int TA = 2;
  V8 tbuf[TA];
#pragma unroll
  for (int j = 0; j < TA; ++j) tbuf[j] = ld_tr<V8, KP>(ks, r0 + 16 * (j % 2), 32 * (j / 2), lane);
  __builtin_amdgcn_sched_barrier(0);
  // the causal mask only bites on the half-tiles that reach past the wave's first query
  if (kh + 31 > qw0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kj = kh + 8 * (i / 4) + 4 * hi + (i % 4);
      if (kj > qi) s[i] = -INFINITY;
    }
  }
  V8 dsb[2];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float p = exp2_fast(fmaf(s[i], scale_log2, -lse2));
    dsb[i / 8][i % 8] = (T)(p * (dp[i] - delta));
  }
  // dQ^T += K^T dS^T, keys in the permuted order of dsb, K^T read transposed out of ks
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 2 * (D / 32); ++j) {
    dqa[j / 2] = Mfma<T>::run(tbuf[j % TA], dsb[j % 2], dqa[j / 2]);
    if (j + TA < 2 * (D / 32))
      tbuf[j % TA] = ld_tr<V8, KP>(ks, r0 + 16 * ((j + TA) % 2), 32 * ((j + TA) / 2), lane);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// dq_half on swizzled 32-row tiles (attention.hpp: SwzFill, swz_row_base, SwzTr): the K and V
// row operands at (swz_row_base ^ 32 c), the K^T operands through SwzTr.
template <typename T>
__device__ __forceinline__ void dq_tile_swz(const char* ks, const char* vs, int kh, int qw0, int qi,
                                            int lane, float scale_log2, float lse2, float delta,
                                            const typename Mfma<T>::v8 (&qb)[8],
                                            const typename Mfma<T>::v8 (&db)[8],
                                            f32x16 (&dqa)[4]) {
  using V8 = typename Mfma<T>::v8;
  const int hi = lane >> 5;
  __builtin_amdgcn_s_setprio(1);  // MFMA runs at raised priority, as in the forward
  f32x16 s = f32x16{}, dp = f32x16{};
  const uint32_t r0 = swz_row_base(lane);
  constexpr int KA = 3;
  V8 kbuf[KA], vbuf[KA];
#pragma unroll
  for (int c = 0; c < KA; ++c) {
    kbuf[c] = ld16<V8>(ks + (r0 ^ (32u * c)));
    vbuf[c] = ld16<V8>(vs + (r0 ^ (32u * c)));
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < 8; ++c) {
    s = Mfma<T>::run(kbuf[c % KA], qb[c], s);
    dp = Mfma<T>::run(vbuf[c % KA], db[c], dp);
    if (c + KA < 8) {
      kbuf[c % KA] = ld16<V8>(ks + (r0 ^ (32u * (c + KA))));
      vbuf[c % KA] = ld16<V8>(vs + (r0 ^ (32u * (c + KA))));
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  const SwzTr kt(lane);
  constexpr int TA = 2;
  V8 tbuf[TA];
#pragma unroll
  for (int j = 0; j < TA; ++j) tbuf[j] = kt.template read<V8>(ks, 16 * (j & 1), j >> 1);
  __builtin_amdgcn_sched_barrier(0);
  if (kh + 31 > qw0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int kj = kh + 8 * (i / 4) + 4 * hi + (i % 4);
      if (kj > qi) s[i] = -INFINITY;
    }
  }
  __builtin_amdgcn_s_setprio(0);
  V8 dsb[2];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const float p = exp2_fast(fmaf(s[i], scale_log2, -lse2));
    dsb[i / 8][i % 8] = (T)(p * (dp[i] - delta));
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    dqa[j / 2] = Mfma<T>::run(tbuf[j % TA], dsb[j % 2], dqa[j / 2]);
    if (j + TA < 8) tbuf[j % TA] = kt.template read<V8>(ks, 16 * ((j + TA) & 1), (j + TA) >> 1);
    __builtin_amdgcn_sched_barrier(0);
  }
  __builtin_amdgcn_s_setprio(0);
}

// 2 wavefronts per SIMD without spills (unbounded, the compiler settles at 1).
template <typename T, int D, int NW>
__global__ __launch_bounds__(64 * NW, 2) void k_attn_bwd_dq(const AttnBwdArgs b) {
  using V8 = typename Mfma<T>::v8;
  const AttnArgs& a = b.f;
  constexpr int NT = 64 * NW, BM = 32 * NW;  // queries per block
  constexpr int BN = kAttnBN;
  constexpr int KP = D + kRowPad;
  __shared__ __align__(16) T ks[BN * KP];  // K row-major (A operand of S^T; read transposed for dQ^T)
  __shared__ __align__(16) T vs[BN * KP];  // V row-major (A operand of dP^T)

  const int seq = blockIdx.z, h = blockIdx.y;
  int start, end;
  seq_bounds(a.cu, seq, a.T, &start, &end);
  const int ntiles = (end - start + BM - 1) / BM;
  if ((int)blockIdx.x >= ntiles) return;
  const int q0 = start + (ntiles - 1 - (int)blockIdx.x) * BM;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lq = lane & 31, hi = lane >> 5;
  const int kvh = h / (a.HQ / a.HK);
  const int qw0 = q0 + 32 * w;
  const int qi = qw0 + lq;
  const bool qok = qi < end;
  const bool wave_live = qw0 < end;
  const int wq_last = qw0 + 31 < end ? qw0 + 31 : end - 1;

  // Q and dO of this lane's query as B operands; delta = dO . O (half per lane, then the pair)
  V8 qb[D / 16], db[D / 16];
  float delta = 0.f;
  {
    const int64_t col = (int64_t)h * D + 8 * hi;
    const T* qrow = static_cast<const T*>(a.q) + (int64_t)qi * a.q_rs + col;
    const T* drow = static_cast<const T*>(b.dout) + (int64_t)qi * b.do_rs + col;
    const T* orow = static_cast<const T*>(a.o) + (int64_t)qi * a.o_rs + col;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      qb[c] = qok ? ld16<V8>(qrow + 16 * c) : V8{};
      db[c] = qok ? ld16<V8>(drow + 16 * c) : V8{};
      const V8 o8 = qok ? ld16<V8>(orow + 16 * c) : V8{};
#pragma unroll
      for (int e = 0; e < 8; ++e) delta = fmaf((float)db[c][e], (float)o8[e], delta);
    }
    delta = pair_sum(delta);
    if (qok && hi == 0) b.delta[(int64_t)h * a.T + qi] = delta;
  }
  const float lse2 = qok ? a.lse[(int64_t)h * a.T + qi] * kLog2e : 0.f;

  f32x16 dqa[D / 32];
#pragma unroll
  for (int md = 0; md < D / 32; ++md) dqa[md] = f32x16{};
  const int kend = end < q0 + BM ? end : q0 + BM;
  const T* kbase = static_cast<const T*>(a.k) + (int64_t)kvh * D;
  const T* vbase = static_cast<const T*>(a.v) + (int64_t)kvh * D;

  // K and V of the next key tile are read into registers while the current tile is computed
  TileRows<T, D, BN, NT> kr, vr;
  if (start < kend) {
    kr.load(kbase, a.k_rs, start, kend, tid);
    vr.load(vbase, a.v_rs, start, kend, tid);
  }
  for (int kt = start; kt < kend; kt += BN) {
    __syncthreads();
    kr.template store<KP>(ks, tid);
    vr.template store<KP>(vs, tid);
    __syncthreads();
    if (kt + BN < kend) {
      kr.load(kbase, a.k_rs, kt + BN, kend, tid);
      vr.load(vbase, a.v_rs, kt + BN, kend, tid);
    }
    if (!wave_live || kt > wq_last) continue;

    // one 32-key half at a time (fewer live registers: 3 wavefronts per SIMD instead of 2)
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
      dq_half<T, D, KP>(ks, vs, 32 * sb, kt + 32 * sb, qw0, qi, lane, a.scale_log2, lse2, delta,
                        qb, db, dqa);
  }
  if (!qok) return;
  store_rows_t<T, D>(static_cast<T*>(b.dq) + (int64_t)qi * b.dq_rs + (int64_t)h * D, dqa, hi,
                     a.scale);
}

// dQ at D = 128 with the K / V tiles moved as the forward moves them: swizzled 32-key tiles
// filled by dwordx4 LDS DMA through a ring of two buffers (tile t + 1 in flight while tile t is
// consumed, one barrier per tile). Same prologue as k_attn_bwd_dq; dq_tile_swz is dq_half on
// the swizzled tiles.
template <typename T, int NW>
__global__ __launch_bounds__(64 * NW, 2) void k_attn_bwd_dq_dma(const AttnBwdArgs b, int qtiles,
                                                                 int order) {
  constexpr int D = 128;
  constexpr int BN = 32;
  using V8 = typename Mfma<T>::v8;
  const AttnArgs& a = b.f;
  constexpr int BM = 32 * NW;  // queries per block
  __shared__ __align__(1024) char kv[2][2][BN * 256];  // [buffer][K, V][swizzled tile]

  // XCD-aware order: the query tiles of one (sequence, head) run on one XCD
  const int lin = block_order((int)blockIdx.x, qtiles, a.HQ * a.n_seq, order, a.HQ, a.cu, a.n_seq,
                              a.T);
  const int bx = lin % qtiles, rest = lin / qtiles;
  const int h = rest % a.HQ, seq = rest / a.HQ;
  if (seq >= a.n_seq) return;
  int start, end;
  seq_bounds(a.cu, seq, a.T, &start, &end);
  const int ntiles_q = (end - start + BM - 1) / BM;
  if (bx >= ntiles_q) return;
  const int q0 = start + (ntiles_q - 1 - bx) * BM;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, hi = lane >> 5;
  const int kvh = h / (a.HQ / a.HK);
  const int qw0 = q0 + 32 * w;
  const int qi = qw0 + lq;
  const bool qok = qi < end;
  const bool wave_live = qw0 < end;
  const int wq_last = qw0 + 31 < end ? qw0 + 31 : end - 1;

  V8 qb[D / 16], db[D / 16];
  float delta = 0.f;
  {
    const int64_t col = (int64_t)h * D + 8 * hi;
    const T* qrow = static_cast<const T*>(a.q) + (int64_t)qi * a.q_rs + col;
    const T* drow = static_cast<const T*>(b.dout) + (int64_t)qi * b.do_rs + col;
    const T* orow = static_cast<const T*>(a.o) + (int64_t)qi * a.o_rs + col;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      qb[c] = qok ? ld16<V8>(qrow + 16 * c) : V8{};
      db[c] = qok ? ld16<V8>(drow + 16 * c) : V8{};
      const V8 o8 = qok ? ld16<V8>(orow + 16 * c) : V8{};
#pragma unroll
      for (int e = 0; e < 8; ++e) delta = fmaf((float)db[c][e], (float)o8[e], delta);
    }
    delta = pair_sum(delta);
    if (qok && hi == 0) b.delta[(int64_t)h * a.T + qi] = delta;
  }
  const float lse2 = qok ? a.lse[(int64_t)h * a.T + qi] * kLog2e : 0.f;

  f32x16 dqa[D / 32];
#pragma unroll
  for (int md = 0; md < D / 32; ++md) dqa[md] = f32x16{};
  const int kend = end < q0 + BM ? end : q0 + BM;
  const char* kbase = reinterpret_cast<const char*>(static_cast<const T*>(a.k) + (int64_t)kvh * D);
  const char* vbase = reinterpret_cast<const char*>(static_cast<const T*>(a.v) + (int64_t)kvh * D);
  const int ntiles = (kend - start + BN - 1) / BN;
  // wavefront w fills row groups w and w + NW of the K and V tiles (rows past kend repeat row
  // kend - 1: finite data, always masked)
  SwzFill<BN, NW> fk(lane, w, a.k_rs * (int64_t)sizeof(T));
  SwzFill<BN, NW> fv(lane, w, a.v_rs * (int64_t)sizeof(T));
  fk.seq_begin(kbase, start);  // tiles are issued in order: whole ones step the running addresses
  fv.seq_begin(vbase, start);
  auto issue = [&](char* kd, char* vd, int kt) {
    if (kt + BN <= kend) {
      fk.seq_whole(kd);
      fv.seq_whole(vd);
    } else {
      swz_fill2(fk, kd, kbase, fv, vd, vbase, kt, kend);
    }
  };

  if (ntiles > 0) issue(kv[0][0], kv[0][1], start);
  // Tile t sits in buffer B = t % 2, the loop unrolled by two so that B is a constant and the
  // tiles' LDS addresses fold into the reads' immediate offsets, as in the forward
  // (config-5-like backward 4.70 -> 4.66 ms, the same bits). The dK / dV kernel is left rolled:
  // unrolled it spills at its 256 registers and measured 4.5% slower.
  auto tile = [&](int t, auto bc) {
    constexpr int B = decltype(bc)::value;
    // this wavefront's DMA of tile t has landed; the barrier publishes every wavefront's rows
    // and certifies that tile t - 1, in the other buffer, is consumed
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
    if (t + 1 < ntiles) issue(kv[B ^ 1][0], kv[B ^ 1][1], start + (t + 1) * BN);
    const int kt = start + t * BN;
    if (!wave_live || kt > wq_last) return;
    dq_tile_swz<T>(kv[B][0], kv[B][1], kt, qw0, qi, lane, a.scale_log2, lse2, delta, qb, db, dqa);
  };
  int t = 0;
  for (; t + 1 < ntiles; t += 2) {
    tile(t, std::integral_constant<int, 0>{});
    tile(t + 1, std::integral_constant<int, 1>{});
  }
  if (t < ntiles) tile(t, std::integral_constant<int, 0>{});
  if (!qok) return;
  store_rows_t<T, D>(static_cast<T*>(b.dq) + (int64_t)qi * b.dq_rs + (int64_t)h * D, dqa, hi,
                     a.scale);
}

// dK / dV blocks: NW wavefronts (32 keys each) and query tiles of BQ rows. D = 128 takes 4
// wavefronts with 32-query tiles (two blocks per CU, each hiding the other's barriers); 8
// wavefronts (256 keys, one block per CU by LDS) measured slower at config 5 (backward 10.8
// against 8.4 ms when tuned) and, with the longest-first block order, at config 4 (0.182 against
// 0.171 ms with the query heads split six ways). D = 64 takes 4 wavefronts and 64-query tiles.
template <typename T, int D, int NW, int BQ>
__global__ __launch_bounds__(64 * NW, 2) void k_attn_bwd_dkdv(const AttnBwdArgs b, int ktiles,
                                                               int order) {
  constexpr int NT = 64 * NW, BK = 32 * NW;
  using V8 = typename Mfma<T>::v8;
  const AttnArgs& a = b.f;
  constexpr int RP = D + kRowPad;  // row-major pitch
  // DMA (D = 128): the Q / dO / lse / delta of a work item move by LDS DMA into a ring of two
  // buffers, item it + 1 in flight while item it is consumed, one barrier per item; query rows
  // past the sequence end repeat its last row and are masked (p = 0). Otherwise (D = 64: rows of
  // 128 bytes) they move through registers, the next item prefetched, rows past the end zeroed.
  // With DMA the tiles are swizzled and unpadded (attention.hpp: SwzFill, swz_row_base, SwzTr;
  // 256-byte rows), otherwise row-major with pitch RP.
  constexpr bool DMA = D == 128;
  constexpr int NB = DMA ? 2 : 1;
  constexpr int ROWB = DMA ? 256 : RP * (int)sizeof(T);  // bytes per tile row
  __shared__ __align__(1024) char qs[NB][BQ * ROWB];   // Q (A operand of S; transposed, of dK^T)
  __shared__ __align__(1024) char ds_[NB][BQ * ROWB];  // dO (A operand of dP; transposed, of dV^T)
  __shared__ __align__(16) float ld_s[NB][2 * BQ];  // lse (log2 units without DMA), then delta
  __shared__ __align__(1024) char vsm[BK * ROWB];  // this block's V rows (B operands of dP)

  // XCD-aware order: the key tiles of one (sequence, kv head, part) run on one XCD (they read
  // the same Q / dO rows)
  const int split = b.split;                 // query-head groups per kv head
  const int lin = block_order((int)blockIdx.x, ktiles, a.HK * split * a.n_seq, order, a.HK * split,
                              a.cu, a.n_seq, a.T);
  const int bx = lin % ktiles, rest = lin / ktiles;
  const int yy = rest % (a.HK * split), seq = rest / (a.HK * split);
  if (seq >= a.n_seq) return;
  const int kh = yy / split, part = yy % split;
  int start, end;
  seq_bounds(a.cu, seq, a.T, &start, &end);
  const int ntiles = (end - start + BK - 1) / BK;
  if (bx >= ntiles) return;
  const int k0 = start + bx * BK;  // early key tiles see the most queries
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int lq = lane & 31, hi = lane >> 5;
  const int kw0 = k0 + 32 * w;  // this wavefront's first key
  const int kj = kw0 + lq;      // this lane's key
  const bool kok = kj < end;
  const bool wave_live = kw0 < end;
  const int gs = a.HQ / a.HK / split;          // query heads of this block
  const int h0 = kh * (a.HQ / a.HK) + part * gs;

  // K of this lane's key as B operands in registers (B[d][key] = K[key][d]); the block's V rows
  // in LDS, read as the B operands of dP (published by the first barrier of the loop).
  V8 kb[D / 16];
  {
    const T* krow = static_cast<const T*>(a.k) + (int64_t)kj * a.k_rs + (int64_t)kh * D + 8 * hi;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) kb[c] = kok ? ld16<V8>(krow + 16 * c) : V8{};
  }
  {
    TileRows<T, D, BK, NT> vr;
    vr.load(static_cast<const T*>(a.v) + (int64_t)kh * D, a.v_rs, k0, end, tid);
    if constexpr (DMA)
      vr.store_swz(vsm, tid);
    else
      vr.template store<RP>(reinterpret_cast<T*>(vsm), tid);
  }
  // row-operand reads of this wave's V rows (32 w + lq) and of the Q / dO tiles' rows
  // (32 qh + lq): chunk pair c at byte rop + rowc(c) of the row group's base
  const uint32_t rop = DMA ? swz_row_base(lane) : (uint32_t)(lq * RP * (int)sizeof(T) + 16 * hi);
  auto rowc = [&](int c) -> uint32_t { return DMA ? (rop ^ (32u * c)) : rop + 32u * c; };
  const char* vlds = vsm + 32 * w * ROWB;
  const SwzTr trd(lane);
  f32x16 dka[D / 32], dva[D / 32];
#pragma unroll
  for (int md = 0; md < D / 32; ++md) dka[md] = dva[md] = f32x16{};

  // Work items (head, query tile) in order.
  const int nqt = (end - k0 + BQ - 1) / BQ;
  const int items = gs * nqt;
  // register path: the next item's Q, dO, lse and delta, loaded while the current one is computed
  TileRows<T, D, BQ, NT> pq, pd;
  float lse_n = 0.f, del_n = 0.f;
  auto prefetch = [&](int it) {
    const int h = h0 + it / nqt, qt = k0 + (it % nqt) * BQ;
    const int64_t col = (int64_t)h * D;
    pq.load(static_cast<const T*>(a.q) + col, a.q_rs, qt, end, tid);
    pd.load(static_cast<const T*>(b.dout) + col, b.do_rs, qt, end, tid);
    if (tid < BQ) {
      const int t = qt + tid;
      lse_n = t < end ? a.lse[(int64_t)h * a.T + t] * kLog2e : 0.f;
      del_n = t < end ? b.delta[(int64_t)h * a.T + t] : 0.f;
    }
  };
  // DMA path: wavefront w moves rows w, w + NW, ... of Q and dO (one 256-byte row per
  // instruction) and wavefront 0 the lse / delta words (64 per instruction)
  const int wu = __builtin_amdgcn_readfirstlane(w);
  // DMA path: wavefront w fills row groups w, w + NW, ... of the swizzled Q and dO tiles (rows
  // past the sequence end repeat its last row) and wavefront 0 the lse / delta words
  // items are issued in order: a query head's whole tiles step the fillers' running addresses
  SwzFill<BQ, NW> fq(lane, wu, a.q_rs * (int64_t)sizeof(T));
  SwzFill<BQ, NW> fd(lane, wu, b.do_rs * (int64_t)sizeof(T));
  auto issue = [&](int it, int buf) {
    const int h = h0 + it / nqt, qt = k0 + (it % nqt) * BQ;
    const int64_t col = (int64_t)h * D;
    const char* qbase = reinterpret_cast<const char*>(static_cast<const T*>(a.q) + col);
    const char* dbase = reinterpret_cast<const char*>(static_cast<const T*>(b.dout) + col);
    if (it % nqt == 0) {
      fq.seq_begin(qbase, k0);
      fd.seq_begin(dbase, k0);
    }
    if (qt + BQ <= end) {
      fq.seq_whole(qs[buf]);
      fd.seq_whole(ds_[buf]);
    } else {
      swz_fill2(fq, qs[buf], qbase, fd, ds_[buf], dbase, qt, end);
    }
    if (wu == 0) {
#pragma unroll
      for (int k = 0; k < 2 * BQ / 64; ++k) {
        const int f = 64 * k + lane;  // word f of [lse | delta]
        const int t0 = qt + (f < BQ ? f : f - BQ);
        const int t = t0 < end ? t0 : end - 1;
        const float* src = (f < BQ ? a.lse : b.delta) + (int64_t)h * a.T + t;
        lds_dma_dword(src, &ld_s[buf][64 * k]);
      }
    }
  };
  if (items > 0) {
    if constexpr (DMA)
      issue(0, 0);
    else
      prefetch(0);
  }

  for (int it = 0; it < items; ++it) {
    const int qt = k0 + (it % nqt) * BQ;
    const int buf = DMA ? (it & 1) : 0;
    if constexpr (DMA) {
      // this wavefront's DMA of item it has landed; the barrier publishes every wavefront's
      // rows and certifies that item it - 1 (the other buffer) is consumed
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      __syncthreads();
      if (it + 1 < items) issue(it + 1, buf ^ 1);
    } else {
      __syncthreads();  // the previous item's LDS reads are done
      pq.template store<RP>(reinterpret_cast<T*>(qs[0]), tid);
      pd.template store<RP>(reinterpret_cast<T*>(ds_[0]), tid);
      if (tid < BQ) {
        ld_s[0][tid] = lse_n;
        ld_s[0][BQ + tid] = del_n;
      }
      __syncthreads();
      if (it + 1 < items) prefetch(it + 1);
    }
    // every query of the tile comes before this wave's keys: nothing to add
    if (!wave_live || qt + BQ - 1 < kw0) continue;
    const char* qsb = qs[buf];
    const char* dsb = ds_[buf];
    const float* lse_s = ld_s[buf];
    const float* del_s = ld_s[buf] + BQ;
    // with DMA, rows past the sequence end hold repeated data: mask them like future queries
    const int qlim = DMA ? end : 0x7fffffff;
    const float lmul = DMA ? kLog2e : 1.f;

    // one 32-query half at a time
#pragma unroll
    for (int qh = 0; qh < BQ / 32; ++qh) {
      __builtin_amdgcn_s_setprio(1);  // MFMA runs at raised priority, as in the forward
      f32x16 s = f32x16{}, dp = f32x16{};
      const char* qrow = qsb + 32 * qh * ROWB;
      const char* drow = dsb + 32 * qh * ROWB;
      {
        // operands read two chunks ahead, pinned by scheduling barriers (the largest read-ahead
        // that fits 256 registers: config 5 backward 5.02 -> 4.95 ms)
        constexpr int RA = 2;
        V8 qbf[RA], dbf[RA], vbf[RA];
#pragma unroll
        for (int c = 0; c < RA; ++c) {
          qbf[c] = ld16<V8>(qrow + rowc(c));
          dbf[c] = ld16<V8>(drow + rowc(c));
          vbf[c] = ld16<V8>(vlds + rowc(c));
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          s = Mfma<T>::run(qbf[c % RA], kb[c], s);
          dp = Mfma<T>::run(dbf[c % RA], vbf[c % RA], dp);
          if (c + RA < D / 16) {
            qbf[c % RA] = ld16<V8>(qrow + rowc(c + RA));
            dbf[c % RA] = ld16<V8>(drow + rowc(c + RA));
            vbf[c % RA] = ld16<V8>(vlds + rowc(c + RA));
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      __builtin_amdgcn_s_setprio(0);
      // s[i] is S[q][kj] for query row r = 32 qh + 8 (i / 4) + 4 hi + i % 4 of the tile. Rows
      // past the sequence end have Q = dO = 0 (staged as zeros), so they add nothing to dK or
      // dV whatever their p; only the causal mask needs applying, and only on the half-tiles
      // whose first query precedes the wave's last key.
      if (qt + 32 * qh < kw0 + 31 || qt + 32 * qh + 31 >= qlim) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int t = qt + 32 * qh + 8 * (i / 4) + 4 * hi + (i % 4);
          if (t < kj || t >= qlim) s[i] = -INFINITY;
        }
      }
      V8 pb[2], sb_[2];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 l4 = *reinterpret_cast<const float4*>(&lse_s[32 * qh + 8 * j + 4 * hi]);
        const float4 d4 = *reinterpret_cast<const float4*>(&del_s[32 * qh + 8 * j + 4 * hi]);
        const float lr[4] = {l4.x, l4.y, l4.z, l4.w}, dr[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int i = 4 * j + e;
          const float p = exp2_fast(fmaf(s[i], a.scale_log2, -lr[e] * lmul));
          pb[i / 8][i % 8] = (T)p;
          sb_[i / 8][i % 8] = (T)(p * (dp[i] - dr[e]));
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_s_setprio(1);
      // dV^T += dO^T P and dK^T += Q^T dS, queries in the permuted order of pb / sb_: operand
      // pair i = (md, c2) = (i / 2, i % 2) read RB pairs ahead, pinned by scheduling barriers
      // (the compiler kept one pair ahead: config-5-like backward 4.66 -> 4.56 ms, the same
      // bits; three ahead, or the first pairs read before the exponentials, spill at 256
      // registers)
      constexpr int RB = 2;
      V8 dotb[RB], qtb[RB];
      auto rd = [&](int i, int slot) {
        const int md = i >> 1, rb = 32 * qh + 16 * (i & 1);
        if constexpr (DMA) {
          dotb[slot] = trd.template read<V8>(dsb, rb, md);
          qtb[slot] = trd.template read<V8>(qsb, rb, md);
        } else {
          dotb[slot] = ld_tr<V8, RP>(reinterpret_cast<const T*>(dsb), rb, 32 * md, lane);
          qtb[slot] = ld_tr<V8, RP>(reinterpret_cast<const T*>(qsb), rb, 32 * md, lane);
        }
      };
#pragma unroll
      for (int i = 0; i < RB; ++i) rd(i, i);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 2 * (D / 32); ++i) {
        const int md = i >> 1, c2 = i & 1;
        dva[md] = Mfma<T>::run(dotb[i % RB], pb[c2], dva[md]);
        dka[md] = Mfma<T>::run(qtb[i % RB], sb_[c2], dka[md]);
        if (i + RB < 2 * (D / 32)) rd(i + RB, i % RB);
        __builtin_amdgcn_sched_barrier(0);
      }
      __builtin_amdgcn_s_setprio(0);
    }
  }
  if (!kok) return;
  if (split == 1) {
    store_rows_t<T, D>(static_cast<T*>(b.dk) + (int64_t)kj * b.dk_rs + (int64_t)kh * D, dka, hi,
                       a.scale);
    store_rows_t<T, D>(static_cast<T*>(b.dv) + (int64_t)kj * b.dv_rs + (int64_t)kh * D, dva, hi,
                       1.f);
    return;
  }
  // fp32 partials [split][T][HK][D] of dK^T / scale and dV^T, summed by k_attn_dkdv_reduce
  const int64_t plane = a.T * a.HK * D;
  float* pk = b.part + (int64_t)part * plane + ((int64_t)kj * a.HK + kh) * D + 4 * hi;
  float* pv = pk + (int64_t)split * plane;
#pragma unroll
  for (int md = 0; md < D / 32; ++md)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      *reinterpret_cast<float4*>(pk + 32 * md + 8 * j) =
          make_float4(dka[md][4 * j], dka[md][4 * j + 1], dka[md][4 * j + 2], dka[md][4 * j + 3]);
      *reinterpret_cast<float4*>(pv + 32 * md + 8 * j) =
          make_float4(dva[md][4 * j], dva[md][4 * j + 1], dva[md][4 * j + 2], dva[md][4 * j + 3]);
    }
}

// dK = scale * sum_s dK_s, dV = sum_s dV_s over the split partials, s ascending. One thread per
// 4 consecutive elements of a [T, HK, D] plane.
template <typename T>
__global__ __launch_bounds__(256) void k_attn_dkdv_reduce(const AttnBwdArgs b, int D) {
  const int64_t plane = b.f.T * b.f.HK * D;
  const int64_t e = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
  if (e >= plane) return;
  const int64_t t = e / ((int64_t)b.f.HK * D), r = e % ((int64_t)b.f.HK * D);
  for (int which = 0; which < 2; ++which) {
    const float* src = b.part + (int64_t)which * b.split * plane + e;
    float4 acc = *reinterpret_cast<const float4*>(src);
    for (int s = 1; s < b.split; ++s) {
      const float4 v = *reinterpret_cast<const float4*>(src + (int64_t)s * plane);
      acc.x += v.x;
      acc.y += v.y;
      acc.z += v.z;
      acc.w += v.w;
    }
    const float mul = which == 0 ? b.f.scale : 1.f;
    T o4[4] = {(T)(acc.x * mul), (T)(acc.y * mul), (T)(acc.z * mul), (T)(acc.w * mul)};
    T* dst = static_cast<T*>(which == 0 ? b.dk : b.dv) + t * (which == 0 ? b.dk_rs : b.dv_rs) + r;
    *reinterpret_cast<uint2*>(dst) = __builtin_bit_cast(uint2, o4);
  }
}

template <typename T, int D>
hipError_t bwd_run(const AttnBwdArgs& b, int max_seqlen, hipStream_t s) {
  // 4 wavefronts (128 queries) per dQ block: 8 measured slower (with 256 causal queries per
  // block the early wavefronts idle through the later key tiles).
  constexpr int QW = 4;
  const dim3 gq((max_seqlen + 32 * QW - 1) / (32 * QW), b.f.HQ, b.f.n_seq);
  if constexpr (D == 128) {
    const int64_t n = xcd_grid(gq.x, (int64_t)gq.y * gq.z);
    if (n > 0x7fffffff) return hipErrorInvalidValue;
    // 2 blocks resident per CU (launch bound)
    hipLaunchKernelGGL((k_attn_bwd_dq_dma<T, QW>), dim3((unsigned)n), dim3(64 * QW), 0, s, b,
                       (int)gq.x, attn_order(n, 2, b.f.n_seq));
  } else {
    hipLaunchKernelGGL((k_attn_bwd_dq<T, D, QW>), gq, dim3(64 * QW), 0, s, b);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  bool too_big = false;
  auto dkdv = [&](auto nw, auto bq) {
    constexpr int NW = decltype(nw)::value, BQ = decltype(bq)::value;
    const int64_t ktiles = (max_seqlen + 32 * NW - 1) / (32 * NW);
    const int64_t n = xcd_grid(ktiles, (int64_t)b.f.HK * b.split * b.f.n_seq);
    if (n > 0x7fffffff) {
      too_big = true;
      return;
    }
    // 2 blocks resident per CU (launch bound)
    hipLaunchKernelGGL((k_attn_bwd_dkdv<T, D, NW, BQ>), dim3((unsigned)n), dim3(64 * NW), 0, s, b,
                       (int)ktiles, attn_order(n, 2, b.f.n_seq));
  };
  if constexpr (D == 128) {
    dkdv(std::integral_constant<int, 4>{}, std::integral_constant<int, 32>{});
  } else {
    dkdv(std::integral_constant<int, 4>{}, std::integral_constant<int, 64>{});
  }
  if (too_big) return hipErrorInvalidValue;
  e = hipGetLastError();
  if (e != hipSuccess || b.split == 1) return e;
  const int64_t quads = b.f.T * b.f.HK * D / 4;
  hipLaunchKernelGGL((k_attn_dkdv_reduce<T>), dim3((unsigned)((quads + 255) / 256)), dim3(256), 0,
                     s, b, D);
  return hipGetLastError();
}

template <typename T>
hipError_t bwd_d(const AttnBwdArgs& b, int D, int max_seqlen, hipStream_t s, bool* sup) {
  *sup = true;
  if (D == 128) return bwd_run<T, 128>(b, max_seqlen, s);
  if (D == 64) return bwd_run<T, 64>(b, max_seqlen, s);
  *sup = false;
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_attn_bwd(const AttnBwdArgs& b, int dt, int D, int max_seqlen, hipStream_t s,
                           bool* sup) {
  if (dt == 1) return bwd_d<_Float16>(b, D, max_seqlen, s, sup);
  if (dt == 2) return bwd_d<__bf16>(b, D, max_seqlen, s, sup);
  *sup = false;
  return hipErrorInvalidValue;
}

}  // namespace esep

// Varlen causal attention (GQA) on the packed token layout for gfx950 (MI355X): the consumer
// of the RoPE output. Replaces the per-row scaled_dot_product_attention loop of the reference
// decoder (solution/body/packed.py:404-436: per original row, causal, query head h reads kv
// head h / (HQ / HK), scale = attn.scaling).
//
// Layout. q [T, HQ, D], k / v [T, HK, D], o [T, HQ, D] with a token (row) stride each and the
// heads of a token contiguous; cu_seqlens int32 [n_seq + 1] splits the T tokens into
// sequences that attend only within themselves; lse fp32 [HQ, T] (natural-log sum of
// exp(scale * s) per query), kept for the backward.
//
// Forward mapping (flash-attention style, one pass, online softmax). A block of 4 wavefronts
// owns 128 queries of one sequence and one query head; wavefront w owns queries 32w..32w+31 of
// the block, heaviest query tiles first. At D = 128 the keys come in tiles of 32 moved by LDS
// DMA through a two-buffer ring (the next tile in flight during the current one); at D = 64 in
// tiles of 64 staged through registers and consumed in halves of 32. Scores are computed transposed, S^T = K Q^T, with
// v_mfma_f32_32x32x16 (K from LDS as the A operand, the wave's Q held in registers as the B
// operand), so each lane owns one query and 16 of a half's 32 scores; the other 16 sit in lane
// l ^ 32, and a row max or sum is a register reduction plus one cross-half exchange. The probabilities go straight from the
// score registers into O^T += V^T P^T: the contraction over keys is permuted so that the B
// operand a lane needs is exactly the scores it holds, and V^T (read transposed out of the row-major V tile) is
// read in the same permuted key order.
//
// MFMA lane layouts (checked on the device against a CPU product): v_mfma_f32_32x32x16_{bf16,f16}
// takes A[i][k] from lane i % 32 + 32 * (k / 8), element k % 8; B[k][j] from lane
// j + 32 * (k / 8), element k % 8; and returns D[i][j] in lane j + 32 * ((i / 4) % 2), element
// 4 * (i / 8) + i % 4.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace esep {

struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;              // [HQ, T]
  const int32_t* cu;       // [n_seq + 1]
  int64_t q_rs, k_rs, v_rs, o_rs;  // token strides (elements)
  int64_t T;
  int n_seq;
  int HQ, HK;
  float scale;       // softmax scale (1/sqrt(D) in Qwen2)
  float scale_log2;  // scale * log2(e)
};

// Backward arguments: the forward's plus dO, the saved lse, the workspace (per-query delta,
// fp32 [HQ, T], written by the dQ kernel and read by the dK/dV kernel; then the dK / dV partials
// when the query heads of a kv head are split over blocks) and the gradients.
struct AttnBwdArgs {
  AttnArgs f;  // q, k, v, o, lse (read), cu, strides, sizes, scale
  const void* dout;
  float* delta;  // [HQ, T]
  float* part;   // [2][split][T][HK][D] fp32 dK / dV partials (split > 1)
  void* dq;
  void* dk;
  void* dv;
  int64_t do_rs, dq_rs, dk_rs, dv_rs;
  int split;  // blocks per kv head and key tile (a divisor of HQ / HK)
};

constexpr int kAttnBM = 128;  // queries per forward / dQ block (4 wavefronts x 32)
constexpr int kAttnBN = 64;   // keys per tile
constexpr int kAttnThreads = 256;
constexpr int kAttnBQ = 64;   // queries per dK / dV tile

hipError_t launch_attn_fwd(const AttnArgs& a, int dt, int D, int max_seqlen, hipStream_t s,
                           bool* supported);
hipError_t launch_attn_bwd(const AttnBwdArgs& a, int dt, int D, int max_seqlen, hipStream_t s,
                           bool* supported);

// ---------------------------------------------------------------------------------------
// Device helpers shared by the attention kernels
// ---------------------------------------------------------------------------------------
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <typename T>
struct Mfma;
template <>
struct Mfma<__bf16> {
  typedef __bf16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 run(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<_Float16> {
  typedef _Float16 v8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16 run(v8 a, v8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Row pitch (elements) of the row-major LDS tiles: D + kRowPad. At D = 128 the pitch is 152 bf16
// = 76 dwords, rows at bank offsets 12 r mod 64: the 8 rows a transposing operand read (ld_tr)
// touches and the 16 rows of a 16-byte row read both spread over the banks. Measured on the
// backward at config 5: +8 (68 dwords) 11.6 ms, +16 11.4, +24 10.8, +32 (16 r: 4-way row
// conflicts) 13.2, +40 10.7, +48 11.0.
constexpr int kRowPad = 24;

// 2^x on the hardware's v_exp_f32 alone (no denormal-range scaling: results below 2^-126 flush
// to 0, far below what a probability contributes next to the sums they enter).
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// max / sum of a lane's value and lane l ^ 32's, equal in both lanes (v_permlane32_swap hands
// each lane the pair {own, partner} without going through LDS; + and max are commutative, so
// both halves get the same bits).
__device__ __forceinline__ float pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}

template <typename V>
__device__ __forceinline__ V ld16(const void* p) {
  return __builtin_bit_cast(V, *reinterpret_cast<const uint4*>(p));
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

// A operand (8 elements) of v_mfma_f32_32x32x16 read transposed out of a row-major LDS matrix M
// (pitch P elements): A[i][kk] = M[r0 + pi(kk)][c0 + i], i < 32, kk < 16, where pi is the
// permuted contraction order of the score accumulators (kk 0-3, 4-7, 8-11, 12-15 -> rows 0-3,
// 8-11, 4-7, 12-15: the rows a lane holds in its B operand). Two ds_read_b64_tr_b16: within a
// 16-lane group the hardware hands lane j, slot k, element j % 4 of the 8-byte segment
// addressed by lane 4 k + j / 4 (checked on the device), so lane 16 g + 4 k + m addresses row
// r0 + 4 (g / 2) + k (+ 8 for the second read), columns c0 + 16 (g % 2) + 4 m .. + 3.
template <typename V, int P, typename T>
__device__ __forceinline__ V ld_tr(const T* M, int r0, int c0, int lane) {
  const int g = lane >> 4, k = (lane >> 2) & 3, m = lane & 3;
  T* p = const_cast<T*>(M) + (r0 + 4 * (g >> 1) + k) * P + c0 + 16 * (g & 1) + 4 * m;
  typedef __attribute__((address_space(3))) s16x4* lds_ptr;
  const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(p));
  const s16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(p + 8 * P));
  return __builtin_bit_cast(V, __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7));
}

// One LDS DMA instruction: lane l reads the dword at g (its own address) and the wavefront
// writes the 64 dwords to LDS bytes lds .. lds + 255 (lane l at lds + 4 l). Issued from asm so
// that the compiler does not track it: its own LDS-DMA tracking cannot tell the two buffers
// apart for the transposing reads and would wait for the next tile before reading this one.
// The kernel waits for the DMA itself (s_waitcnt vmcnt(0) before the barrier that publishes a
// tile). The LDS address goes in M0 through the "{m0}" operand constraint: the compiler itself
// loads M0 before the instruction and knows what M0 holds afterwards (the asm only reads it),
// so no M0 value of the compiler's own is ever overwritten behind its back.
__device__ __forceinline__ void lds_dma_dword(const void* g, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("global_load_lds_dword %0, off" ::"v"(g), "{m0}"(m) : "memory");
}

// s_waitcnt vmcnt(0) (expcnt, lgkmcnt left at their maxima): through the builtin, so that the
// compiler's own wait tracking sees it too.
constexpr int kWaitVm0 = 0x0F70;

// ---------------------------------------------------------------------------------------
// Swizzled, unpadded LDS tiles of 256-byte token rows (D = 128, 16-bit elements), filled 1 KiB
// per DMA instruction.
//
// Chunk c (16 bytes) of tile row r sits at chunk position c ^ swz(r), swz(r) = 4 (r & 3) +
// ((r >> 2) & 3): the 16 rows a row-operand read touches (one chunk each, SwzRow) and the
// 4 rows x 4 chunks a transposing read touches in one pass (SwzTr) land on 16 different
// positions, so neither read has bank conflicts without a pitch pad (checked on the CPU).
// global_load_lds_dwordx4 writes lane l's 16 bytes at M0 + 16 l (checked on the device), so one
// instruction fills 4 whole rows: lane l loads the global chunk that belongs at its position,
// ((l & 15) ^ swz(row)) of row l >> 4 of its 4-row group.
// ---------------------------------------------------------------------------------------
__device__ __forceinline__ void lds_dma_x4_s(const void* base, uint32_t voff, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(m) : "memory");
}
__device__ __forceinline__ void lds_dma_x4(const void* g, const void* lds) {
  const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(m) : "memory");
}

__device__ __forceinline__ int swz(int r) { return 4 * (r & 3) + ((r >> 2) & 3); }

// One wavefront's share of filling a ROWS-row swizzled tile from token rows r0 .. r0 + ROWS - 1
// of a tensor (base: row 0's first element of the head; rs: bytes between token rows): with
// NW wavefronts (a multiple of 4), wavefront w fills the 4-row groups w, w + NW, ... Rows at or
// past rend repeat row rend - 1. A whole tile is addressed from an SGPR base; a partial one
// clamps each lane's row.
template <int ROWS, int NW>
struct SwzFill {
  static_assert(NW % 4 == 0 && ROWS % (4 * NW) == 0, "groups per wavefront");
  int w, lrow, lchunk;
  int64_t rs;
  const char* cur;  // seq_begin / seq_whole: the next whole tile's first row group
  int64_t tstep;    // bytes of ROWS token rows
  uint32_t voff;
  __device__ __forceinline__ SwzFill(int lane, int w_, int64_t rs_)
      : w(w_), rs(rs_), cur(nullptr), tstep(0) {
    lrow = lane >> 4;
    lchunk = (lane & 15) ^ (4 * lrow + (w & 3));  // swz(4 q + lrow) with q & 3 = w & 3
    voff = (uint32_t)(lrow * rs) + 16u * (uint32_t)lchunk;
  }
  __device__ __forceinline__ void whole(char* dst, const char* base, int r0) const {
#pragma unroll
    for (int i = 0; i < ROWS / (4 * NW); ++i) {
      const int q = w + NW * i;
      lds_dma_x4_s(base + (int64_t)(r0 + 4 * q) * rs, voff, dst + 1024 * q);
    }
  }
  __device__ __forceinline__ void partial(char* dst, const char* base, int r0, int rend) const {
#pragma unroll
    for (int i = 0; i < ROWS / (4 * NW); ++i) {
      const int q = w + NW * i;
      const int r = r0 + 4 * q + lrow < rend ? r0 + 4 * q + lrow : rend - 1;
      lds_dma_x4(base + (int64_t)r * rs + 16 * lchunk, dst + 1024 * q);
    }
  }

  // Consecutive whole tiles: `cur` (an SGPR pair) addresses this wavefront's first 4-row group
  // of the next tile and moves ROWS rows per tile; the wavefront's other groups of a tile are
  // per-lane offsets from it. A tile then costs one 64-bit add instead of a 64-bit multiply and
  // add per DMA instruction (forward: config 5 1.46 -> 1.445 ms, the packed decoder's shape
  // 39.3 -> 38.0 us; the backward unchanged).
  __device__ __forceinline__ void seq_begin(const char* base, int r0) {
    cur = base + (int64_t)(r0 + 4 * w) * rs;
    tstep = (int64_t)ROWS * rs;
  }
  __device__ __forceinline__ void seq_whole(char* dst) {
#pragma unroll
    for (int i = 0; i < ROWS / (4 * NW); ++i)
      lds_dma_x4_s(cur, voff + (uint32_t)(4 * NW * i) * (uint32_t)rs, dst + 1024 * (w + NW * i));
    cur += tstep;
  }
};

// Two tiles of the same rows (e.g. K and V) with one whole-or-partial decision.
template <int ROWS, int NW>
__device__ __forceinline__ void swz_fill2(const SwzFill<ROWS, NW>& fa, char* da, const char* ba,
                                          const SwzFill<ROWS, NW>& fb, char* db, const char* bb,
                                          int r0, int rend) {
  if (r0 + ROWS <= rend) {
    fa.whole(da, ba, r0);
    fb.whole(db, bb, r0);
  } else {
    fa.partial(da, ba, r0, rend);
    fb.partial(db, bb, r0, rend);
  }
}

// Row operand (A or B of v_mfma_f32_32x32x16 with the rows in lanes): lane (lq, hi) reads
// chunk 2c + hi of tile row lq (+ 32 h for rows 32 h + lq) at byte
// (swz_row_base(lane) ^ 32 c) + 8192 h.
__device__ __forceinline__ uint32_t swz_row_base(int lane) {
  const int lq = lane & 31, hi = lane >> 5, f = swz(lq);
  return 256u * lq + 16u * ((hi ^ f) & 1) + 32u * (f >> 1);
}

// Transposing operand read (ld_tr's lane mapping) out of a swizzled tile: rows rb + 4 (g >> 1)
// + k (+ 8), columns 32 md + 16 (g & 1) + 4 m, for rb a multiple of 16. Byte offset
// ((o_u | 64 k) ^ 64 md) + 256 rb for the lower (u = 0) and upper (u = 1) read, with
// o_u = 256 (4 (g >> 1) + k + 8 u) + 16 L_u + 8 (m & 1) and
// L_u = (2 (g & 1) + (m >> 1)) ^ (((g >> 1) + 2 u) & 3).
struct SwzTr {
  uint32_t o[2];
  __device__ __forceinline__ explicit SwzTr(int lane) {
    const int g = lane >> 4, k = (lane >> 2) & 3, m = lane & 3;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int L = (2 * (g & 1) + (m >> 1)) ^ (((g >> 1) + 2 * u) & 3);
      o[u] = (256u * (4 * (g >> 1) + k + 8 * u) + 16u * L + 8u * (m & 1)) | (64u * k);
    }
  }
  template <typename V>
  __device__ __forceinline__ V read(const char* tile, int rb, int md) const {
    typedef __attribute__((address_space(3))) s16x4* lds_ptr;
    const uint32_t x = 64u * md, y = 256u * rb;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(tile + ((o[0] ^ x) + y)));
    const s16x4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(tile + ((o[1] ^ x) + y)));
    return __builtin_bit_cast(V, __builtin_shufflevector(lo, up, 0, 1, 2, 3, 4, 5, 6, 7));
  }
};

// XCD-aware block order. The hardware deals the workgroups of a launch round-robin over the 8
// XCDs (workgroup b to XCD b % 8), each with its own L2. A kernel that wants the C blocks of one
// group (e.g. all query tiles of one (sequence, head): they read the same K / V rows) on one
// XCD launches xcd_grid(C, groups) one-dimensional blocks and maps its workgroup id through
// xcd_order: XCD x then takes groups x, x + 8, x + 16, ... whole, so every XCD still gets a mix
// of groups (sequences of different lengths). The result is the block's index in the
// group-major order (group * C + index in the group); indices past C * groups (the padding to a
// multiple of 8 groups) belong to no group and their blocks exit.
__device__ __forceinline__ int xcd_order(int b, int C) {
  const int xcd = b % 8, slot = b / 8;
  return (xcd + 8 * (slot / C)) * C + slot % C;
}
inline int64_t xcd_grid(int64_t C, int64_t groups) { return (groups + 7) / 8 * 8 * C; }

// xcd_order with each XCD running its groups tile-major: tile 0 of every group it holds, then
// tile 1, and so on, in the order the hardware dispatches its workgroups. The kernels number a
// group's tiles heaviest first (causal: the query tile with the most keys, the key tile with
// the most queries), so every XCD starts its longest blocks before its short ones
// (longest-processing-time first); groups stay whole on one XCD as with xcd_order. It pays when
// the grid is resident in about one round (short inputs: the longest blocks set the kernel's
// time); on long inputs the group-by-group order of xcd_order keeps a group's K / V (or Q / dO)
// reads close together in time in its XCD's L2 and is faster (block_order picks).
__device__ __forceinline__ int xcd_order_lpt(int b, int C, int groups) {
  const int xcd = b % 8, slot = b / 8;
  const int per_xcd = (groups + 7) / 8;
  return (xcd + 8 * (slot % per_xcd)) * C + slot / per_xcd;
}
// Whether a grid of `blocks` workgroups of a kernel that keeps `per_cu` of them resident on each
// of MI355X's 256 CUs runs longest-first (xcd_order_lpt): at most two rounds of residency.
constexpr int64_t kAttnCUs = 256;
inline int use_lpt(int64_t blocks, int per_cu) { return blocks <= 2 * kAttnCUs * per_cu ? 1 : 0; }

// Sequence s's token range [start, end), clamped into [0, T].
__device__ __forceinline__ void seq_bounds(const int32_t* cu, int s, int64_t T, int* start,
                                           int* end) {
  const int tt = (int)T;
  const int c0 = cu[s], c1 = cu[s + 1];
  *start = c0 < 0 ? 0 : (c0 > tt ? tt : c0);
  *end = c1 < *start ? *start : (c1 > tt ? tt : c1);
}

// The sequence of rank r when the n_seq <= 64 sequences are ordered longest first (ties by
// index): lane s ranks sequence s against all others, and the lane holding rank r is found by
// ballot. Every lane of the wavefront gets the answer (n_seq when r is out of range).
__device__ __forceinline__ int seq_of_rank(const int32_t* cu, int n_seq, int64_t T, int r) {
  const int lane = (int)(threadIdx.x & 63);
  int len = -1;
  if (lane < n_seq) {
    int s, e;
    seq_bounds(cu, lane, T, &s, &e);
    len = e - s;
  }
  int rank = 0;
  for (int j = 0; j < n_seq; ++j) {
    const int lj = __builtin_amdgcn_readlane(len, j);
    rank += (lj > len || (lj == len && j < lane)) ? 1 : 0;
  }
  const uint64_t hit = __ballot(lane < n_seq && rank == r);
  return hit != 0 ? (int)__builtin_ctzll(hit) : n_seq;
}

// Block orders of the D = 128 attention kernels, chosen per launch (attn_order):
//   kOrderGroups  xcd_order: each XCD runs its groups one after another;
//   kOrderLpt     xcd_order_lpt: each XCD runs its groups tile-major, longest tiles first (grids
//                 resident in at most two rounds);
//   kOrderSorted  the groups (gps per sequence, sequence-major) sorted by their sequence's
//                 length, longest first, and dealt to the 8 XCDs in snake order (XCD 0..7, then
//                 7..0, ...): every XCD gets a near-equal share of the work and runs its groups
//                 heaviest first, each group whole with its tiles in a row as with xcd_order
//                 (n_seq <= 64). Dealing groups round-robin in index order instead put a
//                 sequence's 4 kv-head groups of config 5's dK / dV on XCDs 0-3 or 4-7 by the
//                 sequence's parity, and the two halves' work differed by 38%.
// The result is the block's index in the group-major order (group * C + tile); a padding block
// gets an index past the last group and exits.
constexpr int kOrderGroups = 0, kOrderLpt = 1, kOrderSorted = 2;
__device__ __forceinline__ int block_order(int b, int C, int groups, int mode, int gps,
                                           const int32_t* cu, int n_seq, int64_t T) {
  if (mode == kOrderGroups) return xcd_order(b, C);
  if (mode == kOrderLpt) return xcd_order_lpt(b, C, groups);
  const int xcd = b % 8, slot = b / 8;
  const int j = slot / C, tile = slot % C;
  const int p = 8 * j + ((j & 1) ? 7 - xcd : xcd);  // position in the sorted group list
  if (p >= groups) return groups * C;
  const int seq = seq_of_rank(cu, n_seq, T, p / gps);
  return (seq * gps + p % gps) * C + tile;
}

// The order a grid of `blocks` workgroups takes when `per_cu` of them stay resident per CU.
inline int attn_order(int64_t blocks, int per_cu, int n_seq) {
  if (use_lpt(blocks, per_cu)) return kOrderLpt;
  return n_seq <= 64 ? kOrderSorted : kOrderGroups;
}

// A [ROWS x D] tile (token rows r0 .. r0 + ROWS - 1 below rend; the rest reads as 0) moved
// through registers into LDS. load() issues every global read of the thread before any is
// used (one memory round trip per tile, not one per chunk); the tile can be loaded before the
// barrier that frees its LDS buffer and stored after it.
//   rows():  thread tid holds chunks idx = tid + NT j: row idx % ROWS, 8-column chunk
//            idx / ROWS; store_rows() writes them row-major with pitch P.
template <typename T, int D, int ROWS, int NT = kAttnThreads>
struct TileRows {
  static constexpr int N = ROWS * (D / 8) / NT;
  static_assert(N >= 1 && ROWS * (D / 8) % NT == 0, "tile / block mismatch");
  uint4 r[N];

  __device__ __forceinline__ void load(const T* base, int64_t rs, int r0, int rend, int tid) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = tid + NT * j;
      const int row = r0 + idx % ROWS, dc = idx / ROWS;
      r[j] = row < rend ? *reinterpret_cast<const uint4*>(base + (int64_t)row * rs + 8 * dc)
                        : make_uint4(0, 0, 0, 0);
    }
  }

  template <int P>
  __device__ __forceinline__ void store(T* dst, int tid) const {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const int idx = tid + NT * j;
      *reinterpret_cast<uint4*>(&dst[(idx % ROWS) * P + 8 * (idx / ROWS)]) = r[j];
    }
  }

  // the same rows into a swizzled, unpadded tile (256-byte rows: D = 128 of 16-bit elements;
  // chunk c of row r at position c ^ swz(r))
  __device__ __forceinline__ void store_swz(char* dst, int tid) const;
};

template <typename T, int D, int ROWS, int NT>
__device__ __forceinline__ void TileRows<T, D, ROWS, NT>::store_swz(char* dst, int tid) const {
  static_assert(D * sizeof(T) == 256, "swizzled tiles have 256-byte rows");
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const int idx = tid + NT * j;
    const int row = idx % ROWS, chunk = idx / ROWS;
    *reinterpret_cast<uint4*>(dst + 256 * row + 16 * (chunk ^ swz(row))) = r[j];
  }
}

// Store a wavefront's [32 tokens x D] result held transposed in MFMA accumulators (acc[md]
// element 4 j + e is column 32 md + 8 j + 4 hi + e of token `row`), times `mul`.
template <typename T, int D>
__device__ __forceinline__ void store_rows_t(T* row, const f32x16 (&acc)[D / 32], int hi,
                                             float mul) {
#pragma unroll
  for (int md = 0; md < D / 32; ++md)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      T o4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) o4[e] = (T)(acc[md][4 * j + e] * mul);
      *reinterpret_cast<uint2*>(row + 32 * md + 8 * j + 4 * hi) = __builtin_bit_cast(uint2, o4);
    }
}

}  // namespace esep

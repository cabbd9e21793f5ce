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
// the block. Keys are walked in tiles of 64 (the tiles the causal mask leaves), heaviest query
// tiles first. Scores are computed transposed, S^T = K Q^T, with v_mfma_f32_32x32x16 (K from
// LDS as the A operand, the wave's Q held in registers as the B operand), so each lane owns one
// query and 32 of a tile's 64 scores; the other 32 sit in lane l ^ 32, and a row max or sum is
// a register reduction plus one cross-half exchange. The probabilities go straight from the
// score registers into O^T += V^T P^T: the contraction over keys is permuted so that the B
// operand a lane needs is exactly the scores it holds, and V^T (staged transposed in LDS) is
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

constexpr int kAttnBM = 128;  // queries per block (4 wavefronts x 32)
constexpr int kAttnBN = 64;   // keys per tile
constexpr int kAttnThreads = 256;

hipError_t launch_attn_fwd(const AttnArgs& a, int dt, int D, int max_seqlen, hipStream_t s,
                           bool* supported);

}  // namespace esep

/*
 * esep_body.h — C ABI of libesep_body.so: the decoder-body RMSNorm and rotary-embedding
 * kernels (forward and backward) for AMD Instinct MI355X (gfx950).
 *
 * The reference implementation of this path is a set of Triton kernels launched from Python
 * (gojosatorukz/esep-soup-kernels, solution/body/norm_rope.py). Each entry point below replaces
 * one launch site of that file; the citation on each declaration names it. The Python layer
 * (solution/body/norm_rope.py in this repository) keeps the reference's public API and calls
 * these functions through ctypes.
 *
 * Conventions
 *  - Every pointer is a device pointer unless stated otherwise. The library never allocates,
 *    frees or synchronizes: the caller owns every buffer, including workspaces.
 *  - Work is enqueued asynchronously on `stream` (a hipStream_t passed as void*; NULL is the
 *    default stream).
 *  - Return value: 0 on success; a negative ESEP_E* code for a rejected argument (nothing was
 *    launched); a positive hipError_t if a launch failed. esep_last_error() returns a message for
 *    the last failure on the calling thread.
 *  - Strides and leading dimensions are in elements, not bytes. The innermost dimension is
 *    always contiguous (stride 1).
 *  - Element types are the esep_dtype codes below.
 */
#ifndef ESEP_BODY_H
#define ESEP_BODY_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ESEP_ABI_VERSION 1

/* Element type codes. */
enum esep_dtype {
  ESEP_F32 = 0,
  ESEP_F16 = 1,
  ESEP_BF16 = 2,
  ESEP_I32 = 3,
  ESEP_I64 = 4
};

/* Error codes (negative returns). */
enum esep_status {
  ESEP_OK = 0,
  ESEP_EINVAL = -1,   /* bad pointer / dtype / flag combination */
  ESEP_ESHAPE = -2,   /* unsupported or inconsistent size */
  ESEP_EALIGN = -3    /* a buffer that must be 16-byte aligned is not (weight-gradient partials) */
};

/* Widest row the RMSNorm kernels accept (columns). The reference caps rows at
 * NORM_BLOCK = 2048 (solution/body/norm_rope.py:73, :215). */
#define ESEP_NORM_MAX_COLS 16384

/* Most gradients of one norm output summed by the backward kernel. Reference: MAX_DY
 * (solution/body/norm_rope.py:113). */
#define ESEP_MAX_DY 5

/* ABI version of the loaded library (ESEP_ABI_VERSION at build time). */
int esep_abi_version(void);

/* Message of the last failed call on this thread ("" if none). Valid until the next call. */
const char* esep_last_error(void);

/*
 * RMSNorm forward with optional fused residual add.
 * Replaces the launch of _add_rmsnorm_fwd at solution/body/norm_rope.py:232-236 (AddRMSNorm.forward)
 * and :321-322 (rmsnorm_recompute); kernel math follows norm_rope.py:83-109.
 *
 *   r      = x (+ delta)                 fp32 math; if r_out != NULL it is stored in x's dtype,
 *                                         and for a 16-bit x the stored (rounded) r is normalized
 *   rstd_t = 1 / sqrt(mean_j r_tj^2 + eps)
 *   y_tj   = w_j * (r_tj * rstd_t)        stored as y_dt
 *   xs[t, slot[j]] = r_tj * rstd_t        for slot[j] >= 0, when n_special > 0
 *
 * x [rows, n] (x_dt), row stride ld_x; delta [rows, n] (delta_dt) or NULL, stride ld_delta;
 * w [n] fp32; r_out [rows, n] (x_dt) or NULL, stride ld_r (ignored without delta);
 * y [rows, n] (y_dt), stride ld_y; rstd [rows] fp32 or NULL; slot [n] int32 or NULL;
 * xs [rows, n_special] fp32 (contiguous) or NULL.
 * Requires 1 <= n <= ESEP_NORM_MAX_COLS; rows >= 0 (rows == 0 launches nothing).
 */
int esep_rmsnorm_fwd(const void* x, int x_dt, int64_t ld_x,
                     const void* delta, int delta_dt, int64_t ld_delta,
                     const float* w,
                     void* r_out, int64_t ld_r,
                     void* y, int y_dt, int64_t ld_y,
                     float* rstd,
                     const int32_t* slot, float* xs, int n_special,
                     int64_t rows, int64_t n, float eps, void* stream);

/*
 * Number of rows of the fp32 [P, n] weight-gradient workspace that esep_rmsnorm_bwd needs for
 * this shape. Depends only on (rows, n), never on the device, so the two-stage dw reduction
 * is bitwise reproducible. No reference counterpart (the reference computes no weight
 * gradient: norm_rope.py:286 returns None for it).
 */
int64_t esep_rmsnorm_partials(int64_t rows, int64_t n);

/*
 * RMSNorm backward (dx, and optionally the weight gradient).
 * Replaces the launch of _add_rmsnorm_bwd at solution/body/norm_rope.py:279-283
 * (AddRMSNorm.backward); kernel math follows norm_rope.py:116-162.
 *
 *   dy     = sum_{i < n_dy} dys[i]            fp32 registers (dys[i] [rows, n] dy_dt, stride ld_dy)
 *   xhat   = x * rstd                          (from_y == 0; x is the normalized input r)
 *          = x / w, xs[t, slot[j]] where slot[j] >= 0   (from_y == 1; x is the saved output y)
 *   rstd   = saved rstd[t], or recomputed from x when rstd == NULL (from_y == 0 only)
 *   g      = dy * w;  proj = sum_j g * xhat / n
 *   dr     = rstd * (g - xhat * proj) (+ dr_out)         (dr_out fp32 [rows, n] or NULL)
 *   dr_f32 [rows, n] fp32 or NULL  <- dr
 *   dx_lp  [rows, n] dx_dt or NULL <- dr rounded to dx_dt
 *   dw_j   = sum_t dy_tj * xhat_tj             when dw_partials != NULL: stage 1 writes the
 *            partials [P, n] fp32, 16-byte aligned (P = esep_rmsnorm_partials(rows, n),
 *            n_partials must equal P; a misaligned buffer returns ESEP_EALIGN);
 *            with dw != NULL stage 2 then sums them in a fixed order into dw [n] (dw_dt), else
 *            the caller reduces them later with esep_dgamma_reduce. rows == 0 gives dw = 0.
 * n_dy == 0 and dr_out != NULL gives dr = dr_out. Contiguous rows for dr_out, dr_f32, dx_lp
 * use ld_out; x uses ld_x.
 */
int esep_rmsnorm_bwd(const void* const* dys, int n_dy, int dy_dt, int64_t ld_dy,
                     const float* dr_out,
                     const void* x, int x_dt, int64_t ld_x, int from_y,
                     const float* rstd,
                     const float* w,
                     const int32_t* slot, const float* xs, int n_special,
                     float* dr_f32, void* dx_lp, int dx_dt, int64_t ld_out,
                     float* dw_partials, int64_t n_partials, void* dw, int dw_dt,
                     int64_t rows, int64_t n, float eps, void* stream);

/*
 * esep_rmsnorm_bwd with a weight gradient, allocating nothing: the [P, n] fp32 partials live in a
 * scratch array inside the library (8 MiB of device memory on every GPU the library runs on,
 * held until the process ends), so the caller passes no workspace. No counterpart in the
 * reference; it is for callers that cannot allocate device memory (code under HIP graph
 * capture that may not call hipMalloc, tight serving loops, harnesses that forbid allocation).
 * Arguments are those of esep_rmsnorm_bwd without dw_partials / n_partials; dw is required.
 * Limit: esep_rmsnorm_partials(rows, n) * n <= 2^21 floats (config 4's 8192 x 1536 and config
 * 5's 65536 x 3584 fit), else ESEP_ESHAPE. The scratch array belongs to the device current on
 * the calling thread; its address is looked up there on the first call. A non-NULL stream on
 * another device is rejected with ESEP_EINVAL before anything is launched. Every call fully
 * writes the partials it then reads, but all calls on one GPU share the array: calls that can
 * overlap on one GPU (on different streams, or from threads that do not order their streams)
 * race and must not be issued.
 */
int esep_rmsnorm_bwd_noalloc(const void* const* dys, int n_dy, int dy_dt, int64_t ld_dy,
                             const float* dr_out,
                             const void* x, int x_dt, int64_t ld_x, int from_y,
                             const float* rstd,
                             const float* w,
                             const int32_t* slot, const float* xs, int n_special,
                             float* dr_f32, void* dx_lp, int dx_dt, int64_t ld_out,
                             void* dw, int dw_dt,
                             int64_t rows, int64_t n, float eps, void* stream);

/*
 * Stage 2 of the weight gradient on its own: dw[j] = sum_{p < n_partials} partials[p, j], summed
 * in an order that depends on n_partials only (bitwise equal to the stage 2 inside
 * esep_rmsnorm_bwd for the same partials). partials: fp32 [n_partials, n] contiguous and
 * 16-byte aligned (else ESEP_EALIGN);
 * n_partials == 0 writes zeros. No reference counterpart (the reference computes no weight
 * gradient: norm_rope.py:286 returns None for it); for callers that run stage 1 per micro-batch
 * or on several streams and reduce once.
 */
int esep_dgamma_reduce(const float* partials, int64_t n_partials, int64_t n, void* dw, int dw_dt,
                       void* stream);

/*
 * Stage 2 for several norms in one launch: for each item i, dw_i[j] = sum_p partials_i[p, j]
 * exactly as esep_dgamma_reduce computes it (bitwise the same dw_i). No reference counterpart
 * (the reference computes no weight gradient); for a training step whose norm-weight gradients
 * are read only after the backward sweep: the sweep's norm backwards write their partials
 * (dw == NULL, each its own buffer) and one launch reduces them all instead of one launch per
 * norm. All items share n and dw_dt; `items` is a host array of 1 .. ESEP_DGAMMA_BATCH_MAX
 * entries, read during the call (copied into the launch).
 */
#define ESEP_DGAMMA_BATCH_MAX 64
typedef struct {
  const float* partials; /* fp32 [n_partials, n] contiguous, 16-byte aligned (NULL only when
                            n_partials == 0) */
  int64_t n_partials;
  void* dw;              /* [n] of dw_dt */
} esep_dgamma_item;
int esep_dgamma_reduce_batch(const esep_dgamma_item* items, int n_items, int64_t n, int dw_dt,
                             void* stream);

/*
 * Rotary embedding on q and k in one launch (forward with sin_sign = +1, backward with -1).
 * Replaces the launch of _rope_kernel at solution/body/norm_rope.py:388-392 (_launch_rope);
 * kernel math follows norm_rope.py:330-369 (rotate_half convention of HF apply_rotary_pos_emb).
 *
 * Tokens are indexed (b, s) with b < B, s < S. Element (b, s, h, d) of a tensor X lives at
 * X + b*X_strides[0] + s*X_strides[1] + h*X_strides[2] + d. The packed reference layout
 * [T, H, D] is B = 1, S = T; HF's [B, H, S, D] view is any permutation of strides.
 *
 *   angle_j = float(pos) * inv_freq[j]          one fp32 multiply, j < D/2
 *   c = cos(angle), s = sin_sign * sin(angle)   computed in registers (no cos/sin table)
 *   x = q (+ q_delta, added in the storage dtype) | k
 *   out[:D/2] = x1*c - x2*s,  out[D/2:] = x2*c + x1*s
 *
 * Position source (exactly one):
 *   positions != NULL: pos = positions[b*pos_strides[0] + s*pos_strides[1]] (pos_dt I32/I64);
 *   cu_seqlens != NULL (B must be 1): pos = s - cu_seqlens[i] for cu_seqlens[i] <= s <
 *     cu_seqlens[i+1], i < n_seq (int32, cu_seqlens[0] == 0, cu_seqlens[n_seq] == S);
 *   both NULL: pos = s (HF's default arange positions per row).
 * inv_freq: fp32 [D/2] (the model's rotary inv_freq buffer). dt: F32, F16 or BF16 for all of
 * q, q_delta, k, q_out, k_out. D/2 must be 32, 64 or 128 (D = 64, 128, 256).
 */
int esep_rope(const void* q, const int64_t q_strides[3],
              const void* q_delta, const int64_t qd_strides[3],
              const void* k, const int64_t k_strides[3],
              void* q_out, const int64_t qo_strides[3],
              void* k_out, const int64_t ko_strides[3],
              int dt, int64_t B, int64_t S, int HQ, int HK, int D,
              const void* positions, int pos_dt, const int64_t pos_strides[2],
              const int32_t* cu_seqlens, int n_seq,
              const float* inv_freq, float sin_sign, void* stream);

/*
 * Varlen causal attention forward with grouped kv heads, over the packed token layout.
 * Replaces the per-row scaled_dot_product_attention loop of the reference decoder,
 * solution/body/packed.py:404-436 (_attention: per original row, is_causal=True,
 * scale=attn.scaling, query head h reads kv head h / (HQ / HK) as HF's repeat_kv).
 *
 *   q [T, HQ, D], k, v [T, HK, D], o [T, HQ, D]    dt (fp16 or bf16), heads of a token
 *                                                  contiguous, token strides q_rs ... o_rs
 *                                                  (multiples of 8, at most 2^22 elements)
 *   cu_seqlens int32 [n_seq + 1]                   sequence s is tokens [cu[s], cu[s+1]);
 *                                                  offsets are clamped into [0, T]
 *   max_seqlen >= every sequence length            (sizes the launch)
 *   o[t, h] = sum_{j in seq(t), j <= t} softmax_j(scale * q[t, h] . k[j, h']) v[j, h']
 *   lse [HQ, T] fp32 or NULL                       ln sum_j exp(scale * q . k), for the backward
 * Fully in fp32 inside (scores, softmax, accumulation); one rounding at the store of o.
 * No reference C counterpart: the reference calls torch's SDPA once per row.
 */
int esep_attn_fwd(const void* q, int64_t q_rs, const void* k, int64_t k_rs, const void* v,
                  int64_t v_rs, void* o, int64_t o_rs, float* lse, int dt, int64_t T, int HQ,
                  int HK, int D, const int32_t* cu_seqlens, int n_seq, int max_seqlen,
                  float scale, void* stream);

/*
 * Floats of fp32 workspace that esep_attn_bwd needs for this shape (depends on the shape only).
 * No reference counterpart (the reference's SDPA allocates inside torch).
 */
int64_t esep_attn_bwd_workspace(int64_t T, int HQ, int HK, int D);

/*
 * Backward of esep_attn_fwd (same layout and argument meanings), deterministic (no atomics).
 * Replaces the autograd backward of the reference's per-row SDPA calls (packed.py:428-429).
 *
 *   o, lse    the forward's output and its saved lse
 *   dout      [T, HQ, D] gradient of o
 *   workspace fp32, esep_attn_bwd_workspace(T, HQ, HK, D) floats, 16-byte aligned, caller-
 *             allocated (per-query rowsum(dout * o), then dK / dV partials when the query heads
 *             of a kv head are spread over several blocks to fill the GPU; written then read)
 *   dq [T, HQ, D], dk, dv [T, HK, D]   outputs in dt; dk and dv sum over the query heads of
 *                                      their group in a fixed order
 * Two kernels on the stream: dQ (and delta) per query tile, then dK and dV per key tile.
 */
int esep_attn_bwd(const void* q, int64_t q_rs, const void* k, int64_t k_rs, const void* v,
                  int64_t v_rs, const void* o, int64_t o_rs, const void* dout, int64_t do_rs,
                  const float* lse, float* workspace, void* dq, int64_t dq_rs, void* dk,
                  int64_t dk_rs, void* dv, int64_t dv_rs, int dt, int64_t T, int HQ, int HK,
                  int D, const int32_t* cu_seqlens, int n_seq, int max_seqlen, float scale,
                  void* stream);

/*
 * SwiGLU of the Qwen2 MLP, element-wise over n elements of one dtype (fp32 / fp16 / bf16),
 * contiguous, 16-byte aligned. Replaces the example kernels the reference decoder calls,
 * solution/swiglu.py:15-37 (example_swiglu_fwd_kernel / example_swiglu_bwd_kernel, launched at
 * swiglu.py:49-50, :59-60 and solution/body/packed.py:538, :558):
 *   s = sigmoid(gate) in fp32;  out = gate * s * up
 *   dup = dout * gate * s;  dgate = dout * up * s * (1 + gate * (1 - s))
 * out may alias gate; dgate may alias gate and dup may alias up (each element is read before it
 * is written), as the recompute MLP uses them.
 */
int esep_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dt,
                    void* stream);
int esep_swiglu_bwd(const void* dout, const void* gate, const void* up, void* dgate, void* dup,
                    int64_t n, int dt, void* stream);

/*
 * Dropout on the LoRA input with the mask regenerated from a key (LoRA path of q_proj / v_proj).
 * Replaces the reference's Triton launches at solution/body/lora.py:160-161
 * (lora_dropout_fwd_kernel in lora_dropout) and :180-182 (lora_dropout_bwd_kernel in
 * lora_down_bwd); kernel math follows lora.py:67-137.
 *   keep(e) = uniform(key, e) >= p     uniform: Philox4x32-10 (Salmon et al., SC 2011) at counter
 *                                      e / 4, word e % 4, (word >> 8) * 2^-24; key = *key (int64
 *                                      in device memory, e.g. drawn by torch's CUDA generator)
 *   fwd:  xd = x * keep / (1 - p)
 *   bwd:  xd = x * keep / (1 - p) (regenerated);  dx = [dx +] g * keep / (1 - p)  (accumulate)
 * x, xd, g, dx: n contiguous elements of dtype dt, 16-byte aligned; 0 < p < 1. dx may alias g.
 */
int esep_lora_dropout_fwd(const void* x, const int64_t* key, void* xd, int64_t n, float p, int dt,
                          void* stream);
int esep_lora_dropout_bwd(const void* x, const void* g, const int64_t* key, void* xd, void* dx,
                          int64_t n, float p, int accumulate, int dt, void* stream);

/*
 * NF4 double-quant weight dequantization (QLoRA / bitsandbytes Linear4bit format). Replaces the
 * reference's Triton launch at solution/nf4/dequant.py:85-89 (dequantize_nf4; kernel math
 * dequant.py:35-57):
 *   scale[b] = (code2[absmax[b]] * absmax2[b / 256]) + *offset     each op rounded in fp32
 *   out[e]   = nf4[nibble(e)] * scale[e / 64]                       rounded to out_dt once
 * packed: n_blocks * 32 bytes (byte i: element 2i in the high nibble, 2i + 1 in the low one),
 * 8-byte aligned; absmax uint8 [n_blocks]; absmax2 fp32 [ceil(n_blocks / 256)]; code2 fp32 [256];
 * offset: one fp32 in device memory; nf4 fp32 [16]; out: n_blocks * 64 elements of out_dt
 * (fp16 as the reference, also bf16 / fp32), 16-byte aligned.
 */
int esep_nf4_dequant(const void* packed, const uint8_t* absmax, const float* absmax2,
                     const float* code2, const float* offset, const float* nf4, void* out,
                     int out_dt, int64_t n_blocks, void* stream);

/*
 * Several NF4 weights in one launch. Replaces the reference's one-launch multi-weight kernel
 * (solution/nf4/dequant.py:129-166 nf4_dequant_multi_kernel, launched by dequantize_nf4_multi
 * :185-205, up to 3 weights into one W_cat): each weight decodes exactly as esep_nf4_dequant (bit
 * for bit) into its own `out` (slices of one W_cat, or separate buffers). `weights` is a host
 * array of 1 .. ESEP_NF4_MULTI_MAX entries, read during the call (copied into the launch).
 */
#define ESEP_NF4_MULTI_MAX 8
typedef struct {
  const void* packed;     /* n_blocks * 32 bytes, 8-byte aligned */
  const uint8_t* absmax;  /* [n_blocks] */
  const float* absmax2;   /* [ceil(n_blocks / 256)] */
  const float* code2;     /* [256] */
  const float* offset;    /* one fp32 in device memory */
  const float* nf4;       /* [16] */
  void* out;              /* n_blocks * 64 elements of out_dt, 16-byte aligned */
  int64_t n_blocks;
} esep_nf4_weight;
int esep_nf4_dequant_multi(const esep_nf4_weight* weights, int n_weights, int out_dt, void* stream);

/*
 * Fused LM head: softmax statistics and dlogits of one logits chunk. Replaces the reference's
 * Triton launch at solution/head/op.py:79-84 (_run; kernel head_row_softmax_kernel,
 * solution/head/kernels.py:37-93). For each row r of z ([rows, V] of dt, row stride ld):
 *   lse[r]    = log sum_v exp(z[r,v])                 (fp32, online over the row)
 *   ent[r]    = -sum_v p_v log p_v, p = softmax(z[r])  (as log S - T / S, no cancellation)
 *   amax[r]   = first v with z[r,v] = max_v z[r,v]     (int32)
 *   tlogit[r] = z[r, target[r]], or 0 when target[r] is outside [0, V)
 * and, when write_g and cew[r] != 0, z[r] is overwritten in place with
 *   g[r,v] = (p_v - [v == target[r]]) * g_scale        (rounded to dt)
 * dt: fp16 (the reference's) or bf16. target int64 [rows]; cew fp32 [rows] (read only when
 * write_g); 1 <= V <= 2^30; ld >= V. z, lse, tlogit, ent, amax may be any device pointers;
 * 16-byte aligned z with ld and V multiples of 8 takes the 16-byte-load path.
 */
int esep_head_row_softmax(void* z, int64_t ld, const int64_t* target, const float* cew,
                          float* lse, float* tlogit, float* ent, int32_t* amax, int64_t rows,
                          int64_t V, int write_g, float g_scale, int dt, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ESEP_BODY_H */

// The extern "C" boundary of libesep_body.so (declared in include/esep_body.h): argument
// checks, launch-shape selection, dispatch to the kernel templates. No allocation, no
// synchronization, no global mutable state except the per-thread error message.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "attention.hpp"
#include "dropout.hpp"
#include "esep_body.h"
#include "head.hpp"
#include "nf4.hpp"
#include "rmsnorm.hpp"
#include "rope.hpp"
#include "swiglu.hpp"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  snprintf(g_err, sizeof(g_err), "%s: %s", what, hipGetErrorString(e));
  return (int)e;
}

bool float_dt(int dt) { return dt == ESEP_F32 || dt == ESEP_F16 || dt == ESEP_BF16; }
int dt_bytes(int dt) { return dt == ESEP_F32 || dt == ESEP_I32 ? 4 : (dt == ESEP_I64 ? 8 : 2); }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool ld_ok(int64_t ld, int dt) { return ((ld * dt_bytes(dt)) & 15) == 0; }

// Row-group shape for n columns: the fewest wavefronts per row (wpr) that keep at most three
// 8-element chunks per lane, and the chunk count per lane for that wpr (at least 2: the
// smallest instantiated kernel). n <= 16384 gives wpr <= 11.
void norm_shape(int64_t n, int* wpr, int* nv) {
  const int64_t chunks = (n + 7) / 8;
  const int w = (int)((chunks + 3 * 64 - 1) / (3 * 64));
  const int v = (int)((chunks + 64 * w - 1) / (64 * w));
  *wpr = w < 1 ? 1 : w;
  *nv = v < 2 ? 2 : v;
}

// Threads per backward block with a weight gradient: 256 when a row is one wavefront (n <= 1536:
// four row groups, each lane summing its columns over 8 rows at config 4), else 512 (one or
// more groups of wpr wavefronts). Measured at config 4 (8192 x 1536, main kernel with its
// partials): 256 threads 15.6 us, 512 threads 16.0 us; P = 512 blocks of 256 threads 15.7 us.
int bwd_block_threads(int wpr) { return wpr == 1 ? 256 : 512; }
int bwd_groups(int wpr) {
  const int g = bwd_block_threads(wpr) / (64 * wpr);
  return g > 0 ? g : 1;
}

// LDS bytes of the backward's weight-gradient tree for gpb groups with NV chunks per lane:
// the most slots any tree level parks at once, each NV * 64 * wpr * 8 floats.
size_t bwd_tree_lds(int gpb, int nv, int wpr) {
  int top = 1;
  while (top < gpb) top <<= 1;
  int slots = 0;
  for (int half = top >> 1; half >= 1; half >>= 1) {
    const int hi = 2 * half < gpb ? 2 * half : gpb;
    if (hi - half > slots) slots = hi - half;
  }
  return (size_t)slots * (size_t)nv * 64 * (size_t)wpr * 8 * sizeof(float);
}

// Block count P of the backward pass with a weight gradient (= rows of the [P, n] partials):
// one block per gpb rows, at least 1, at most 256 (one block per CU, each row group taking
// several rows) or, from 2^26 elements on, 512 (two blocks per CU: at config 5 247 us against
// 297 with 256; at config 4 P = 512 costs 20.8 us against 19.2). Only (rows, n) enter, so the
// weight-gradient summation order is fixed for a shape.
int64_t bwd_partials(int64_t rows, int64_t n) {
  int wpr, nv;
  norm_shape(n, &wpr, &nv);
  const int64_t gpb = bwd_groups(wpr);
  const int64_t cap = rows * n >= (int64_t{1} << 26) ? 512 : 256;
  int64_t p = (rows + gpb - 1) / gpb;
  if (p > cap) p = cap;
  return p < 1 ? 1 : p;
}

// Blocks per (kv head, key tile) of the attention dK / dV kernel: split the kv head's query
// heads over more blocks, each writing fp32 partials, when one block per (kv head, 128-key tile)
// would leave the GPU short of work. The rule counts 256-token key spans per kv head and takes
// the smallest divisor s of HQ / HK with spans * s >= 384 (768 of the kernel's 128-key blocks,
// one and a half rounds of its two blocks per CU); it depends on the shape only. The partials
// cost traffic (at config 4 a 6-way split writes and re-reads 100 MB), but with the
// longest-first block order (xcd_order_lpt) the finer split balances better: config 4 backward
// 0.182 ms with split 3, 0.171 ms with 6.
int attn_split(int64_t T, int HQ, int HK) {
  const int G = HQ / HK;
  const int64_t blocks = ((T + 255) / 256) * HK;  // 256-token key spans
  int s = 1;
  while (blocks * s < 384 && s < G) {
    ++s;
    while (G % s) ++s;
  }
  return s;
}

}  // namespace

extern "C" {

int esep_abi_version(void) { return ESEP_ABI_VERSION; }

const char* esep_last_error(void) { return g_err; }

int esep_rmsnorm_fwd(const void* x, int x_dt, int64_t ld_x, const void* delta, int delta_dt,
                     int64_t ld_delta, const float* w, void* r_out, int64_t ld_r, void* y, int y_dt,
                     int64_t ld_y, float* rstd, const int32_t* slot, float* xs, int n_special,
                     int64_t rows, int64_t n, float eps, void* stream) {
  g_err[0] = 0;
  if (n < 1 || n > ESEP_NORM_MAX_COLS)
    return fail(ESEP_ESHAPE, "rmsnorm_fwd: n=%lld outside [1, %d]", (long long)n, ESEP_NORM_MAX_COLS);
  if (rows < 0) return fail(ESEP_ESHAPE, "rmsnorm_fwd: rows=%lld < 0", (long long)rows);
  if (!float_dt(x_dt) || !float_dt(y_dt) || (delta != nullptr && !float_dt(delta_dt)))
    return fail(ESEP_EINVAL, "rmsnorm_fwd: bad dtype code");
  if (x == nullptr || y == nullptr || w == nullptr)
    return fail(ESEP_EINVAL, "rmsnorm_fwd: x, y and w are required");
  if (n_special < 0 || (n_special > 0 && (slot == nullptr || xs == nullptr)))
    return fail(ESEP_EINVAL, "rmsnorm_fwd: n_special > 0 needs slot and xs");
  if (ld_x < n || ld_y < n || (delta && ld_delta < n) || (delta && r_out && ld_r < n))
    return fail(ESEP_ESHAPE, "rmsnorm_fwd: leading dimension smaller than n");
  if (rows == 0) return 0;

  esep::FwdArgs a{};
  a.x = x;
  a.delta = delta;
  a.w = w;
  a.r_out = delta ? r_out : nullptr;
  a.y = y;
  a.rstd = rstd;
  a.slot = slot;
  a.xs = xs;
  a.ld_x = ld_x;
  a.ld_d = ld_delta;
  a.ld_r = ld_r;
  a.ld_y = ld_y;
  a.rows = rows;
  a.n = (int)n;
  a.n_special = n_special;
  a.eps = eps;
  int wpr, nv;
  norm_shape(n, &wpr, &nv);
  a.wpr = wpr;
  bool vec = (n % 8) == 0 && aligned16(x) && aligned16(y) && aligned16(w) && ld_ok(ld_x, x_dt) &&
             ld_ok(ld_y, y_dt);
  if (delta) vec = vec && aligned16(delta) && ld_ok(ld_delta, delta_dt);
  if (a.r_out) vec = vec && aligned16(r_out) && ld_ok(ld_r, x_dt);
  if (n_special > 0) vec = vec && aligned16(slot);
  a.vec = vec ? 1 : 0;

  const int gpb = wpr >= 4 ? 1 : 4 / wpr;
  a.gpb = gpb;
  const dim3 block(gpb * 64 * wpr);
  const int64_t blocks = (rows + gpb - 1) / gpb;
  if (blocks > 0x7fffffff) return fail(ESEP_ESHAPE, "rmsnorm_fwd: too many rows");
  bool sup = false;
  const hipError_t e = esep::launch_rmsnorm_fwd(a, x_dt, delta ? delta_dt : -1, y_dt, nv,
                                                dim3((unsigned)blocks), block,
                                                static_cast<hipStream_t>(stream), &sup);
  if (!sup)
    return fail(ESEP_EINVAL, "rmsnorm_fwd: unsupported dtypes x=%d delta=%d y=%d", x_dt,
                delta ? delta_dt : -1, y_dt);
  if (e != hipSuccess) return hip_fail(e, "rmsnorm_fwd launch");
  return 0;
}

int64_t esep_rmsnorm_partials(int64_t rows, int64_t n) {
  if (rows <= 0 || n < 1 || n > ESEP_NORM_MAX_COLS) return 0;
  return bwd_partials(rows, n);
}

int esep_rmsnorm_bwd(const void* const* dys, int n_dy, int dy_dt, int64_t ld_dy,
                     const float* dr_out, const void* x, int x_dt, int64_t ld_x, int from_y,
                     const float* rstd, const float* w, const int32_t* slot, const float* xs,
                     int n_special, float* dr_f32, void* dx_lp, int dx_dt, int64_t ld_out,
                     float* dw_partials, int64_t n_partials, void* dw, int dw_dt, int64_t rows,
                     int64_t n, float eps, void* stream) {
  g_err[0] = 0;
  if (n < 1 || n > ESEP_NORM_MAX_COLS)
    return fail(ESEP_ESHAPE, "rmsnorm_bwd: n=%lld outside [1, %d]", (long long)n, ESEP_NORM_MAX_COLS);
  if (rows < 0) return fail(ESEP_ESHAPE, "rmsnorm_bwd: rows=%lld < 0", (long long)rows);
  if (n_dy < 0 || n_dy > ESEP_MAX_DY)
    return fail(ESEP_EINVAL, "rmsnorm_bwd: n_dy=%d outside [0, %d]", n_dy, ESEP_MAX_DY);
  if (n_dy > 0 && (dys == nullptr || !float_dt(dy_dt)))
    return fail(ESEP_EINVAL, "rmsnorm_bwd: dys / dy dtype");
  for (int i = 0; i < n_dy; ++i)
    if (dys[i] == nullptr) return fail(ESEP_EINVAL, "rmsnorm_bwd: dys[%d] is NULL", i);
  if (n_dy > 0 && (x == nullptr || !float_dt(x_dt) || w == nullptr))
    return fail(ESEP_EINVAL, "rmsnorm_bwd: x, x dtype and w are required");
  if (from_y && rstd == nullptr)
    return fail(ESEP_EINVAL, "rmsnorm_bwd: from_y needs the saved rstd");
  if (n_special < 0 || (n_special > 0 && (!from_y || slot == nullptr || xs == nullptr)))
    return fail(ESEP_EINVAL, "rmsnorm_bwd: n_special > 0 needs from_y, slot and xs");
  if (dx_lp != nullptr && !float_dt(dx_dt)) return fail(ESEP_EINVAL, "rmsnorm_bwd: dx dtype");
  if (dw != nullptr && (!float_dt(dw_dt) || dw_partials == nullptr))
    return fail(ESEP_EINVAL, "rmsnorm_bwd: dw needs dw_partials and a float dtype");
  if (dw_partials != nullptr) {
    if (!aligned16(dw_partials))
      return fail(ESEP_EALIGN, "rmsnorm_bwd: dw_partials must be 16-byte aligned");
    const int64_t want = esep_rmsnorm_partials(rows, n);
    if (rows > 0 && n_partials != want)
      return fail(ESEP_ESHAPE, "rmsnorm_bwd: n_partials=%lld, this shape needs %lld",
                  (long long)n_partials, (long long)want);
  }
  if ((n_dy > 0 && (ld_dy < n || ld_x < n)) ||
      ((dr_out || dr_f32 || dx_lp) && ld_out < n))
    return fail(ESEP_ESHAPE, "rmsnorm_bwd: leading dimension smaller than n");
  if (rows == 0) {  // no rows: dw is the empty sum, 0
    if (dw == nullptr) return 0;
    bool sup = false;
    const hipError_t e = esep::launch_dgamma_reduce(dw_partials, 0, (int)n, dw, dw_dt,
                                                    static_cast<hipStream_t>(stream), &sup);
    return e == hipSuccess ? 0 : hip_fail(e, "rmsnorm_bwd dw reduce launch");
  }
  // Stage 1 (weight-gradient partials) runs when a workspace is given: with dw, stage 2
  // follows here; without, the caller reduces later (esep_dgamma_reduce).
  const bool part = dw_partials != nullptr;

  esep::BwdArgs a{};
  for (int i = 0; i < n_dy; ++i) a.dy[i] = dys[i];
  a.n_dy = n_dy;
  a.ld_dy = ld_dy;
  a.dr_out = dr_out;
  a.x = x;
  a.ld_x = ld_x;
  a.from_y = from_y ? 1 : 0;
  a.rstd = rstd;
  a.w = w;
  a.slot = slot;
  a.xs = xs;
  a.n_special = n_special;
  a.dr = dr_f32;
  a.dx = dx_lp;
  a.ld_out = ld_out;
  a.part = part ? dw_partials : nullptr;
  a.rows = rows;
  a.n = (int)n;
  a.eps = eps;
  int wpr, nv;
  norm_shape(n, &wpr, &nv);
  a.wpr = wpr;
  // Without a weight gradient: blocks of 4 row groups of one wavefront (or one group of wpr
  // wavefronts).
  const int gpb = part ? bwd_groups(wpr) : (wpr >= 4 ? 1 : 4 / wpr);
  a.gpb = gpb;

  const int xdt = n_dy > 0 ? x_dt : ESEP_F32;
  const int dydt = n_dy > 0 ? dy_dt : xdt;
  const int odt = dx_lp ? dx_dt : ESEP_F32;
  bool vec = (n % 8) == 0 && aligned16(w);
  for (int i = 0; i < n_dy; ++i) vec = vec && aligned16(dys[i]);
  if (n_dy > 0) vec = vec && ld_ok(ld_dy, dy_dt) && aligned16(x) && ld_ok(ld_x, x_dt);
  if (dr_out) vec = vec && aligned16(dr_out);
  if (dr_f32) vec = vec && aligned16(dr_f32);
  if (dx_lp) vec = vec && aligned16(dx_lp) && ld_ok(ld_out, dx_dt);
  if (dr_out || dr_f32) vec = vec && ld_ok(ld_out, ESEP_F32);
  if (n_special > 0) vec = vec && aligned16(slot);
  a.vec = vec ? 1 : 0;

  // The fast kernels (vector rows, one dy, xhat from x, no dr_out). Rows of one wavefront
  // (n <= 1536) run the pipelined kernel, grid-strided over at most 256 blocks of 4 wavefronts
  // without a weight gradient too (one wavefront per SIMD; config 4: 8 rows each, 14.3 us,
  // against 14.7 us on 512 blocks). Wider rows run the wide kernel, one row per group.
  const int threads = gpb * 64 * wpr;
  const bool plain = vec && n_dy == 1 && !from_y && dr_out == nullptr && n_special == 0;
  int64_t blocks = part ? bwd_partials(rows, n) : (rows + gpb - 1) / gpb;
  // The pipelined kernel's grid: the partials' P blocks, or at most 256 without them. It takes at
  // most 64 rows per row group (one saved-rstd vector load); longer runs go to the wide kernel,
  // whose grid-strided rows and fixed-order block sums give the same partials bit for bit.
  const int64_t pipe_blocks = (!part && blocks > 256) ? 256 : blocks;
  const int64_t rows_per_group = (rows + pipe_blocks * gpb - 1) / (pipe_blocks * gpb);
  a.fast = 0;
  if (plain && wpr == 1 && threads == esep::kBwdPipeThreads && rows_per_group <= 64) {
    a.fast = 1;
    blocks = pipe_blocks;
  } else if (plain) {
    a.fast = 2;
  }
  if (blocks > 0x7fffffff) return fail(ESEP_ESHAPE, "rmsnorm_bwd: too many rows");
  // LDS. The pipelined kernel keeps, with a weight gradient, one slot of nv * 64 * 8 floats per
  // row group for the block sum (4 groups: 24 KiB). The wide kernel also stages the weight
  // vector in one slot of nv * 64 * wpr * 8 floats (at most (8 + 1) * 3 * 2 KiB per wpr). The
  // general kernel parks at most bwd_tree_lds slots at once (it always runs NV = 3 element-wise).
  const size_t slot_bytes = (size_t)nv * 64 * wpr * 8 * sizeof(float);
  size_t lds = 0;
  if (a.fast == 1)
    lds = part ? (size_t)gpb * slot_bytes : 0;
  else if (a.fast == 2)
    lds = (part ? (size_t)gpb + 1 : 1) * slot_bytes;
  else if (part)
    lds = bwd_tree_lds(gpb, vec ? nv : 3, wpr);
  bool sup = false;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e = esep::launch_rmsnorm_bwd(a, xdt, dydt, odt, nv, dim3((unsigned)blocks),
                                          dim3(threads), lds, s, &sup);
  if (!sup)
    return fail(ESEP_EINVAL, "rmsnorm_bwd: unsupported dtypes x=%d dy=%d dx=%d", xdt, dydt, odt);
  if (e != hipSuccess) return hip_fail(e, "rmsnorm_bwd launch");
  if (dw) {
    e = esep::launch_dgamma_reduce(dw_partials, blocks, (int)n, dw, dw_dt, s, &sup);
    if (e != hipSuccess) return hip_fail(e, "rmsnorm_bwd dw reduce launch");
  }
  return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------------------
// Weight-gradient partials of esep_rmsnorm_bwd_noalloc: a file-scope device array (every GPU
// the library runs on holds its own copy until the process ends). Host code never passes the
// array's name to a kernel: that is a host-side stand-in, not a device address. Its address on
// each device is looked up once, with that device current, and kept in g_scratch_ptr.
// ---------------------------------------------------------------------------------------
namespace {

constexpr int64_t kScratchFloats = int64_t{2} << 20;  // 8 MiB of fp32 partials per GPU
constexpr int kScratchDevices = 64;
static __device__ __align__(256) float scratch[kScratchFloats];
std::mutex g_scratch_lock;
float* g_scratch_ptr[kScratchDevices] = {};

// The scratch array's device address on the current device (looked up on first use there).
int scratch_on_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "rmsnorm_bwd_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kScratchDevices)
    return fail(ESEP_EINVAL, "rmsnorm_bwd_noalloc: device %d outside [0, %d)", dev, kScratchDevices);
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol,
                      "rmsnorm_bwd_noalloc: hipGetSymbolAddress(scratch)");
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace

extern "C" {

int esep_rmsnorm_bwd_noalloc(const void* const* dys, int n_dy, int dy_dt, int64_t ld_dy,
                             const float* dr_out, const void* x, int x_dt, int64_t ld_x,
                             int from_y, const float* rstd, const float* w, const int32_t* slot,
                             const float* xs, int n_special, float* dr_f32, void* dx_lp,
                             int dx_dt, int64_t ld_out, void* dw, int dw_dt, int64_t rows,
                             int64_t n, float eps, void* stream) {
  g_err[0] = 0;
  if (dw == nullptr)
    return fail(ESEP_EINVAL, "rmsnorm_bwd_noalloc: dw is required (without a weight gradient "
                "esep_rmsnorm_bwd needs no workspace)");
  if (n < 1 || n > ESEP_NORM_MAX_COLS || rows < 0)
    return fail(ESEP_ESHAPE, "rmsnorm_bwd_noalloc: rows=%lld, n=%lld", (long long)rows, (long long)n);
  const int64_t P = bwd_partials(rows, n);
  if (P * n > kScratchFloats)
    return fail(ESEP_ESHAPE, "rmsnorm_bwd_noalloc: %lld x %lld partials exceed the %lld-float "
                "scratch (use esep_rmsnorm_bwd with a workspace)", (long long)P, (long long)n,
                (long long)kScratchFloats);
  // the scratch array is the current device's: a stream of another device would run the
  // kernels there against an address that is not valid on it
  if (stream != nullptr) {
    int cur = -1;
    hipDevice_t sdev = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(e, "rmsnorm_bwd_noalloc: hipGetDevice");
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return hip_fail(e, "rmsnorm_bwd_noalloc: hipStreamGetDevice");
    if (sdev != cur)
      return fail(ESEP_EINVAL, "rmsnorm_bwd_noalloc: the stream is on device %d, the current "
                  "device is %d (make the stream's device current first)", (int)sdev, cur);
  }
  float* part = nullptr;
  const int rc = scratch_on_current_device(&part);
  if (rc != 0) return rc;
  return esep_rmsnorm_bwd(dys, n_dy, dy_dt, ld_dy, dr_out, x, x_dt, ld_x, from_y, rstd, w, slot,
                          xs, n_special, dr_f32, dx_lp, dx_dt, ld_out, part, rows > 0 ? P : 0,
                          dw, dw_dt, rows, n, eps, stream);
}

int esep_dgamma_reduce(const float* partials, int64_t n_partials, int64_t n, void* dw, int dw_dt,
                       void* stream) {
  g_err[0] = 0;
  if (n < 1 || n > ESEP_NORM_MAX_COLS)
    return fail(ESEP_ESHAPE, "dgamma_reduce: n=%lld outside [1, %d]", (long long)n, ESEP_NORM_MAX_COLS);
  if (n_partials < 0) return fail(ESEP_ESHAPE, "dgamma_reduce: n_partials < 0");
  if (dw == nullptr || !float_dt(dw_dt) || (n_partials > 0 && partials == nullptr))
    return fail(ESEP_EINVAL, "dgamma_reduce: dw, its float dtype and the partials are required");
  if (n_partials > 0 && !aligned16(partials))
    return fail(ESEP_EALIGN, "dgamma_reduce: partials must be 16-byte aligned");
  bool sup = false;
  const hipError_t e = esep::launch_dgamma_reduce(partials, n_partials, (int)n, dw, dw_dt,
                                                  static_cast<hipStream_t>(stream), &sup);
  return e == hipSuccess ? 0 : hip_fail(e, "dgamma_reduce launch");
}

int esep_dgamma_reduce_batch(const esep_dgamma_item* items, int n_items, int64_t n, int dw_dt,
                             void* stream) {
  g_err[0] = 0;
  static_assert(ESEP_DGAMMA_BATCH_MAX == esep::kDgammaBatchMax, "batch limit mismatch");
  if (items == nullptr || n_items < 1 || n_items > ESEP_DGAMMA_BATCH_MAX)
    return fail(ESEP_EINVAL, "dgamma_reduce_batch: n_items=%d outside [1, %d] or no items",
                n_items, ESEP_DGAMMA_BATCH_MAX);
  if (n < 1 || n > ESEP_NORM_MAX_COLS)
    return fail(ESEP_ESHAPE, "dgamma_reduce_batch: n=%lld outside [1, %d]", (long long)n,
                ESEP_NORM_MAX_COLS);
  if (!float_dt(dw_dt)) return fail(ESEP_EINVAL, "dgamma_reduce_batch: dw needs a float dtype");
  esep::DgammaBatch b = {};
  for (int i = 0; i < n_items; ++i) {
    const esep_dgamma_item& it = items[i];
    if (it.n_partials < 0)
      return fail(ESEP_ESHAPE, "dgamma_reduce_batch: item %d has n_partials < 0", i);
    if (it.dw == nullptr || (it.n_partials > 0 && it.partials == nullptr))
      return fail(ESEP_EINVAL, "dgamma_reduce_batch: item %d needs dw and its partials", i);
    if (it.n_partials > 0 && !aligned16(it.partials))
      return fail(ESEP_EALIGN, "dgamma_reduce_batch: item %d's partials are not 16-byte aligned", i);
    b.part[i] = it.partials;
    b.P[i] = it.n_partials;
    b.dw[i] = it.dw;
  }
  bool sup = false;
  const hipError_t e = esep::launch_dgamma_reduce_batch(b, n_items, (int)n, dw_dt,
                                                        static_cast<hipStream_t>(stream), &sup);
  return e == hipSuccess ? 0 : hip_fail(e, "dgamma_reduce_batch launch");
}

int esep_rope(const void* q, const int64_t q_strides[3], const void* q_delta,
              const int64_t qd_strides[3], const void* k, const int64_t k_strides[3], void* q_out,
              const int64_t qo_strides[3], void* k_out, const int64_t ko_strides[3], int dt,
              int64_t B, int64_t S, int HQ, int HK, int D, const void* positions, int pos_dt,
              const int64_t pos_strides[2], const int32_t* cu_seqlens, int n_seq,
              const float* inv_freq, float sin_sign, void* stream) {
  g_err[0] = 0;
  if (!float_dt(dt)) return fail(ESEP_EINVAL, "rope: bad dtype code %d", dt);
  if (D != 64 && D != 128 && D != 256) return fail(ESEP_ESHAPE, "rope: D=%d not in {64,128,256}", D);
  if (B < 0 || S < 0 || HQ < 0 || HK < 0 || HQ + HK < 1)
    return fail(ESEP_ESHAPE, "rope: bad sizes B=%lld S=%lld HQ=%d HK=%d", (long long)B,
                (long long)S, HQ, HK);
  if ((HQ > 0 && (q == nullptr || q_out == nullptr || q_strides == nullptr || qo_strides == nullptr)) ||
      (HK > 0 && (k == nullptr || k_out == nullptr || k_strides == nullptr || ko_strides == nullptr)))
    return fail(ESEP_EINVAL, "rope: q/q_out (k/k_out) and their strides are required");
  if (q_delta != nullptr && (HQ == 0 || qd_strides == nullptr))
    return fail(ESEP_EINVAL, "rope: q_delta needs q heads and strides");
  if (inv_freq == nullptr) return fail(ESEP_EINVAL, "rope: inv_freq is required");
  if (positions != nullptr && cu_seqlens != nullptr)
    return fail(ESEP_EINVAL, "rope: give positions or cu_seqlens, not both");
  if (positions != nullptr && ((pos_dt != ESEP_I32 && pos_dt != ESEP_I64) || pos_strides == nullptr))
    return fail(ESEP_EINVAL, "rope: positions need an int32/int64 dtype and strides");
  if (cu_seqlens != nullptr && (B != 1 || n_seq < 1))
    return fail(ESEP_EINVAL, "rope: cu_seqlens needs B == 1 and n_seq >= 1");
  const int64_t tokens = B * S;
  if (tokens == 0) return 0;
  if ((tokens + 3) / 4 > 0x7fffffff) return fail(ESEP_ESHAPE, "rope: too many tokens");

  esep::RopeArgs a{};
  const int64_t zero[3] = {0, 0, 0};
  const int64_t* qs = HQ > 0 ? q_strides : zero;
  const int64_t* qos = HQ > 0 ? qo_strides : zero;
  const int64_t* ks = HK > 0 ? k_strides : zero;
  const int64_t* kos = HK > 0 ? ko_strides : zero;
  const int64_t* qds = q_delta ? qd_strides : zero;
  for (int i = 0; i < 3; ++i) {
    a.q_s[i] = qs[i];
    a.qo_s[i] = qos[i];
    a.k_s[i] = ks[i];
    a.ko_s[i] = kos[i];
    a.qd_s[i] = qds[i];
  }
  a.q = q;
  a.qd = q_delta;
  a.k = k;
  a.qo = q_out;
  a.ko = k_out;
  a.B = B;
  a.S = S;
  a.HQ = HQ;
  a.HK = HK;
  a.pos = positions;
  a.pos_i64 = pos_dt == ESEP_I64 ? 1 : 0;
  a.pos_s[0] = positions ? pos_strides[0] : 0;
  a.pos_s[1] = positions ? pos_strides[1] : 0;
  a.cu = cu_seqlens;
  a.n_seq = n_seq;
  a.inv_freq = inv_freq;
  a.sign = sin_sign;
  bool vec = true;
  auto chk = [&](const void* p, const int64_t* st) {
    if (p == nullptr) return;
    vec = vec && aligned16(p);
    for (int i = 0; i < 3; ++i) vec = vec && ld_ok(st[i], dt);
  };
  if (HQ > 0) {
    chk(q, q_strides);
    chk(q_out, qo_strides);
    chk(q_delta, qd_strides);
  }
  if (HK > 0) {
    chk(k, k_strides);
    chk(k_out, ko_strides);
  }
  a.vec = vec ? 1 : 0;
  bool sup = false;
  const hipError_t e = esep::launch_rope(a, dt, D / 2, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "rope: unsupported dtype %d / D %d", dt, D);
  if (e != hipSuccess) return hip_fail(e, "rope launch");
  return 0;
}

// Token strides of the attention tensors, in elements, at most 2^22 (8 MiB of 16-bit
// elements): the LDS-DMA tile fills address a wavefront's rows with 32-bit per-lane byte
// offsets of up to 20 strides from an SGPR base.
constexpr int64_t kAttnMaxStride = int64_t{1} << 22;

int esep_attn_fwd(const void* q, int64_t q_rs, const void* k, int64_t k_rs, const void* v,
                  int64_t v_rs, void* o, int64_t o_rs, float* lse, int dt, int64_t T, int HQ,
                  int HK, int D, const int32_t* cu_seqlens, int n_seq, int max_seqlen,
                  float scale, void* stream) {
  g_err[0] = 0;
  if (dt != ESEP_F16 && dt != ESEP_BF16)
    return fail(ESEP_EINVAL, "attn_fwd: dtype %d is not fp16 / bf16", dt);
  if (D != 64 && D != 128) return fail(ESEP_ESHAPE, "attn_fwd: D=%d not in {64, 128}", D);
  if (T < 0 || T > 0x7fffffff || HQ < 1 || HK < 1 || HQ % HK != 0 || n_seq < 0 || max_seqlen < 0)
    return fail(ESEP_ESHAPE, "attn_fwd: bad sizes T=%lld HQ=%d HK=%d n_seq=%d max_seqlen=%d",
                (long long)T, HQ, HK, n_seq, max_seqlen);
  if (q_rs < (int64_t)HQ * D || o_rs < (int64_t)HQ * D || k_rs < (int64_t)HK * D ||
      v_rs < (int64_t)HK * D)
    return fail(ESEP_ESHAPE, "attn_fwd: token stride smaller than heads * D");
  if (q_rs > kAttnMaxStride || o_rs > kAttnMaxStride || k_rs > kAttnMaxStride ||
      v_rs > kAttnMaxStride)
    return fail(ESEP_ESHAPE, "attn_fwd: token stride above %lld elements", (long long)kAttnMaxStride);
  if (T == 0 || n_seq == 0 || max_seqlen == 0) return 0;
  if (q == nullptr || k == nullptr || v == nullptr || o == nullptr || cu_seqlens == nullptr)
    return fail(ESEP_EINVAL, "attn_fwd: q, k, v, o and cu_seqlens are required");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || (q_rs & 7) ||
      (k_rs & 7) || (v_rs & 7) || (o_rs & 7))
    return fail(ESEP_EALIGN, "attn_fwd: q, k, v, o need 16-byte alignment and token strides "
                             "that are multiples of 8 elements");
  if (!(scale > 0.f)) return fail(ESEP_EINVAL, "attn_fwd: scale must be positive");
  esep::AttnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.o = o;
  a.lse = lse;
  a.cu = cu_seqlens;
  a.q_rs = q_rs;
  a.k_rs = k_rs;
  a.v_rs = v_rs;
  a.o_rs = o_rs;
  a.T = T;
  a.n_seq = n_seq;
  a.HQ = HQ;
  a.HK = HK;
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  bool sup = false;
  const hipError_t e = esep::launch_attn_fwd(a, dt, D, max_seqlen, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "attn_fwd: unsupported dtype / D");
  return e == hipSuccess ? 0 : hip_fail(e, "attn_fwd launch");
}

int64_t esep_attn_bwd_workspace(int64_t T, int HQ, int HK, int D) {
  if (T <= 0 || HQ < 1 || HK < 1 || HQ % HK != 0 || D < 1) return 0;
  const int s = attn_split(T, HQ, HK);
  const int64_t delta = ((int64_t)HQ * T + 3) & ~(int64_t)3;  // keeps the partials 16-byte aligned
  return delta + (s > 1 ? 2 * (int64_t)s * T * HK * D : 0);
}

int esep_attn_bwd(const void* q, int64_t q_rs, const void* k, int64_t k_rs, const void* v,
                  int64_t v_rs, const void* o, int64_t o_rs, const void* dout, int64_t do_rs,
                  const float* lse, float* workspace, void* dq, int64_t dq_rs, void* dk,
                  int64_t dk_rs, void* dv, int64_t dv_rs, int dt, int64_t T, int HQ, int HK,
                  int D, const int32_t* cu_seqlens, int n_seq, int max_seqlen, float scale,
                  void* stream) {
  g_err[0] = 0;
  if (dt != ESEP_F16 && dt != ESEP_BF16)
    return fail(ESEP_EINVAL, "attn_bwd: dtype %d is not fp16 / bf16", dt);
  if (D != 64 && D != 128) return fail(ESEP_ESHAPE, "attn_bwd: D=%d not in {64, 128}", D);
  if (T < 0 || T > 0x7fffffff || HQ < 1 || HK < 1 || HQ % HK != 0 || n_seq < 0 || max_seqlen < 0)
    return fail(ESEP_ESHAPE, "attn_bwd: bad sizes T=%lld HQ=%d HK=%d n_seq=%d max_seqlen=%d",
                (long long)T, HQ, HK, n_seq, max_seqlen);
  const int64_t wq = (int64_t)HQ * D, wk = (int64_t)HK * D;
  if (q_rs < wq || o_rs < wq || do_rs < wq || dq_rs < wq || k_rs < wk || v_rs < wk ||
      dk_rs < wk || dv_rs < wk)
    return fail(ESEP_ESHAPE, "attn_bwd: token stride smaller than heads * D");
  for (int64_t rs : {q_rs, o_rs, do_rs, dq_rs, k_rs, v_rs, dk_rs, dv_rs})
    if (rs > kAttnMaxStride)
      return fail(ESEP_ESHAPE, "attn_bwd: token stride above %lld elements",
                  (long long)kAttnMaxStride);
  if (T == 0 || n_seq == 0 || max_seqlen == 0) return 0;
  const void* ptrs[] = {q, k, v, o, dout, dq, dk, dv};
  for (const void* p : ptrs)
    if (p == nullptr) return fail(ESEP_EINVAL, "attn_bwd: q, k, v, o, dout, dq, dk, dv are required");
  if (lse == nullptr || workspace == nullptr || cu_seqlens == nullptr)
    return fail(ESEP_EINVAL, "attn_bwd: lse, the workspace and cu_seqlens are required");
  if (!aligned16(workspace)) return fail(ESEP_EALIGN, "attn_bwd: workspace needs 16-byte alignment");
  const int64_t rss[] = {q_rs, k_rs, v_rs, o_rs, do_rs, dq_rs, dk_rs, dv_rs};
  for (int i = 0; i < 8; ++i)
    if (!aligned16(ptrs[i]) || (rss[i] & 7))
      return fail(ESEP_EALIGN, "attn_bwd: tensors need 16-byte alignment and token strides "
                               "that are multiples of 8 elements");
  if (!(scale > 0.f)) return fail(ESEP_EINVAL, "attn_bwd: scale must be positive");
  esep::AttnBwdArgs b{};
  b.f.q = q;
  b.f.k = k;
  b.f.v = v;
  b.f.o = const_cast<void*>(o);
  b.f.lse = const_cast<float*>(lse);
  b.f.cu = cu_seqlens;
  b.f.q_rs = q_rs;
  b.f.k_rs = k_rs;
  b.f.v_rs = v_rs;
  b.f.o_rs = o_rs;
  b.f.T = T;
  b.f.n_seq = n_seq;
  b.f.HQ = HQ;
  b.f.HK = HK;
  b.f.scale = scale;
  b.f.scale_log2 = scale * 1.4426950408889634f;
  b.dout = dout;
  b.delta = workspace;
  b.split = attn_split(T, HQ, HK);
  b.part = workspace + (((int64_t)HQ * T + 3) & ~(int64_t)3);
  b.dq = dq;
  b.dk = dk;
  b.dv = dv;
  b.do_rs = do_rs;
  b.dq_rs = dq_rs;
  b.dk_rs = dk_rs;
  b.dv_rs = dv_rs;
  bool sup = false;
  const hipError_t e = esep::launch_attn_bwd(b, dt, D, max_seqlen, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "attn_bwd: unsupported dtype / D");
  return e == hipSuccess ? 0 : hip_fail(e, "attn_bwd launch");
}

int esep_swiglu_fwd(const void* gate, const void* up, void* out, int64_t n, int dt,
                    void* stream) {
  g_err[0] = 0;
  if (!float_dt(dt)) return fail(ESEP_EINVAL, "swiglu_fwd: bad dtype code %d", dt);
  if (n < 0) return fail(ESEP_ESHAPE, "swiglu_fwd: n=%lld < 0", (long long)n);
  if (n == 0) return 0;
  if (gate == nullptr || up == nullptr || out == nullptr)
    return fail(ESEP_EINVAL, "swiglu_fwd: gate, up and out are required");
  if (!aligned16(gate) || !aligned16(up) || !aligned16(out))
    return fail(ESEP_EALIGN, "swiglu_fwd: tensors need 16-byte alignment");
  bool sup = false;
  const hipError_t e = esep::launch_swiglu_fwd(gate, up, out, n, dt, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "swiglu_fwd: unsupported dtype");
  return e == hipSuccess ? 0 : hip_fail(e, "swiglu_fwd launch");
}

int esep_swiglu_bwd(const void* dout, const void* gate, const void* up, void* dgate, void* dup,
                    int64_t n, int dt, void* stream) {
  g_err[0] = 0;
  if (!float_dt(dt)) return fail(ESEP_EINVAL, "swiglu_bwd: bad dtype code %d", dt);
  if (n < 0) return fail(ESEP_ESHAPE, "swiglu_bwd: n=%lld < 0", (long long)n);
  if (n == 0) return 0;
  if (dout == nullptr || gate == nullptr || up == nullptr || dgate == nullptr || dup == nullptr)
    return fail(ESEP_EINVAL, "swiglu_bwd: dout, gate, up, dgate and dup are required");
  if (!aligned16(dout) || !aligned16(gate) || !aligned16(up) || !aligned16(dgate) || !aligned16(dup))
    return fail(ESEP_EALIGN, "swiglu_bwd: tensors need 16-byte alignment");
  if (dgate == dup) return fail(ESEP_EINVAL, "swiglu_bwd: dgate and dup must not alias");
  bool sup = false;
  const hipError_t e = esep::launch_swiglu_bwd(dout, gate, up, dgate, dup, n, dt,
                                               static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "swiglu_bwd: unsupported dtype");
  return e == hipSuccess ? 0 : hip_fail(e, "swiglu_bwd launch");
}

int esep_lora_dropout_fwd(const void* x, const int64_t* key, void* xd, int64_t n, float p, int dt,
                          void* stream) {
  g_err[0] = 0;
  if (!float_dt(dt)) return fail(ESEP_EINVAL, "lora_dropout_fwd: bad dtype code %d", dt);
  if (n < 0) return fail(ESEP_ESHAPE, "lora_dropout_fwd: n=%lld < 0", (long long)n);
  if (!(p > 0.f && p < 1.f)) return fail(ESEP_EINVAL, "lora_dropout_fwd: p must be in (0, 1)");
  if (n == 0) return 0;
  if (x == nullptr || key == nullptr || xd == nullptr)
    return fail(ESEP_EINVAL, "lora_dropout_fwd: x, key and xd are required");
  if (!aligned16(x) || !aligned16(xd) || (reinterpret_cast<uintptr_t>(key) & 7))
    return fail(ESEP_EALIGN, "lora_dropout_fwd: x, xd need 16-byte and key 8-byte alignment");
  bool sup = false;
  const hipError_t e = esep::launch_dropout_fwd(x, key, xd, n, p, dt, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "lora_dropout_fwd: unsupported dtype");
  return e == hipSuccess ? 0 : hip_fail(e, "lora_dropout_fwd launch");
}

int esep_lora_dropout_bwd(const void* x, const void* g, const int64_t* key, void* xd, void* dx,
                          int64_t n, float p, int accumulate, int dt, void* stream) {
  g_err[0] = 0;
  if (!float_dt(dt)) return fail(ESEP_EINVAL, "lora_dropout_bwd: bad dtype code %d", dt);
  if (n < 0) return fail(ESEP_ESHAPE, "lora_dropout_bwd: n=%lld < 0", (long long)n);
  if (!(p > 0.f && p < 1.f)) return fail(ESEP_EINVAL, "lora_dropout_bwd: p must be in (0, 1)");
  if (n == 0) return 0;
  if (x == nullptr || g == nullptr || key == nullptr || xd == nullptr || dx == nullptr)
    return fail(ESEP_EINVAL, "lora_dropout_bwd: x, g, key, xd and dx are required");
  if (!aligned16(x) || !aligned16(g) || !aligned16(xd) || !aligned16(dx) ||
      (reinterpret_cast<uintptr_t>(key) & 7))
    return fail(ESEP_EALIGN, "lora_dropout_bwd: tensors need 16-byte and key 8-byte alignment");
  if (xd == dx || xd == g) return fail(ESEP_EINVAL, "lora_dropout_bwd: xd must not alias g or dx");
  bool sup = false;
  const hipError_t e = esep::launch_dropout_bwd(x, g, key, xd, dx, n, p, accumulate ? 1 : 0, dt,
                                                static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "lora_dropout_bwd: unsupported dtype");
  return e == hipSuccess ? 0 : hip_fail(e, "lora_dropout_bwd launch");
}

int esep_nf4_dequant(const void* packed, const uint8_t* absmax, const float* absmax2,
                     const float* code2, const float* offset, const float* nf4, void* out,
                     int out_dt, int64_t n_blocks, void* stream) {
  g_err[0] = 0;
  if (!float_dt(out_dt)) return fail(ESEP_EINVAL, "nf4_dequant: bad output dtype code %d", out_dt);
  if (n_blocks < 0) return fail(ESEP_ESHAPE, "nf4_dequant: n_blocks=%lld < 0", (long long)n_blocks);
  if (n_blocks == 0) return 0;
  if (packed == nullptr || absmax == nullptr || absmax2 == nullptr || code2 == nullptr ||
      offset == nullptr || nf4 == nullptr || out == nullptr)
    return fail(ESEP_EINVAL, "nf4_dequant: every pointer is required");
  if ((reinterpret_cast<uintptr_t>(packed) & 7) || !aligned16(out))
    return fail(ESEP_EALIGN, "nf4_dequant: packed needs 8-byte and out 16-byte alignment");
  esep::Nf4Args a{packed, absmax, absmax2, code2, offset, nf4, out, n_blocks};
  bool sup = false;
  const hipError_t e = esep::launch_nf4_dequant(a, out_dt, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "nf4_dequant: unsupported output dtype");
  return e == hipSuccess ? 0 : hip_fail(e, "nf4_dequant launch");
}

static_assert(ESEP_NF4_MULTI_MAX == esep::kNf4MultiMax, "multi-weight limit of the ABI and the kernel");

int esep_nf4_dequant_multi(const esep_nf4_weight* weights, int n_weights, int out_dt,
                           void* stream) {
  g_err[0] = 0;
  if (!float_dt(out_dt))
    return fail(ESEP_EINVAL, "nf4_dequant_multi: bad output dtype code %d", out_dt);
  if (weights == nullptr || n_weights < 1 || n_weights > ESEP_NF4_MULTI_MAX)
    return fail(ESEP_EINVAL, "nf4_dequant_multi: need 1..%d weights (got %d)", ESEP_NF4_MULTI_MAX,
                n_weights);
  esep::Nf4Multi m{};
  m.n = n_weights;
  m.q0[0] = 0;
  for (int i = 0; i < n_weights; ++i) {
    const esep_nf4_weight& w = weights[i];
    if (w.n_blocks < 0 || w.n_blocks > (int64_t{1} << 40))
      return fail(ESEP_ESHAPE, "nf4_dequant_multi: weight %d n_blocks=%lld out of range", i,
                  (long long)w.n_blocks);
    if (w.packed == nullptr || w.absmax == nullptr || w.absmax2 == nullptr ||
        w.code2 == nullptr || w.offset == nullptr || w.nf4 == nullptr || w.out == nullptr)
      return fail(ESEP_EINVAL, "nf4_dequant_multi: weight %d: every pointer is required", i);
    if ((reinterpret_cast<uintptr_t>(w.packed) & 7) || !aligned16(w.out))
      return fail(ESEP_EALIGN,
                  "nf4_dequant_multi: weight %d: packed needs 8-byte and out 16-byte alignment", i);
    m.w[i] = esep::Nf4Args{w.packed, w.absmax, w.absmax2, w.code2, w.offset, w.nf4, w.out,
                           w.n_blocks};
    m.q0[i + 1] = m.q0[i] + 4 * w.n_blocks;
  }
  for (int i = n_weights; i < esep::kNf4MultiMax; ++i) m.q0[i + 1] = m.q0[n_weights];
  if (m.q0[n_weights] / 256 >= 0x7fffffffLL)
    return fail(ESEP_ESHAPE, "nf4_dequant_multi: too many blocks for one launch");
  bool sup = false;
  const hipError_t e =
      esep::launch_nf4_dequant_multi(m, out_dt, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "nf4_dequant_multi: unsupported output dtype");
  return e == hipSuccess ? 0 : hip_fail(e, "nf4_dequant_multi launch");
}

int esep_head_row_softmax(void* z, int64_t ld, const int64_t* target, const float* cew,
                          float* lse, float* tlogit, float* ent, int32_t* amax, int64_t rows,
                          int64_t V, int write_g, float g_scale, int dt, void* stream) {
  g_err[0] = 0;
  if (dt != ESEP_F16 && dt != ESEP_BF16)
    return fail(ESEP_EINVAL, "head_row_softmax: logits must be fp16 or bf16 (dtype code %d)", dt);
  if (rows < 0 || rows > 0x7fffffffLL)
    return fail(ESEP_ESHAPE, "head_row_softmax: rows=%lld out of range", (long long)rows);
  if (V < 1 || V > (1LL << 30))
    return fail(ESEP_ESHAPE, "head_row_softmax: V=%lld outside [1, 2^30]", (long long)V);
  if (ld < V) return fail(ESEP_ESHAPE, "head_row_softmax: ld=%lld < V=%lld", (long long)ld,
                          (long long)V);
  if (rows == 0) return 0;
  if (z == nullptr || target == nullptr || lse == nullptr || tlogit == nullptr || ent == nullptr ||
      amax == nullptr || (write_g && cew == nullptr))
    return fail(ESEP_EINVAL, "head_row_softmax: z, target, lse, tlogit, ent, amax (and cew with "
                             "write_g) are required");
  if (reinterpret_cast<uintptr_t>(z) & 1)
    return fail(ESEP_EALIGN, "head_row_softmax: z must be 2-byte aligned");
  const bool vec = aligned16(z) && (ld & 7) == 0 && (V & 7) == 0;
  esep::HeadArgs a{z, target, cew, lse, tlogit, ent, amax, rows, ld, V, g_scale, write_g ? 1 : 0};
  bool sup = false;
  const hipError_t e =
      esep::launch_head_row(a, dt, vec, static_cast<hipStream_t>(stream), &sup);
  if (!sup) return fail(ESEP_EINVAL, "head_row_softmax: unsupported dtype");
  return e == hipSuccess ? 0 : hip_fail(e, "head_row_softmax launch");
}

}  // extern "C"

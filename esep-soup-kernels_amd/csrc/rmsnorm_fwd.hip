// Instantiations and launch dispatch of the RMSNorm forward kernel.
// Supported (x, delta, y) element types:
//   x fp32: delta none/fp32/fp16/bf16, y fp32/fp16/bf16   (fp32 residual stream, reference API)
//   x fp16: delta none/fp16, y fp16/fp32
//   x bf16: delta none/bf16, y bf16/fp32                  (16-bit activations, HF semantics)
#include "rmsnorm.hpp"

namespace esep {

// Rows per wavefront of the plain forward at n <= 1536 (one wavefront per row). Measured at
// config 4 (8192 x 1536 bf16, per launch): 1 row 9.97 us, 2 10.2, 3 10.06, 4 9.79, 6 12.96,
// 8 12.04 (too few wavefronts left); 4 rows built under the 1024-thread bound (78 VGPRs, the
// compiler schedules the loads differently) 9.05. Rows per group with several wavefronts per
// row (n > 1536) measured slower at config 5 (2 to 4 rows: 174-175 us against 170).
constexpr int kFwdRowsPerWave = 4;
// With a delta (the reference API's add_rmsnorm: fp32 residual + bf16 delta -> fp32 r_out, bf16
// y at 8192 x 1536): 1 row 31.3 us against 32.0 for the general kernel, 2 rows 31.6, 4 rows 37.7.
constexpr int kFwdDeltaRowsPerWave = 1;

template <typename TX, typename TD, typename TY>
static hipError_t fwd_nv(const FwdArgs& a, int nv, dim3 grid, dim3 block, hipStream_t s) {
  constexpr int RPW = std::is_void_v<TD> ? kFwdRowsPerWave : kFwdDeltaRowsPerWave;
  if constexpr (RPW > 0) {
    if (a.vec && a.wpr == 1 && a.n_special == 0 && block.x == 256) {
      const dim3 g((unsigned)((a.rows + 4 * RPW - 1) / (4 * RPW)));
      if (nv == 2) hipLaunchKernelGGL((k_rmsnorm_fwd_multi<2, TX, TD, TY, RPW>), g, block, 0, s, a);
      else hipLaunchKernelGGL((k_rmsnorm_fwd_multi<3, TX, TD, TY, RPW>), g, block, 0, s, a);
      return hipGetLastError();
    }
  }
  if (!a.vec) {
    hipLaunchKernelGGL((k_rmsnorm_fwd<3, false, TX, TD, TY>), grid, block, 0, s, a);
    return hipGetLastError();
  }
  switch (nv) {
    case 2: hipLaunchKernelGGL((k_rmsnorm_fwd<2, true, TX, TD, TY>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((k_rmsnorm_fwd<3, true, TX, TD, TY>), grid, block, 0, s, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <typename TX, typename TD>
static hipError_t fwd_y(const FwdArgs& a, int y_dt, int nv, dim3 g, dim3 b, hipStream_t s,
                        bool* sup) {
  *sup = true;
  if (y_dt == 0) return fwd_nv<TX, TD, float>(a, nv, g, b, s);
  if (y_dt == 1 && !std::is_same_v<TX, __bf16>) return fwd_nv<TX, TD, _Float16>(a, nv, g, b, s);
  if (y_dt == 2 && !std::is_same_v<TX, _Float16>) return fwd_nv<TX, TD, __bf16>(a, nv, g, b, s);
  *sup = false;
  return hipErrorInvalidValue;
}

hipError_t launch_rmsnorm_fwd(const FwdArgs& a, int x_dt, int d_dt, int y_dt, int nv, dim3 grid,
                              dim3 block, hipStream_t s, bool* sup) {
  *sup = false;
  if (x_dt == 0) {
    if (d_dt < 0) return fwd_y<float, void>(a, y_dt, nv, grid, block, s, sup);
    if (d_dt == 0) return fwd_y<float, float>(a, y_dt, nv, grid, block, s, sup);
    if (d_dt == 1) return fwd_y<float, _Float16>(a, y_dt, nv, grid, block, s, sup);
    if (d_dt == 2) return fwd_y<float, __bf16>(a, y_dt, nv, grid, block, s, sup);
  } else if (x_dt == 1) {
    if (d_dt < 0) return fwd_y<_Float16, void>(a, y_dt, nv, grid, block, s, sup);
    if (d_dt == 1) return fwd_y<_Float16, _Float16>(a, y_dt, nv, grid, block, s, sup);
  } else if (x_dt == 2) {
    if (d_dt < 0) return fwd_y<__bf16, void>(a, y_dt, nv, grid, block, s, sup);
    if (d_dt == 2) return fwd_y<__bf16, __bf16>(a, y_dt, nv, grid, block, s, sup);
  }
  return hipErrorInvalidValue;
}

}  // namespace esep

// Instantiations and launch dispatch of the RMSNorm backward kernel and of the weight-gradient
// reduction. Supported (x, dy, dx) element types:
//   x fp32 (the fp32 residual): dy fp32/fp16/bf16, dx fp32/fp16/bf16
//   x fp16 (saved fp16 output or fp16 input): dy fp16/fp32, dx fp16/fp32; with dy fp16 also
//          dx bf16 (the reference API's saved-output backward with a bf16 residual delta)
//   x bf16 (saved bf16 output or bf16 input): dy bf16/fp32, dx bf16/fp32; with dy bf16 also
//          dx fp16 (the same with an fp16 delta)
// A call that writes no low-precision dx uses dx type fp32 (nothing is stored through it).
#include "rmsnorm.hpp"

namespace esep {

template <typename TX, typename TDY, typename TO>
static hipError_t bwd_nv(const BwdArgs& a, int nv, dim3 grid, dim3 block, size_t lds,
                         hipStream_t s) {
  if (!a.vec) {
    hipLaunchKernelGGL((k_rmsnorm_bwd<3, false, TX, TDY, TO>), grid, block, lds, s, a);
    return hipGetLastError();
  }
  // The fast kernels serve the plain backward (one dy, xhat from x, no dr_out): the pipelined
  // one for rows of one wavefront, the wide one otherwise; the entry point decides with the
  // launch shape.
  const bool fast = a.fast != 0;
  if (a.fast == 1) {
    if (block.x != (unsigned)kBwdPipeThreads || a.gpb != kBwdPipeThreads / kWave || a.wpr != 1)
      return hipErrorInvalidValue;
    // saved rstd and dx only (the common call) run a form with those parts fixed, and so does
    // dx only with the weight gradient and rstd recomputed (config 4 with rstd recomputed: 16.25
    // us per launch in the trace with the parts read from the arguments)
    const bool common = a.rstd != nullptr && a.dr == nullptr && a.dx != nullptr;
    const bool recompute = a.rstd == nullptr && a.dr == nullptr && a.dx != nullptr && a.part != nullptr;
    const int fix = common ? (a.part != nullptr ? 1 : 2) : recompute ? 3 : 0;
    if (fix == 1) {
      if (nv == 2) hipLaunchKernelGGL((k_rmsnorm_bwd_pipe<2, TX, TDY, TO, 1>), grid, block, lds, s, a);
      else hipLaunchKernelGGL((k_rmsnorm_bwd_pipe<3, TX, TDY, TO, 1>), grid, block, lds, s, a);
    } else if (fix == 3) {
      if (nv == 2) hipLaunchKernelGGL((k_rmsnorm_bwd_pipe<2, TX, TDY, TO, 3>), grid, block, lds, s, a);
      else hipLaunchKernelGGL((k_rmsnorm_bwd_pipe<3, TX, TDY, TO, 3>), grid, block, lds, s, a);
    } else if (fix == 2) {
      if (nv == 2) hipLaunchKernelGGL((k_rmsnorm_bwd_pipe<2, TX, TDY, TO, 2>), grid, block, lds, s, a);
      else hipLaunchKernelGGL((k_rmsnorm_bwd_pipe<3, TX, TDY, TO, 2>), grid, block, lds, s, a);
    } else {
      if (nv == 2) hipLaunchKernelGGL((k_rmsnorm_bwd_pipe<2, TX, TDY, TO, 0>), grid, block, lds, s, a);
      else hipLaunchKernelGGL((k_rmsnorm_bwd_pipe<3, TX, TDY, TO, 0>), grid, block, lds, s, a);
    }
    return hipGetLastError();
  }
  if (a.fast == 2) {
    if (nv == 2) hipLaunchKernelGGL((k_rmsnorm_bwd_wide<2, TX, TDY, TO>), grid, block, lds, s, a);
    else hipLaunchKernelGGL((k_rmsnorm_bwd_wide<3, TX, TDY, TO>), grid, block, lds, s, a);
    return hipGetLastError();
  }
  // The reference API's other calls without a weight gradient or exact channels.
  if (!fast && a.part == nullptr && a.n_special == 0 && a.n_dy > 0 &&
      block.x <= (unsigned)kBwdApiThreads) {
    if (nv == 2) hipLaunchKernelGGL((k_rmsnorm_bwd_api<2, TX, TDY, TO>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_rmsnorm_bwd_api<3, TX, TDY, TO>), grid, block, 0, s, a);
    return hipGetLastError();
  }
  if (nv == 2) hipLaunchKernelGGL((k_rmsnorm_bwd<2, true, TX, TDY, TO>), grid, block, lds, s, a);
  else hipLaunchKernelGGL((k_rmsnorm_bwd<3, true, TX, TDY, TO>), grid, block, lds, s, a);
  return hipGetLastError();
}

template <typename T> constexpr int kCode = std::is_same_v<T, float> ? 0 : (std::is_same_v<T, _Float16> ? 1 : 2);

template <typename TX, typename TDY>
static hipError_t bwd_o(const BwdArgs& a, int o_dt, int nv, dim3 g, dim3 b, size_t lds,
                        hipStream_t s, bool* sup) {
  *sup = true;
  if (o_dt == 0) return bwd_nv<TX, TDY, float>(a, nv, g, b, lds, s);
  constexpr int xc = kCode<TX>, dc = kCode<TDY>;
  if constexpr (xc == 0 || xc == 1 || (xc == 2 && dc == 2))
    if (o_dt == 1) return bwd_nv<TX, TDY, _Float16>(a, nv, g, b, lds, s);
  if constexpr (xc == 0 || xc == 2 || (xc == 1 && dc == 1))
    if (o_dt == 2) return bwd_nv<TX, TDY, __bf16>(a, nv, g, b, lds, s);
  *sup = false;
  return hipErrorInvalidValue;
}

hipError_t launch_rmsnorm_bwd(const BwdArgs& a, int x_dt, int dy_dt, int o_dt, int nv, dim3 grid,
                              dim3 block, size_t lds, hipStream_t s, bool* sup) {
  *sup = false;
  if (x_dt == 0) {
    if (dy_dt == 0) return bwd_o<float, float>(a, o_dt, nv, grid, block, lds, s, sup);
    if (dy_dt == 1) return bwd_o<float, _Float16>(a, o_dt, nv, grid, block, lds, s, sup);
    if (dy_dt == 2) return bwd_o<float, __bf16>(a, o_dt, nv, grid, block, lds, s, sup);
  } else if (x_dt == 1) {
    if (dy_dt == 0) return bwd_o<_Float16, float>(a, o_dt, nv, grid, block, lds, s, sup);
    if (dy_dt == 1) return bwd_o<_Float16, _Float16>(a, o_dt, nv, grid, block, lds, s, sup);
  } else if (x_dt == 2) {
    if (dy_dt == 0) return bwd_o<__bf16, float>(a, o_dt, nv, grid, block, lds, s, sup);
    if (dy_dt == 2) return bwd_o<__bf16, __bf16>(a, o_dt, nv, grid, block, lds, s, sup);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_dgamma_reduce(const float* part, int64_t P, int n, void* dw, int dw_dt,
                                hipStream_t s, bool* sup) {
  *sup = true;
  const dim3 grid((n + kRedCols - 1) / kRedCols), block(256);
  if (dw_dt == 0)
    hipLaunchKernelGGL(k_dgamma_reduce<float>, grid, block, 0, s, part, P, n, static_cast<float*>(dw));
  else if (dw_dt == 1)
    hipLaunchKernelGGL(k_dgamma_reduce<_Float16>, grid, block, 0, s, part, P, n, static_cast<_Float16*>(dw));
  else if (dw_dt == 2)
    hipLaunchKernelGGL(k_dgamma_reduce<__bf16>, grid, block, 0, s, part, P, n, static_cast<__bf16*>(dw));
  else {
    *sup = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_dgamma_reduce_batch(const DgammaBatch& b, int count, int n, int dw_dt,
                                      hipStream_t s, bool* sup) {
  *sup = true;
  const dim3 grid((n + kRedCols - 1) / kRedCols, count), block(256);
  if (dw_dt == 0)
    hipLaunchKernelGGL(k_dgamma_reduce_batch<float>, grid, block, 0, s, b, n);
  else if (dw_dt == 1)
    hipLaunchKernelGGL(k_dgamma_reduce_batch<_Float16>, grid, block, 0, s, b, n);
  else if (dw_dt == 2)
    hipLaunchKernelGGL(k_dgamma_reduce_batch<__bf16>, grid, block, 0, s, b, n);
  else {
    *sup = false;
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace esep

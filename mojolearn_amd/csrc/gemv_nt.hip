// gfx950 skinny-M kernel, OP_NT (the LM layout): X[M x K] . W[N x K]^T, M <= 16.
#include "gemv_body.h"

namespace mlg {

template <int BT, int MR, bool VEC>
__global__ void __launch_bounds__(GV_THREADS) gemv_nt_kernel(GemvArgs g, const float* __restrict__ x) {
  gemv_body<BT, MR, VEC, false, true>(g, x);
}

template <int BT, int MR>
static hipError_t launch_mr(const GemvArgs& g, const float* x, int vec, dim3 grid, hipStream_t s) {
  if (vec) hipLaunchKernelGGL((gemv_nt_kernel<BT, MR, true>), grid, dim3(GV_THREADS), 0, s, g, x);
  else hipLaunchKernelGGL((gemv_nt_kernel<BT, MR, false>), grid, dim3(GV_THREADS), 0, s, g, x);
  return hipGetLastError();
}

template <int BT>
static hipError_t launch_m(const GemvArgs& g, const float* x, int64_t m, int vec, dim3 grid, hipStream_t s) {
  if (m <= 1) return launch_mr<BT, 1>(g, x, vec, grid, s);
  if (m <= 2) return launch_mr<BT, 2>(g, x, vec, grid, s);
  if (m <= 4) return launch_mr<BT, 4>(g, x, vec, grid, s);
  if (m <= 8) return launch_mr<BT, 8>(g, x, vec, grid, s);
  return launch_mr<BT, 16>(g, x, vec, grid, s);
}

hipError_t launch_gemv_nt(const GemvArgs& g, const float* x, int b_type, int64_t m, int vec, dim3 grid,
                    hipStream_t stream) {
  if (b_type == T_F32) return launch_m<T_F32>(g, x, m, vec, grid, stream);
  if (b_type == T_BF16) return launch_m<T_BF16>(g, x, m, vec, grid, stream);
  return launch_m<T_I8>(g, x, m, vec, grid, stream);
}

}  // namespace mlg

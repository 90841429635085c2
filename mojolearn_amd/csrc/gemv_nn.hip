// gfx950 skinny-M kernel, OP_NN: X[M x K] . W[K x N], M <= 16.
#include "gemv_body.h"

namespace mlg {

template <int BT, int MR, bool VEC, bool FULLLEAF, int LEAVES>
__global__ void __launch_bounds__(64 * LEAVES) gemv_nn_kernel(GemvArgs g, const float* __restrict__ x) {
  gemv_body<BT, MR, VEC, FULLLEAF, false, LEAVES>(g, x);
}

template <int BT, int MR>
static hipError_t launch_mr(const GemvArgs& g, const float* x, int vec, int leaves, dim3 grid, hipStream_t s) {
  if (vec == 2 && leaves == GV_WIDE_LEAVES) {
    // the wide workgroups are built for the decode rows (m <= 2) only
    if constexpr (MR <= 2) {
      hipLaunchKernelGGL((gemv_nn_kernel<BT, MR, true, true, GV_WIDE_LEAVES>), grid, dim3(64 * GV_WIDE_LEAVES), 0, s,
                         g, x);
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  if (leaves != GV_LEAVES) return hipErrorInvalidValue;
  if (vec == 2)
    hipLaunchKernelGGL((gemv_nn_kernel<BT, MR, true, true, GV_LEAVES>), grid, dim3(GV_THREADS), 0, s, g, x);
  else if (vec == 1)
    hipLaunchKernelGGL((gemv_nn_kernel<BT, MR, true, false, GV_LEAVES>), grid, dim3(GV_THREADS), 0, s, g, x);
  else
    hipLaunchKernelGGL((gemv_nn_kernel<BT, MR, false, false, GV_LEAVES>), grid, dim3(GV_THREADS), 0, s, g, x);
  return hipGetLastError();
}

template <int BT>
static hipError_t launch_m(const GemvArgs& g, const float* x, int64_t m, int vec, int leaves, dim3 grid,
                           hipStream_t s) {
  if (m <= 1) return launch_mr<BT, 1>(g, x, vec, leaves, grid, s);
  if (m <= 2) return launch_mr<BT, 2>(g, x, vec, leaves, grid, s);
  if (m <= 4) return launch_mr<BT, 4>(g, x, vec, leaves, grid, s);
  if (m <= 8) return launch_mr<BT, 8>(g, x, vec, leaves, grid, s);
  return launch_mr<BT, 16>(g, x, vec, leaves, grid, s);
}

hipError_t launch_gemv_nn(const GemvArgs& g, const float* x, int b_type, int64_t m, int vec, int leaves, dim3 grid,
                          hipStream_t stream) {
  if (b_type == T_F32) return launch_m<T_F32>(g, x, m, vec, leaves, grid, stream);
  if (b_type == T_BF16) return launch_m<T_BF16>(g, x, m, vec, leaves, grid, stream);
  return launch_m<T_I8>(g, x, m, vec, leaves, grid, stream);
}

}  // namespace mlg

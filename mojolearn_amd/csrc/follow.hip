// The product's followers over its stored cells (run_follow in kernels.h).  A workgroup takes
// 1024 columns of a row (4 per thread) and strides over rows; with 16-byte rows, base and second
// buffer (VEC) the 4 cells travel as one 16-byte load and store, otherwise one word each.
// Runs in the kernel's default floating-point mode (denormals kept), so the activations' inner
// operations round exactly as the host's.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "act.h"
#include "device_common.h"
#include "kernels.h"

namespace mlg {

constexpr int FOLLOW_THREADS = 256;
constexpr int FOLLOW_COLS = 4 * FOLLOW_THREADS;  // columns per workgroup
constexpr int64_t FOLLOW_MAX_ROW_BLOCKS = 65535;

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// p: the bias (p[j], EPI_PLUS_BIAS / EPI_BIAS_ACT) or the forward values (p[i * n + j], EPI_ACT_BWD).
template <bool VEC>
__global__ void __launch_bounds__(FOLLOW_THREADS) follow_kernel(float* c, int64_t ldc, int64_t m, int64_t n,
                                                                int zero, int kind, const float* __restrict__ p,
                                                                int act) {
  const int64_t j0 = ((int64_t)blockIdx.x * FOLLOW_THREADS + threadIdx.x) * 4;
  if (j0 >= n) return;
  const bool per_cell = kind == EPI_ACT_BWD;
  const bool reads_p = kind == EPI_PLUS_BIAS || kind == EPI_BIAS_ACT || per_cell;
  for (int64_t i = blockIdx.y; i < m; i += gridDim.y) {
    float* row = c + i * ldc;
    const float* prow = per_cell ? p + i * n : p;
    float v[4] = {0.f, 0.f, 0.f, 0.f}, q[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (VEC) {
      if (!zero) {
        const float4 t = *reinterpret_cast<const float4*>(row + j0);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
      }
      if (reads_p) {
        const float4 t = *reinterpret_cast<const float4*>(prow + j0);
        q[0] = t.x; q[1] = t.y; q[2] = t.z; q[3] = t.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (j0 + e >= n) break;
        if (!zero) v[e] = row[j0 + e];
        if (reads_p) q[e] = prow[j0 + e];
      }
    }
    float y[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = store_word(follow_one(act_ftz(v[e]), kind, q[e], act));
    if constexpr (VEC) {
      *reinterpret_cast<float4*>(row + j0) = make_float4(y[0], y[1], y[2], y[3]);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (j0 + e < n) row[j0 + e] = y[e];
    }
  }
}

hipError_t run_follow(float* c, int64_t ldc, int64_t m, int64_t n, int zero, int kind, const float* p, int act,
                      hipStream_t stream) {
  if (m <= 0 || n <= 0) return hipSuccess;
  const bool reads_p = kind == EPI_PLUS_BIAS || kind == EPI_BIAS_ACT || kind == EPI_ACT_BWD;
  const bool vec = n % 4 == 0 && (m == 1 || ldc % 4 == 0) && aligned16(c) && (!reads_p || aligned16(p));
  const dim3 grid((unsigned)((n + FOLLOW_COLS - 1) / FOLLOW_COLS),
                  (unsigned)(m < FOLLOW_MAX_ROW_BLOCKS ? m : FOLLOW_MAX_ROW_BLOCKS));
  if (vec)
    hipLaunchKernelGGL(follow_kernel<true>, grid, dim3(FOLLOW_THREADS), 0, stream, c, ldc, m, n, zero, kind, p, act);
  else
    hipLaunchKernelGGL(follow_kernel<false>, grid, dim3(FOLLOW_THREADS), 0, stream, c, ldc, m, n, zero, kind, p, act);
  return hipGetLastError();
}

}  // namespace mlg

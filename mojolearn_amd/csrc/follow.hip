// The product's followers over its stored cells (run_follow in kernels.h): one thread a cell,
// rows of C at stride ldc.  Runs in the kernel's default floating-point mode (denormals kept),
// so the activations' inner operations round exactly as the host's.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "act.h"
#include "device_common.h"
#include "kernels.h"

namespace mlg {

__global__ void __launch_bounds__(256) follow_kernel(float* c, int64_t ldc, int64_t m, int64_t n, int zero, int kind,
                                                     const float* __restrict__ p, int act) {
  const int64_t cell = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (cell >= m * n) return;
  const int64_t i = cell / n, j = cell - i * n;
  float* at = c + i * ldc + j;
  const float w = zero ? 0.0f : act_ftz(*at);
  float y = w;
  if (kind == EPI_PLUS_BIAS) y = act_ftz(w + act_ftz(p[j]));
  else if (kind == EPI_BIAS_ACT) y = act_value(act_ftz(w + act_ftz(p[j])), act);
  else if (kind == EPI_ACT_BWD) y = act_bwd_value(w, act_ftz(p[cell]), act);
  *at = store_word(y);
}

hipError_t run_follow(float* c, int64_t ldc, int64_t m, int64_t n, int zero, int kind, const float* p, int act,
                      hipStream_t stream) {
  if (m <= 0 || n <= 0) return hipSuccess;
  const int64_t cells = m * n;
  hipLaunchKernelGGL(follow_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, stream, c, ldc, m, n, zero,
                     kind, p, act);
  return hipGetLastError();
}

}  // namespace mlg

// The activation followers of a product, on one value, as device functions.  Every operation
// is one IEEE single-precision operation in the kernel's default mode (denormals kept): fused
// multiply-adds through __builtin_fmaf, products and sums never contracted (-ffp-contract=off),
// one correctly rounded division.  Flushes are explicit, on the integer word.
//
//   expf     checks/numerics.mojo:370-408 (Cephes single-precision expf, fma reduction)
//   divf     checks/numerics.mojo:1025-1037 (flushed operands, one division, flushed result)
//   sigmoid  checks/numerics.mojo:1079-1085, tanh :1190-1222 (Cephes tanhf, zero keeps its sign)
//   act_value / act_bwd_value  sequence/act_values.mojo:60-85
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlg {

constexpr int ACT_IDENTITY = 0, ACT_LOGISTIC = 1, ACT_TANH = 2, ACT_RELU = 3, ACT_SOFTMAX = 4;
constexpr int EPI_NONE = 0, EPI_PLUS_BIAS = 3, EPI_BIAS_ACT = 4, EPI_ACT_BWD = 5;

__device__ __forceinline__ float act_ftz(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x7F800000u) == 0u ? __uint_as_float(u & 0x80000000u) : x;
}

__device__ __forceinline__ float act_expf(float x) {
  if (x != x) return x;
  if (x > 88.722835f) return __uint_as_float(0x7F800000u);
  if (x < -87.33655f) return 0.0f;
  const float zf = __builtin_floorf(__builtin_fmaf(x, 1.4426950408889634f, 0.5f));
  const int32_t kq = (int32_t)zf;
  float r = __builtin_fmaf(zf, -0.693359375f, x);
  r = __builtin_fmaf(zf, 2.12194440e-4f, r);
  float q = 1.9875691500e-4f;
  q = __builtin_fmaf(q, r, 1.3981999507e-3f);
  q = __builtin_fmaf(q, r, 8.3334519073e-3f);
  q = __builtin_fmaf(q, r, 4.1665795894e-2f);
  q = __builtin_fmaf(q, r, 1.6666665459e-1f);
  q = __builtin_fmaf(q, r, 5.0000001201e-1f);
  const float r2 = r * r;
  float y = __builtin_fmaf(q, r2, r) + 1.0f;
  const int32_t k1 = kq >> 1, k2 = kq - k1;
  y = y * __uint_as_float((uint32_t)(k1 + 127) << 23);
  y = y * __uint_as_float((uint32_t)(k2 + 127) << 23);
  if (y < 1.1754943508222875e-38f) return 0.0f;
  return y;
}

__device__ __forceinline__ float act_divf(float a, float b) { return act_ftz(act_ftz(a) / act_ftz(b)); }

__device__ __forceinline__ float act_sigmoidf(float x) {
  if (x != x) return x;
  return act_divf(1.0f, act_expf(-x) + 1.0f);
}

__device__ __forceinline__ float act_tanhf(float x_in) {
  const float xx = act_ftz(x_in);
  if (xx != xx) return xx;
  if (xx == 0.0f) return xx;
  const float x = __builtin_fabsf(xx);
  if (x > __uint_as_float(0x42317218u)) return xx < 0.0f ? -1.0f : 1.0f;
  if (x >= 0.625f) {
    const float e = act_expf(x + x);
    const float q = act_divf(2.0f, e + 1.0f);
    const float z = 1.0f - q;
    return xx < 0.0f ? -z : z;
  }
  const float zs = x * x;
  float p = -5.70498872745e-3f;
  p = __builtin_fmaf(p, zs, 2.06390887954e-2f);
  p = __builtin_fmaf(p, zs, -5.37397155531e-2f);
  p = __builtin_fmaf(p, zs, 1.33314422036e-1f);
  p = __builtin_fmaf(p, zs, -3.33332819422e-1f);
  const float pz = p * zs;
  return __builtin_fmaf(pz, xx, xx);
}

__device__ __forceinline__ float act_value(float z, int code) {
  if (code == ACT_LOGISTIC) return act_ftz(act_sigmoidf(z));
  if (code == ACT_TANH) return act_ftz(act_tanhf(z));
  if (code == ACT_RELU) return z > 0.0f ? z : 0.0f;
  return z;
}

__device__ __forceinline__ float act_bwd_value(float d, float z, int code) {
  if (code == ACT_LOGISTIC) return act_ftz(act_ftz(d * z) * act_ftz(1.0f - z));
  if (code == ACT_TANH) return act_ftz(d * act_ftz(1.0f - act_ftz(z * z)));
  if (code == ACT_RELU && z == 0.0f) return 0.0f;
  return d;
}

// One follower on a stored cell `c` (already flushed): kind 3 PLUS_BIAS ftz(c + ftz(q)), 4 BIAS_ACT
// act(ftz(c + ftz(q))), 5 ACT_BWD act_bwd(c, ftz(q)); the caller flushes the result and
// canonicalizes NaNs (gemm/checks/gemm_identical.mojo:8884-8912).  Every input of every float
// operation here is flushed on its integer word or cannot move the rounded result when the
// kernel's mode flushes it (r * r in expf and x * x in tanhf, subnormal only for |r|, |x| below
// 2^-62, where the fused multiply-add that reads them rounds to its addend either way), so the
// value does not depend on the kernel's MODE.FP_DENORM.
__device__ __forceinline__ float follow_one(float c, int kind, float q, int act) {
  if (kind == EPI_PLUS_BIAS) return act_ftz(c + act_ftz(q));
  if (kind == EPI_BIAS_ACT) return act_value(act_ftz(c + act_ftz(q)), act);
  if (kind == EPI_ACT_BWD) return act_bwd_value(c, act_ftz(q), act);
  return c;
}

}  // namespace mlg

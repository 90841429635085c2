// mojolearn.identical.gemm.fp32.v1: the numerical plan as host/device helpers.
//
// Leaf rule: gemm/contract.mojo:173-235 (K_LEAF_MIN = 128, MAX_LEAVES = 1024,
// L derived first, P = ceil(k / L) second, so no leaf is ever empty).
// Operation codes: gemm/contract.mojo:252-256 (NN = 0, NT = 1, TN = 2).
#pragma once
#include <stdint.h>

namespace mlg {

constexpr int OP_NN = 0;
constexpr int OP_NT = 1;
constexpr int OP_TN = 2;

constexpr int64_t K_LEAF_MIN = 128;
constexpr int64_t MAX_LEAVES = 1024;

// Element types of a stored operand.
constexpr int T_F32 = 0;   // float32
constexpr int T_BF16 = 1;  // bfloat16 bits, widened exactly (bits << 16)
constexpr int T_I8 = 2;    // int8 code times a per-output-column float32 scale

__host__ __device__ inline int64_t leaf_size(int64_t k) {
  if (k <= 0) return 1;
  if (k <= K_LEAF_MIN) return k;
  int64_t p0 = (k + K_LEAF_MIN - 1) / K_LEAF_MIN;
  if (p0 <= MAX_LEAVES) return K_LEAF_MIN;
  return (k + MAX_LEAVES - 1) / MAX_LEAVES;
}

__host__ __device__ inline int64_t leaf_count(int64_t k, int64_t leaf) {
  if (k <= 0) return 0;
  if (leaf < 1) leaf = 1;
  return (k + leaf - 1) / leaf;
}

}  // namespace mlg

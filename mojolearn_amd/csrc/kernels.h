// Launchers of the gfx950 kernels (mojolearn_amd/csrc/kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlg {

// One product C = op(A) . op(B) under fp32.v1 on device buffers.
struct GemmProblem {
  float* c;              // m x n row-major output
  const void* a;         // A in the layout of `op`, element type a_type (T_F32 or T_BF16)
  const void* b;         // B in the layout of `op`, element type b_type (T_F32, T_BF16, T_I8)
  const float* scales;   // T_I8 only: one float32 scale per output column (n values)
  const float* bias;     // optional: n values, Y = ftz(ftz(C) + ftz(bias[j]))
  int64_t m, n, k;
  int op;                // OP_NN, OP_NT, OP_TN
  int a_type, b_type;
  int64_t leaf;          // leaf size; 0 = the contract's (leaf_size(k))
};

// Workspace floats run_gemm needs for `p` (0 when the product folds in one launch).
int64_t gemm_workspace_floats(const GemmProblem& p, int num_cus);

// Completion counters the product needs (0 or one per 256-column block of the skinny-M
// path); they must be zero on entry and are zero again when the product completes.
int64_t gemm_counter_count(const GemmProblem& p);

// Enqueue the product on `stream`.  `ws` must hold gemm_workspace_floats() floats and
// `counters` gemm_counter_count() zeroed counters.  Returns hipSuccess or the launch error.
hipError_t run_gemm(const GemmProblem& p, float* ws, unsigned int* counters, int num_cus,
                    hipStream_t stream);

// Elementwise conversions used by the low-bit surface (to_bf16 / from_bf16).
hipError_t run_bf16_widen(float* out, const uint16_t* in, int64_t count, hipStream_t stream);
// IEEE float16 bits -> float32, exact (gemm/f16_widen.mojo:12-37).
hipError_t run_f16_widen(float* out, const uint16_t* in, int64_t count, hipStream_t stream);
hipError_t run_bf16_narrow(uint16_t* out, const float* in, int64_t count, hipStream_t stream);

}  // namespace mlg

// Launchers of the gfx950 kernels (mojolearn_amd/csrc/kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

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
  // Stored-operand element strides (row, column) of A and B in the layout of `op`, read only
  // when `strided` is set (else the operands are dense).
  int strided;
  int64_t a_rs, a_cs, b_rs, b_cs;
  int64_t ldc;           // C row stride in elements; 0 = n
  int seed;              // one leaf only: each chain starts from the flushed old C, not +0
  int seq;               // the caller's word (strides, seed): always the tile kernel
  int whole;             // one column range: never split into whole rounds + a grouped tail
  // the activation followers fused into the store (act.h follow_one): 4 BIAS_ACT (epi_p[j]),
  // 5 ACT_BWD (epi_p[i n + j]), with activation `act`; 0 none (the bias, if any, is `bias`)
  int epi, act;
  const float* epi_p;
};

// Workspace floats run_gemm needs for `p`: [completion counters][group roots][A repacked]
// [B repacked], each part 256-byte aligned (0 when the product folds in one launch and loads
// its operands in place).
int64_t gemm_workspace_floats(const GemmProblem& p, int num_cus);

// Completion counters at the start of that workspace (0, or one per column group of a skinny
// product folded across workgroups).  They must be zero on entry; the product leaves them
// zero again when it completes.
int64_t gemm_counter_count(const GemmProblem& p);

// Why the product cannot be launched, or "" if it can: the fold stack covers STACK_ROOTS
// leaf-group roots per cell, a tile grid holds TILE_GROUPS leaf groups (blockIdx.y).
std::string launch_limit(const GemmProblem& p, int num_cus);
constexpr int64_t STACK_ROOTS = int64_t(1) << 20;
constexpr int64_t TILE_GROUPS = 65535;

// Kernels a product dispatches to (run_gemm with `route`: bits set, nothing launched).
constexpr unsigned ROUTE_TILE = 1;          // gemm_mfma_kernel
constexpr unsigned ROUTE_FOLD = 2;          // fold_groups_kernel after it (leaves in several groups)
constexpr unsigned ROUTE_GEMV_NN = 4;       // gemv_nn_kernel
constexpr unsigned ROUTE_GEMV_NT = 8;       // gemv_nt_kernel
constexpr unsigned ROUTE_MFMA4 = 16;        // gemv_mfma4_nn_kernel
constexpr unsigned ROUTE_MFMA16 = 32;       // gemv_mfma_nn_kernel
constexpr unsigned ROUTE_TAIL_SPLIT = 64;   // two column ranges (whole rounds + grouped tail)
constexpr unsigned ROUTE_REPACK = 128;      // repack_rows_kernel first
constexpr unsigned ROUTE_ZERO_K = 256;      // k = 0: +0 stored
constexpr unsigned ROUTE_TILE_STACK = 512;  // a tile folds several leaves in its own stack
constexpr unsigned ROUTE_GEMV_GROUPS = 1024;  // a skinny product folded across workgroups

// Enqueue the product on `stream`.  `ws` must hold gemm_workspace_floats() floats, its
// counters zero.  With `route`, only report the kernels (no launch, no operand read).
// Returns hipSuccess or the launch error.
hipError_t run_gemm(const GemmProblem& p, float* ws, int num_cus, hipStream_t stream, unsigned* route = nullptr);

// Zero `count` words on `stream` with a kernel.
hipError_t run_zero_words(unsigned int* p, int64_t count, hipStream_t stream);

// int8 weights W[k][n] in the decode-packed layout (gemv_packed.hip): k a multiple of 128 with at
// most 1024 leaves, n >= 1.  Bytes of the packed copy (k * 128 * ceil(n / 128)), or -1 for a
// shape the layout does not take.
int64_t int8w_packed_bytes(int64_t k, int64_t n);
// Write the packed copy of codes[k][n] to dst (16-byte aligned, int8w_packed_bytes bytes).
hipError_t run_int8w_pack(void* dst, const int8_t* codes, int64_t k, int64_t n, hipStream_t stream);
// Workspace floats run_gemv_packed needs: [completion counters][group roots], 0 for one group.
int64_t gemv_packed_workspace_floats(int64_t m, int64_t n, int64_t k);
// Words of completion counters at the start of that workspace (zero before its first product;
// every product leaves them zero).
int64_t gemv_packed_counter_count(int64_t m, int64_t n, int64_t k);
// C[m][n] = X[m][k] . W_deq (+ bias) from the packed copy, 1 <= m <= 16: the bits of run_gemm on
// the row-major codes (OP_NN, int8, the contract's leaves).  Empty string, or why it was refused.
std::string gemv_packed_limit(int64_t m, int64_t n, int64_t k, const void* packed);
hipError_t run_gemv_packed(float* c, const float* x, const void* packed, const float* scales, const float* bias,
                           int64_t m, int64_t n, int64_t k, float* ws, int num_cus, hipStream_t stream);
// Read-only streams over an int8 matrix W[rows][cols] (stream_read.hip): pattern 0 the whole
// matrix in address order, pattern 1 the row-major decode kernel's leaf-by-leaf reads, pattern 2
// the decode-packed product's whole-column reads.  Measurement only.
hipError_t run_stream_read(const void* w, int64_t rows, int64_t cols, int pattern, uint32_t* sink,
                           hipStream_t stream);

// Elementwise conversions used by the low-bit surface (to_bf16 / from_bf16).
hipError_t run_bf16_widen(float* out, const uint16_t* in, int64_t count, hipStream_t stream);
// IEEE float16 bits -> float32, exact (gemm/f16_widen.mojo:12-37).
hipError_t run_f16_widen(float* out, const uint16_t* in, int64_t count, hipStream_t stream);
hipError_t run_bf16_narrow(uint16_t* out, const float* in, int64_t count, hipStream_t stream);

// The product's followers over stored cells C[i * ldc + j] (i < m, j < n): `zero` first sets
// every cell to +0 (a product over k = 0); kind 3 adds the bias p[j], kind 4 adds the bias then
// applies activation `act`, kind 5 multiplies by the derivative of activation `act` at
// p[i * n + j]; kind 0 stores the flushed cell.  Epilogue kinds: gemm/checks/gemm_identical.mojo
// :8884-8912; activations sequence/act_values.mojo:60-85.
hipError_t run_follow(float* c, int64_t ldc, int64_t m, int64_t n, int zero, int kind, const float* p, int act,
                      hipStream_t stream);

}  // namespace mlg

// Device helpers shared by the gfx950 kernels of mojolearn.identical.gemm.fp32.v1.
//
// Arithmetic (gemm/IDENTICAL_FP32_CONTRACT.md sections 4-7, oracle
// gemm/host/gemm_oracle.mojo:146-371):
//   leaf t of cell (i,j):  acc = +0.0; for p ascending: acc = ftz(fma(ftz(A_eff[i,p]), ftz(B_eff[p,j]), acc))
//   leaves folded by the fixed balanced tree (adjacent pairs, odd tail carried),
//   each node ftz(ftz(x) + ftz(y)); the output is ftz(root); NaN words -> 0x7FC00000.
//
// How the hardware is made to compute exactly that:
//  * Every kernel first sets MODE.FP_DENORM(f32) = 2: every VALU and matrix instruction
//    flushes subnormal INPUTS to a zero of the same sign and keeps IEEE gradual underflow
//    on its output.  Measured on gfx950 for v_mfma_f32_{32x32x1_2b,16x16x1_4b,4x4x1_16b}_f32,
//    v_fma_f32, v_add_f32, v_mul_f32 (0 mismatching words against fma/add/mul of flushed
//    inputs over 786k triples per instruction, incl. fused-vs-unfused separators, inf/NaN,
//    signed zeros and the round-then-flush boundary).
//  * K=1 MFMA (v_mfma_f32_32x32x1_2b_f32) computes, per output, ONE fma_rn(a, b, c).
//  * Hence raw_{p+1} = fma(ftz a, ftz b, ftz raw_p) and, by induction, ftz(raw_p) is the
//    contract's acc_p: no flush instruction is needed inside the chain.  Fold adds flush
//    their inputs the same way; the one explicit ftz is at the store (seam 5g).
//  * The fold is the register-stack form of the tree: leaf partials pushed in ascending
//    order, slot l merged into the incoming value while bit l of the leaf index is set,
//    drained lowest level first.  Aligned power-of-two leaf groups are subtrees, so a
//    product is split into groups whose roots a second kernel folds with the same rule.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "contract.h"

namespace mlg {

typedef float v32f __attribute__((ext_vector_type(32)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));  // 16 raw bytes

// hwreg(HW_REG_MODE, 4, 2): FP_DENORM single-precision field.
#define MLG_HWREG_FP_DENORM32 ((1 << 11) | (4 << 6) | 1)

__device__ __forceinline__ void set_flush_inputs_mode() {
  __builtin_amdgcn_s_setreg(MLG_HWREG_FP_DENORM32, 2);
}

// Seam 5g plus the surface's NaN canonicalization (core/nan_canon.mojo:55-110),
// spelled on the integer word so no floating-point mode can touch it.
__device__ __forceinline__ float store_word(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7F800000u) == 0u) u &= 0x80000000u;
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) u = 0x7FC00000u;
  return __uint_as_float(u);
}

typedef __attribute__((address_space(3))) void* lds_vptr;
typedef __attribute__((address_space(1))) void* gbl_vptr;

template <int T>
struct Elem {
  static constexpr int bytes = T == T_F32 ? 4 : (T == T_BF16 ? 2 : 1);
  static constexpr int per16 = 16 / bytes;  // elements per 16-byte chunk
};

// Word 3 of a raw buffer resource on gfx9-family targets (32-bit data format, no swizzle).
constexpr int RSRC_WORD3 = 0x00020000;

// Upper tree levels: fold `ngroups` group roots per cell (a subtree per aligned group,
// so the rest of the contract's tree is the same rule applied to the roots).
// The same rule for up to 2^20 scalar partials (twenty levels), slots named.
struct StackF {
  float s0, s1, s2, s3, s4, s5, s6, s7, s8, s9, s10, s11, s12, s13, s14, s15, s16, s17, s18, s19;
#define MLG_PUSH_LEVEL(L)                      \
  if (!((t >> L) & 1)) { s##L = x; return; } \
  x = s##L + x;
  __device__ __forceinline__ void push(float x, int t) {
    MLG_PUSH_LEVEL(0) MLG_PUSH_LEVEL(1) MLG_PUSH_LEVEL(2) MLG_PUSH_LEVEL(3) MLG_PUSH_LEVEL(4)
    MLG_PUSH_LEVEL(5) MLG_PUSH_LEVEL(6) MLG_PUSH_LEVEL(7) MLG_PUSH_LEVEL(8) MLG_PUSH_LEVEL(9)
    MLG_PUSH_LEVEL(10) MLG_PUSH_LEVEL(11) MLG_PUSH_LEVEL(12) MLG_PUSH_LEVEL(13) MLG_PUSH_LEVEL(14)
    MLG_PUSH_LEVEL(15) MLG_PUSH_LEVEL(16) MLG_PUSH_LEVEL(17) MLG_PUSH_LEVEL(18)
    s19 = x;
  }
#undef MLG_PUSH_LEVEL
#define MLG_ROOT_LEVEL(L) \
  if ((t >> L) & 1) x = s##L + x;
  __device__ __forceinline__ float root(float x, int t) const {
    MLG_ROOT_LEVEL(0) MLG_ROOT_LEVEL(1) MLG_ROOT_LEVEL(2) MLG_ROOT_LEVEL(3) MLG_ROOT_LEVEL(4)
    MLG_ROOT_LEVEL(5) MLG_ROOT_LEVEL(6) MLG_ROOT_LEVEL(7) MLG_ROOT_LEVEL(8) MLG_ROOT_LEVEL(9)
    MLG_ROOT_LEVEL(10) MLG_ROOT_LEVEL(11) MLG_ROOT_LEVEL(12) MLG_ROOT_LEVEL(13) MLG_ROOT_LEVEL(14)
    MLG_ROOT_LEVEL(15) MLG_ROOT_LEVEL(16) MLG_ROOT_LEVEL(17) MLG_ROOT_LEVEL(18) MLG_ROOT_LEVEL(19)
    return x;
  }
#undef MLG_ROOT_LEVEL
};

}  // namespace mlg

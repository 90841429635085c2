// The skinny-M (decode GEMV) kernels (gemv_nn.hip, gemv_nt.hip): constants, argument block, launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "contract.h"

namespace mlg {

// Skinny-M product (decode GEMV), OP_NN: X[M x K] . W[K x N], M <= 16.
//
// A wave owns one k-leaf of one column group.  Each lane owns CPL = 4 / bytes consecutive
// columns: one 32-bit word of W per k row (4 int8 codes, 2 bf16 or 1 float32), so the 64
// lanes read 256 contiguous bytes of every W row -- except int8 with whole 128-row leaves,
// where a lane owns 2 columns (a 16-bit word, 128 bytes a wave): twice the waves over the
// same bytes, each with half the conversions and chain steps, and more loads in flight.  The leaf's rows stream into registers
// GV_CH at a time, two buffers requested before the first arithmetic (a whole 128-row leaf
// is in flight at once), and each lane runs CPL x M serial chains in VALU (v_fma_f32 under
// MODE.FP_DENORM = 2 is fma(ftz a, ftz b, ftz acc), like the K=1 MFMA).  x is the same for
// every lane and is read with uniform loads.  A 256-thread workgroup is one column group's
// aligned group of GV_LEAVES leaves -- a subtree of the fold -- whose root it forms through
// LDS.  With more than one group, the roots go to the workspace with agent-scope atomic
// stores and are counted on the column group's counter; the workgroup that completes the
// count folds them (the rest of the contract's tree), writes the output and resets the
// counter.  One launch computes the whole product.  With whole 128-row leaves a workgroup
// may hold GV_WIDE_LEAVES leaves instead (half the groups to fold) when the launch still
// has a workgroup for every CU.
constexpr int GV_THREADS = 256;
constexpr int GV_LEAVES = GV_THREADS / 64;  // leaves per workgroup: an aligned subtree
constexpr int GV_WIDE_LEAVES = 8;
constexpr int GV_MAXM = 16;
constexpr int GV_CH = 128;                  // W rows per register buffer: a whole contract leaf
constexpr int GV_FOLD_BATCH = 16;           // root loads in flight while folding
constexpr int GV_FEW_GROUPS = 8;            // up to this many groups: all roots loaded at once
constexpr int GV_NT = 2;                    // buffer-load cache policy nt: streamed, not kept

// Columns per lane: OP_NT one; OP_NN one 32-bit word, or (FULL: whole 128-row leaves) a
// 16-bit word of int8 codes.
constexpr int gv_cpl(int bt, bool nt, bool full) {
  return nt ? 1 : (bt == T_F32 ? 1 : (bt == T_BF16 || full ? 2 : 4));
}

template <int T, bool NT = false, bool FULL = false>
struct GvCols {
  static constexpr int cpl = gv_cpl(T, NT, FULL);  // columns per lane
  static constexpr int cols = 64 * cpl;            // columns per group
};

struct GemvArgs {
  float* c;
  const void* w;
  const float* scales;
  const float* bias;
  float* ws;              // [ngroups][m][n] group roots when ngroups > 1
  unsigned int* counter;  // [ncg], zero between launches (ngroups > 1)
  int64_t m, n, k, leaf, nleaves;
  int64_t ngroups;        // ceil(nleaves / leaves per workgroup)
  int64_t ncg;            // column groups
};

// OP_NN with whole 128-row leaves and at least this many rows of X: the chains on the matrix
// cores (gemv_mfma.hip; X 16-byte aligned, 16 * K * 4 < 2^31).  Its workgroups are twice as
// wide: MF_LEAVES leaves (an aligned subtree of 8) per workgroup, so the cross-workgroup fold
// has half the roots.
constexpr int GV_MFMA_MIN_M = 9;
// ... and from this many rows up to GV_MFMA4_MAX_M, on the 4 x 4 shape.
constexpr int GV_MFMA4_MIN_M = 3;
constexpr int GV_MFMA4_MAX_M = 8;
constexpr int MF4_LEAVES = 8;  // leaves per workgroup of the 4 x 4 kernel
constexpr int MF4_THREADS = 64 * MF4_LEAVES;
constexpr int MF_THREADS = 512;
constexpr int MF_LEAVES = MF_THREADS / 64;
// Columns a lane of the matrix-core kernels: int8 weights take 16-bit lanes (2 codes, 128-column
// groups: twice the workgroups, two a CU); bf16 and f32 one 32-bit word.
constexpr int mf_cpl(int bt) { return bt == 2 ? 2 : (bt == 1 ? 2 : 1); }

// vec (OP_NN): 0 element loads, 1 word (buffer) loads, 2 word loads of whole 128-row leaves
// (`leaves` per workgroup: GV_LEAVES, or GV_WIDE_LEAVES with vec 2).
hipError_t launch_gemv_nn(const GemvArgs& g, const float* x, int b_type, int64_t m, int vec, int leaves, dim3 grid,
                          hipStream_t stream);
hipError_t launch_gemv_mfma_nn(const GemvArgs& g, const float* x, int b_type, dim3 grid, hipStream_t stream);
// 2 <= m <= 8 on the 4 x 4 shape (same conditions as the 16 x 16 kernel).
hipError_t launch_gemv_mfma4_nn(const GemvArgs& g, const float* x, int b_type, int64_t m, dim3 grid,
                                hipStream_t stream);
// The decode-packed int8 layout (gemv_packed.hip): 64-column groups, `waves` a workgroup:
// PK_WAVES_WHOLE (16 waves of two leaves: 32 leaves, the whole tree at K = 4096) when the launch
// fills the CUs, else 4-leaf groups whose roots fold across workgroups (PK_WAVES_SPLIT: two waves
// of two leaves on the matrix cores, four waves of one leaf on the VALU).
constexpr int PK_GROUP_COLS = 64;
constexpr int PK_WAVES_WHOLE = 16;
constexpr int PK_WAVES_SPLIT = 2;
hipError_t launch_gemv_packed(const GemvArgs& g, const float* x, int waves, dim3 grid, hipStream_t stream);
// The same product on the matrix cores for 3 <= m <= 16 (x 16-byte aligned, m * k * 4 < 2^31).
constexpr int PK_MFMA_MIN_M = 3;
hipError_t launch_gemv_packed_mfma(const GemvArgs& g, const float* x, int waves, dim3 grid, hipStream_t stream);
hipError_t launch_int8w_pack(void* dst, const void* codes, int64_t k, int64_t n, hipStream_t stream);
// vec (OP_NT): 0 element loads, 1 16-byte loads.
hipError_t launch_gemv_nt(const GemvArgs& g, const float* x, int b_type, int64_t m, int vec, dim3 grid,
                          hipStream_t stream);

}  // namespace mlg

// The MFMA GEMM kernel (gemm_mfma.hip): tile constants, argument block, launchers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlg {

// Tiling: 512 threads = 8 waves (2 per SIMD); workgroup tile 128 x 128 cells; each wave owns
// 64 rows x 32 columns = one v_mfma_f32_32x32x1_2b_f32 per k step (block 0 = rows 0-31,
// block 1 = rows 32-63, both against the same 32 columns).  K is staged through LDS in
// KT = 32-step slices, three buffers (loads issued two slices ahead).  Operands travel
// HBM -> LDS with buffer loads straight into LDS (16 bytes per lane, no registers) in their
// stored element type; bf16 widening and int8 x column-scale dequantisation happen when a
// lane reads its MFMA operand out of LDS.
constexpr int NTHREADS = 512;
constexpr int NWAVES = NTHREADS / 64;
constexpr int BM = 128;
constexpr int BN = 128;
constexpr int KT = 32;
constexpr int SLICE_BYTES = BM * KT * 4;  // one operand slice at float32: 16 KB
constexpr int NBUF = 3;                   // slices in LDS: loads run two slices ahead
constexpr int MAX_GROUP_LEAVES = 32;      // one group's leaves fold in registers + one LDS slot

struct GemmArgs {
  float* c;
  const void* a;      // stored operands: 16-byte aligned, rows a multiple of 16 bytes
  const void* b;
  const float* scales;
  const float* bias;
  float* ws;          // group roots [ngroups][m][n] when ngroups > 1
  int64_t m, n, k;
  int64_t leaf;       // L
  int64_t nleaves;    // P
  int64_t group;      // leaves per group (power of two, <= 32)
  int64_t ngroups;
  int64_t a_pitch, b_pitch;  // stored row lengths in elements
  int64_t a_bytes, b_bytes;  // stored operand sizes
  int tiles_m, tiles_n;
  int64_t ldc;        // C row stride
  int seed;           // one leaf: the chain starts from the old C cell
  // the store's follower (act.h follow_one): 0 none, 3 PLUS_BIAS (epi_p[j]), 4 BIAS_ACT
  // (epi_p[j], activation `act`), 5 ACT_BWD (epi_p[i n + j], activation `act`)
  int epi, act;
  const float* epi_p;
};

// XCDs of the device: workgroup b of a launch runs on XCD b % XCDS (round-robin dispatch).
constexpr int XCDS = 8;
// Row tiles walked together: an XCD's 32 concurrent tiles form a block of 4 row tiles x 8
// column tiles, sharing A row panels and B column panels in its L2.
constexpr int TILE_BAND = 4;

// The tile of workgroup b among nb = tm x tn.  Workgroup b runs on XCD b % XCDS; the remap
// gives XCD x a contiguous range of the tile sequence, in the order it dispatches them, and
// the sequence walks bands of TILE_BAND row tiles column by column, so the 32 tiles an XCD runs
// at once form a TILE_BAND x 8 block: the A row panels and B column panels they read are shared
// in that XCD's L2 instead of fetched by every XCD.  A bijection of [0, nb): which tile a
// workgroup computes never changes a cell's arithmetic.
__device__ __forceinline__ int tile_of(int b, int nb, int tm, int tn) {
  const int q = nb / XCDS, r = nb % XCDS;
  const int x = b % XCDS, s = b / XCDS;
  const int seq = (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + s;
  const int band = seq / (TILE_BAND * tn);
  const int rows = tm - band * TILE_BAND < TILE_BAND ? tm - band * TILE_BAND : TILE_BAND;
  const int local = seq - band * TILE_BAND * tn;
  return (band * TILE_BAND + local % rows) * tn + local / rows;
}

// Launch gemm_mfma_kernel<op, a_type, b_type> on `grid` (tiles, leaf groups).
hipError_t launch_mfma(const GemmArgs& g, int op, int a_type, int b_type, dim3 grid, hipStream_t stream);

// Copy [rows][cols] elements of `eb` bytes, element (r, c) at src[r * s_r + c * s_c], into
// [rows][pitch], zero padding.
hipError_t launch_repack(char* dst, const char* src, int64_t rows, int64_t cols, int64_t pitch, int eb,
                         int64_t s_r, int64_t s_c, hipStream_t stream);

// Fold `ngroups` group roots ws[g][m][n] per cell (0 groups: store +0.0), apply the store's
// follower `epi` (as GemmArgs), store.
hipError_t launch_fold_groups(float* c, int64_t ldc, const float* ws, int64_t m, int64_t n, int64_t ngroups,
                              int epi, const float* epi_p, int act, hipStream_t stream);

}  // namespace mlg

// gfx950 skinny-M kernel on the matrix cores, OP_NN with whole 128-row leaves: X[M x K] . W[K x N]
// for 5 <= M <= 16 (the decode batches whose VALU chains would outweigh the weight stream).
//
// Same work split as gemv_nn_kernel: a wave owns one k-leaf of one column group, a lane one
// 32-bit word of every W row (CPL columns), the rows streamed through a register ring.  The
// chains run on v_mfma_f32_16x16x1_4b_f32: four 16 x 16 blocks with K = 1, one fma_rn per output
// element (under MODE.FP_DENORM = 2 it is fma(ftz a, ftz b, ftz c), like v_fma_f32 and the
// K=1 MFMA of the tile kernel).  For byte e of the lane words, lane l feeds A = x[l % 16][p]
// and B = W[p][CPL*l + e], so block l / 16 of the instruction computes rows 0..15 of the 16
// columns {CPL*(16*(l/16) + j) + e : j < 16}; one instruction per word byte per k step
// advances 16 x 64 chains by one step.  The leaf's first step takes +0 as its C operand.
// The epilogue (leaf partials through LDS, the group's subtree, the cross-workgroup fold)
// is gemv_nn_kernel's.
#include "gemv_body.h"

namespace mlg {

typedef float v16f __attribute__((ext_vector_type(16)));

// The wave's x block, rows 0..15 (rows past m repeat row m-1) by the leaf's 128 steps, staged
// in its own LDS area xs[16][GV_CH] before the W ring is requested: x then comes from LDS
// (lgkmcnt) and never makes the loop wait behind the ring's loads (vmcnt is in order).
constexpr int GV_XS = 16 * GV_CH;  // floats of one wave's x block
constexpr int MF_RB = 16;          // W rows per ring block
constexpr int MF_AHEAD = 3;        // blocks requested ahead of the one being consumed

// The lane's CPL columns of one W row from its loaded bits u: bf16 widened exactly, int8
// f32(code) * scale (one rounding; the scale flushed on input by MODE.FP_DENORM = 2).
template <int BT, int CPL>
__device__ __forceinline__ void mf_weights(uint32_t u, const float (&sc)[CPL], float (&wv)[CPL]) {
  if constexpr (BT == T_F32) {
    wv[0] = __uint_as_float(u);
  } else if constexpr (BT == T_BF16) {
    wv[0] = __uint_as_float(u << 16);
    if constexpr (CPL > 1) wv[1] = __uint_as_float(u & 0xFFFF0000u);
  } else {
#pragma unroll
    for (int e = 0; e < CPL; ++e) wv[e] = (float)((int32_t)(u << (24 - 8 * e)) >> 24) * sc[e];
  }
}

// CPL columns a lane: one 32-bit word of every W row, or (CPL * bytes == 2) one 16-bit half.
template <int BT, int CPL>
__device__ __forceinline__ void gv_leaf_mfma(v16f (&acc)[CPL], const char* wleaf, uint32_t loff,
                                             int rowbytes, const float* __restrict__ xl, int64_t k, int m,
                                             float* xs, int lane, const float (&sc)[CPL]) {
  constexpr bool HALF = CPL * Elem<BT>::bytes == 2;
  constexpr int NBLK = GV_CH / MF_RB;
  constexpr int RING = MF_AHEAD + 1;
  // lane l stages row l / 4, steps 32 * (l % 4) .. +31 (x + kb is 16-byte aligned: the host
  // requires an aligned x and k a multiple of 128).  The x loads go out first and the W ring's
  // right after them; the LDS writes then wait for x alone (loads complete in order), so the
  // weight stream is never held behind x's latency.
  const int xr = lane >> 2;
  const f4* src = reinterpret_cast<const f4*>(xl + (int64_t)(xr < m ? xr : m - 1) * k + 32 * (lane & 3));
  f4 xv[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) xv[c] = src[c];
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(wleaf), (short)0, 0x7FFFFFFF, RSRC_WORD3);

  uint32_t ring[RING][MF_RB];
  auto load_row = [&](int row) -> uint32_t {
    if constexpr (HALF) return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)loff, row * rowbytes, 0);
    else return __builtin_amdgcn_raw_buffer_load_b32(rs, (int)loff, row * rowbytes, 0);
  };
#pragma unroll
  for (int b = 0; b < MF_AHEAD; ++b)
#pragma unroll
    for (int i = 0; i < MF_RB; ++i) ring[b][i] = load_row(b * MF_RB + i);
  {
    f4* dst = reinterpret_cast<f4*>(xs + xr * GV_CH + 32 * (lane & 3));
#pragma unroll
    for (int c = 0; c < 8; ++c) dst[c] = xv[c];
  }
  // x[row][p .. p+3] for this lane's row (l % 16), four steps per LDS read, one read ahead in a
  // two-entry buffer indexed by the (unrolled) group's parity, so no register is copied
  const f4* xrow = reinterpret_cast<const f4*>(xs + (lane & 15) * GV_CH);
  f4 xb[2];
  xb[0] = xrow[0];

#pragma unroll
  for (int b = 0; b < NBLK; ++b) {
    if (b + MF_AHEAD < NBLK) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MF_RB; ++i) ring[(b + MF_AHEAD) % RING][i] = load_row((b + MF_AHEAD) * MF_RB + i);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q0 = 0; q0 < MF_RB; q0 += 4) {
      const int s0 = b * MF_RB + q0;
      const int xg = s0 / 4;
      if (s0 + 4 < GV_CH) xb[(xg + 1) & 1] = xrow[xg + 1];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float wv[CPL];
        mf_weights<BT, CPL>(ring[b % RING][q0 + q], sc, wv);
        const float xa = xb[xg & 1][q];
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
          if (s0 + q == 0) acc[e] = __builtin_amdgcn_mfma_f32_16x16x1f32(xa, wv[e], v16f{}, 0, 0, 0);
          else acc[e] = __builtin_amdgcn_mfma_f32_16x16x1f32(xa, wv[e], acc[e], 0, 0, 0);
        }
      }
    }
  }
}

// CPL columns a lane (mf_cpl): with 16-bit lanes two workgroups share a CU (their leaf partials
// and x blocks take 64 KB of LDS each, and the registers are held to four waves a SIMD).
template <int BT, int CPL>
__global__ void __launch_bounds__(MF_THREADS, CPL * Elem<BT>::bytes == 2 ? 2 : 1)
gemv_mfma_nn_kernel(GemvArgs g, const float* __restrict__ x) {
  constexpr int MR = GV_MAXM;
  constexpr int COLS = 64 * CPL;
  constexpr int EB = Elem<BT>::bytes;
  // The waves' leaf partials; a wave's x block lives in its own partial area while it runs
  // its leaf when that area is large enough (int8, bf16), else in an area of its own (f32).
  constexpr int PART = MR * COLS;
  constexpr int XOWN = PART >= GV_XS ? 0 : GV_XS;
  __shared__ __attribute__((aligned(16))) float part[MF_LEAVES][MR][COLS];
  __shared__ __attribute__((aligned(16))) float xown[MF_LEAVES][XOWN > 0 ? XOWN : 1];
  __shared__ unsigned int last_flag;

  set_flush_inputs_mode();
  gv_fetch_args(g, x);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the grid holds at most INT32_MAX workgroups (the host refuses more): a 32-bit split
  const int64_t cg = blockIdx.x % (uint32_t)g.ncg;
  const int64_t grp = blockIdx.x / (uint32_t)g.ncg;
  const int64_t t = grp * MF_LEAVES + wave;  // this wave's leaf
  const int m = (int)g.m;

  v16f acc[CPL];
#pragma unroll
  for (int e = 0; e < CPL; ++e) acc[e] = v16f{};

  if (t < g.nleaves) {
    // this lane's columns, clamped into the operand (their cells are never stored)
    int64_t c0 = cg * COLS + lane * CPL;
    if (c0 >= g.n) c0 = g.n - CPL;
    float sc[CPL];
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      sc[e] = 1.f;
      if constexpr (BT == T_I8) sc[e] = g.scales[c0 + e];
    }
    const int64_t rowbytes = g.n * EB;
    const int64_t kb = t * GV_CH;
    gv_leaf_mfma<BT, CPL>(acc, static_cast<const char*>(g.w) + kb * rowbytes, (uint32_t)(c0 * EB), (int)rowbytes,
                     x + kb, g.k, m, XOWN > 0 ? &xown[wave][0] : &part[wave][0][0], lane, sc);
  }

  // Lane l holds, for word byte e and block blk, rows 4*(l/16)+i of column
  // CPL*(16*blk + l%16) + e in acc[e][4*blk + i].
#pragma unroll
  for (int e = 0; e < CPL; ++e)
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        part[wave][4 * (lane >> 4) + i][CPL * (16 * blk + (lane & 15)) + e] = acc[e][4 * blk + i];
  gv_finish<MR, COLS, MF_LEAVES, MF_THREADS>(g, part, last_flag, tid, grp, cg, m);
}

// ---- 2 <= M <= 8 on v_mfma_f32_4x4x1_16b_f32: sixteen 4 x 4 blocks with K = 1, one fma_rn
// per output element like the other K = 1 shapes.  Output lane l, register r holds
// A[lane 4 (l / 4) + r] * B[lane l] (+ C): lane l feeds A = x[4 g + l % 4][p] (its block's four
// lanes carry rows 4g .. 4g+3) and B = W[p][CPL l + e], and gets column CPL l + e of those four
// rows back.  G groups of four rows, CPL instructions per group per k step: no row is wasted
// below M = 4 (the 16 x 16 shape computes 16).
typedef float v4f __attribute__((ext_vector_type(4)));

template <int BT, int G, int CPL>
__device__ __forceinline__ void gv_leaf_mfma4(v4f (&acc)[G][CPL], const char* wleaf, uint32_t loff, int rowbytes,
                                              const float* __restrict__ xl, int64_t k, int m, float* xs, int lane,
                                              const float (&sc)[CPL]) {
  constexpr bool HALF = CPL * Elem<BT>::bytes == 2;
  constexpr int NBLK = GV_CH / MF_RB;
  constexpr int RING = MF_AHEAD + 1;
  // x rows 0 .. 4G-1 (rows past m repeat row m-1) by the leaf's 128 steps into xs[4G][GV_CH]:
  // 32 f4 a row, 2G f4 a lane (x + kb is 16-byte aligned, k a multiple of 128).  As in the
  // 16 x 16 kernel, x is requested first, the W ring right after, and the LDS writes wait for
  // x alone.
  f4 xv[2 * G];
#pragma unroll
  for (int c = 0; c < 2 * G; ++c) {
    const int idx = lane + 64 * c;
    const int r = idx >> 5, q = idx & 31;
    xv[c] = reinterpret_cast<const f4*>(xl + (int64_t)(r < m ? r : m - 1) * k)[q];
  }
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(wleaf), (short)0, 0x7FFFFFFF, RSRC_WORD3);
  auto load_row = [&](int row) -> uint32_t {
    if constexpr (HALF) return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)loff, row * rowbytes, 0);
    else return __builtin_amdgcn_raw_buffer_load_b32(rs, (int)loff, row * rowbytes, 0);
  };
  uint32_t ring[RING][MF_RB];
#pragma unroll
  for (int b = 0; b < MF_AHEAD; ++b)
#pragma unroll
    for (int i = 0; i < MF_RB; ++i) ring[b][i] = load_row(b * MF_RB + i);
#pragma unroll
  for (int c = 0; c < 2 * G; ++c) {
    const int idx = lane + 64 * c;
    reinterpret_cast<f4*>(xs + (idx >> 5) * GV_CH)[idx & 31] = xv[c];
  }
  const f4* xrow[G];
  f4 xb[2][G];  // one read ahead, indexed by the (unrolled) group's parity: no register copies
#pragma unroll
  for (int g = 0; g < G; ++g) {
    xrow[g] = reinterpret_cast<const f4*>(xs + (4 * g + (lane & 3)) * GV_CH);
    xb[0][g] = xrow[g][0];
  }
#pragma unroll
  for (int b = 0; b < NBLK; ++b) {
    if (b + MF_AHEAD < NBLK) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < MF_RB; ++i) ring[(b + MF_AHEAD) % RING][i] = load_row((b + MF_AHEAD) * MF_RB + i);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q0 = 0; q0 < MF_RB; q0 += 4) {
      const int s0 = b * MF_RB + q0;
      const int xg = s0 / 4;
      if (s0 + 4 < GV_CH) {
#pragma unroll
        for (int g = 0; g < G; ++g) xb[(xg + 1) & 1][g] = xrow[g][xg + 1];
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float wv[CPL];
        mf_weights<BT, CPL>(ring[b % RING][q0 + q], sc, wv);
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float xa = xb[xg & 1][g][q];
#pragma unroll
          for (int e = 0; e < CPL; ++e) {
            if (s0 + q == 0) acc[g][e] = __builtin_amdgcn_mfma_f32_4x4x1f32(xa, wv[e], v4f{}, 0, 0, 0);
            else acc[g][e] = __builtin_amdgcn_mfma_f32_4x4x1f32(xa, wv[e], acc[g][e], 0, 0, 0);
          }
        }
      }
    }
  }
}

// CPL columns a lane (mf_cpl), as in the 16 x 16 kernel.
template <int BT, int G, int CPL>
__global__ void __launch_bounds__(MF4_THREADS, CPL * Elem<BT>::bytes == 2 ? 2 : 1)
gemv_mfma4_nn_kernel(GemvArgs g, const float* __restrict__ x) {
  constexpr int MR = 4 * G;
  constexpr int COLS = 64 * CPL;
  constexpr int EB = Elem<BT>::bytes;
  constexpr int XS = MR * GV_CH;  // floats of one wave's x block
  __shared__ __attribute__((aligned(16))) float part[MF4_LEAVES][MR][COLS];
  __shared__ __attribute__((aligned(16))) float xown[MF4_LEAVES][XS];
  __shared__ unsigned int last_flag;

  set_flush_inputs_mode();
  gv_fetch_args(g, x);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the grid holds at most INT32_MAX workgroups (the host refuses more): a 32-bit split
  const int64_t cg = blockIdx.x % (uint32_t)g.ncg;
  const int64_t grp = blockIdx.x / (uint32_t)g.ncg;
  const int64_t t = grp * MF4_LEAVES + wave;  // this wave's leaf
  const int m = (int)g.m;

  v4f acc[G][CPL];
#pragma unroll
  for (int gg = 0; gg < G; ++gg)
#pragma unroll
    for (int e = 0; e < CPL; ++e) acc[gg][e] = v4f{};

  if (t < g.nleaves) {
    // this lane's columns, clamped into the operand (their cells are never stored)
    int64_t c0 = cg * COLS + lane * CPL;
    if (c0 >= g.n) c0 = g.n - CPL;
    float sc[CPL];
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      sc[e] = 1.f;
      if constexpr (BT == T_I8) sc[e] = g.scales[c0 + e];
    }
    const int64_t rowbytes = g.n * EB;
    const int64_t kb = t * GV_CH;
    gv_leaf_mfma4<BT, G, CPL>(acc, static_cast<const char*>(g.w) + kb * rowbytes, (uint32_t)(c0 * EB),
                              (int)rowbytes, x + kb, g.k, m, &xown[wave][0], lane, sc);
  }

  // lane l: rows 4 gg + r of column CPL l + e in acc[gg][e][r]
#pragma unroll
  for (int gg = 0; gg < G; ++gg)
#pragma unroll
    for (int e = 0; e < CPL; ++e)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[wave][4 * gg + r][CPL * lane + e] = acc[gg][e][r];
  gv_finish<MR, COLS, MF4_LEAVES, MF4_THREADS>(g, part, last_flag, tid, grp, cg, m);
}

hipError_t launch_gemv_mfma4_nn(const GemvArgs& g, const float* x, int b_type, int64_t m, dim3 grid,
                                hipStream_t stream) {
  const bool two = m > 4;
#define MLG_MF4(BT)                                                                                               \
  do {                                                                                                            \
    if (two) hipLaunchKernelGGL((gemv_mfma4_nn_kernel<BT, 2, mf_cpl(BT)>), grid, dim3(MF4_THREADS), 0, stream, g, x); \
    else hipLaunchKernelGGL((gemv_mfma4_nn_kernel<BT, 1, mf_cpl(BT)>), grid, dim3(MF4_THREADS), 0, stream, g, x);     \
  } while (0)
  if (b_type == T_F32) MLG_MF4(T_F32);
  else if (b_type == T_BF16) MLG_MF4(T_BF16);
  else MLG_MF4(T_I8);
#undef MLG_MF4
  return hipGetLastError();
}

hipError_t launch_gemv_mfma_nn(const GemvArgs& g, const float* x, int b_type, dim3 grid, hipStream_t stream) {
  if (b_type == T_F32)
    hipLaunchKernelGGL((gemv_mfma_nn_kernel<T_F32, mf_cpl(T_F32)>), grid, dim3(MF_THREADS), 0, stream, g, x);
  else if (b_type == T_BF16)
    hipLaunchKernelGGL((gemv_mfma_nn_kernel<T_BF16, mf_cpl(T_BF16)>), grid, dim3(MF_THREADS), 0, stream, g, x);
  else hipLaunchKernelGGL((gemv_mfma_nn_kernel<T_I8, mf_cpl(T_I8)>), grid, dim3(MF_THREADS), 0, stream, g, x);
  return hipGetLastError();
}

}  // namespace mlg

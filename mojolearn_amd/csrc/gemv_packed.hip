// gfx950 decode GEMV on int8 weights in the decode-packed layout, and the kernel that packs them.
//
// The row-major decode kernel (gemv_nn_kernel) cannot give one workgroup every leaf of its
// columns: a 64-column strip of a row-major int8 matrix is 64-byte row segments, which read at
// half the speed of 256-byte ones, so its workgroups hold 4 or 8 leaves of 128 columns and the
// leaf groups of a column meet through a cross-workgroup fold (roots to memory, a counter, the
// last workgroup reloading them).  The packed layout makes a 64-column group contiguous:
// code (p, j) -- leaf t = p / 128, block s = (p % 128) / 16 (sixteen rows), row i = p % 16,
// column group cg = j / 64, lane l = j % 64 -- lives at byte
//
//     ((s * P + t) * ncg + cg) * 1024 + l * 16 + i        (P leaves, ncg column groups),
//
// so one 16-byte load gives a lane sixteen rows of its column, the waves of a group read whole
// 1 KB chunks, and block s of every leaf is one contiguous slab of P * ncg KB that the waves,
// which advance together, read at the same time.  A workgroup of 16 waves, each running two
// adjacent leaves, then holds 32 leaves of 64 columns: at K = 4096 the whole contract tree of
// its columns, folded in LDS with no workspace, no counter and no second pass.  Columns past n
// are packed as zero codes and never stored.  The arithmetic and its order are gemv_nn_kernel's:
// per leaf the chain acc = fma(x, f32(code) * scale, acc) in step order from +0, the level-1
// pair of a wave's two leaves added in registers, the rest of the tree over the workgroup's
// pairs (gv_finish, PAIRED), and past 32 leaves the group roots folded by the workgroup that
// completes the count -- so the bits are the row-major product's.
#include "gemv_body.h"

namespace mlg {

constexpr int PK_COLS = 64;              // columns a group: one a lane
constexpr int PK_RB = 16;                // rows a block: one 16-byte load a lane
constexpr int PK_BLOCKS = GV_CH / PK_RB; // 8 blocks a 128-row leaf
constexpr int PK_CHUNK_THREADS = 256;
// Whole-column workgroups request two blocks ahead of the one consumed (measured at M = 1, on
// rotating 58.7 MB weights: 1, 2, 3, 4 and 8 blocks 11.6, 11.5, 11.6, 12.6 and 11.9 us).
constexpr int PK_AHEAD = 2;
// The weight loads are non-temporal (cache policy nt: streamed, not kept in L2): 12.4 -> 11.5 us.
constexpr int PK_AUX = 2;

// One thread per 16-byte chunk (block s, leaf t, group cg, lane l), chunk index
// ((s * P + t) * ncg + cg) * 64 + l: it gathers rows 16s .. 16s+15 of leaf t at column
// 64 cg + l (zero past n) and writes them in row order.
__global__ void __launch_bounds__(PK_CHUNK_THREADS) int8w_pack_kernel(u4* __restrict__ dst,
                                                                      const uint8_t* __restrict__ codes, int64_t n,
                                                                      int64_t P, int64_t ncg, int64_t chunks) {
  const int64_t chunk = (int64_t)blockIdx.x * PK_CHUNK_THREADS + threadIdx.x;
  if (chunk >= chunks) return;
  const int l = (int)(chunk % 64);
  int64_t r = chunk / 64;
  const int64_t cg = r % ncg;
  r /= ncg;
  const int64_t t = r % P;
  const int64_t s = r / P;
  const int64_t p0 = t * GV_CH + s * PK_RB;
  const int64_t j = cg * PK_COLS + l;
  uint32_t w[4] = {0, 0, 0, 0};
  if (j < n) {
#pragma unroll
    for (int i = 0; i < PK_RB; ++i) w[i >> 2] |= (uint32_t)codes[(p0 + i) * n + j] << (8 * (i & 3));
  }
  dst[chunk] = u4{w[0], w[1], w[2], w[3]};
}

// NL adjacent leaves of one lane's column from the packed layout: block s of leaf q at
// base + s * slab + q * lstride (+ lane * 16), AHEAD blocks requested ahead of the one
// consumed.  x is read XB steps at a time (uniform loads) one batch ahead.  acc[q][r] is leaf
// q's chain for row r.
template <int MR, int NL, int AHEAD>
__device__ __forceinline__ void gv_leaves_packed(float (&acc)[NL][MR], const char* base, int64_t slab,
                                                 int lstride, int lane, const float* __restrict__ xl, int64_t k,
                                                 int m, float sc) {
  constexpr int XB = MR * NL <= 2 ? 8 : (16 / (MR * NL) < 2 ? 2 : 16 / (MR * NL));  // steps a batch
  auto block_rs = [&](int s) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base) + s * slab, (short)0, 0x7FFFFFFF, RSRC_WORD3);
  };
  const float* xr[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) xr[r] = xl + (r < m ? r : m - 1) * k;  // rows past m: never stored
  u4 ring[PK_BLOCKS][NL];
#pragma unroll
  for (int s = 0; s < AHEAD; ++s)
#pragma unroll
    for (int q = 0; q < NL; ++q)
      ring[s][q] = __builtin_amdgcn_raw_buffer_load_b128(block_rs(s), lane * 16, q * lstride, PK_AUX);
  float xc[MR][NL][XB], xn[MR][NL][XB];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < NL; ++q)
#pragma unroll
      for (int i = 0; i < XB; ++i) xc[r][q][i] = xr[r][q * GV_CH + i];
#pragma unroll
  for (int s = 0; s < PK_BLOCKS; ++s) {
    if (s + AHEAD < PK_BLOCKS) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < NL; ++q)
        ring[s + AHEAD][q] =
            __builtin_amdgcn_raw_buffer_load_b128(block_rs(s + AHEAD), lane * 16, q * lstride, PK_AUX);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i0 = 0; i0 < PK_RB; i0 += XB) {
      const int s0 = s * PK_RB + i0;  // the leaf step of this batch's first value
      if (s0 + XB < GV_CH) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
          for (int q = 0; q < NL; ++q)
#pragma unroll
            for (int i = 0; i < XB; ++i) xn[r][q][i] = xr[r][q * GV_CH + s0 + XB + i];
      }
#pragma unroll
      for (int i = 0; i < XB; ++i) {
        const int b = i0 + i;  // byte of the chunk: row 16s + b of the leaf
#pragma unroll
        for (int q = 0; q < NL; ++q) {
          const uint32_t u = ring[s][q][b >> 2];
          // f32(code) * scale, one rounding (the scale flushed on input by MODE.FP_DENORM = 2)
          const float w = (float)((int32_t)(u << (24 - 8 * (b & 3))) >> 24) * sc;
#pragma unroll
          for (int r = 0; r < MR; ++r) acc[q][r] = __builtin_fmaf(xc[r][q][i], w, acc[q][r]);
        }
      }
      if (s0 + XB < GV_CH) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
          for (int q = 0; q < NL; ++q)
#pragma unroll
            for (int i = 0; i < XB; ++i) xc[r][q][i] = xn[r][q][i];
      }
    }
  }
}

// WAVES waves a workgroup, each running two adjacent leaves of the workgroup's 64 columns
// (2 * WAVES leaves: an aligned subtree).  g.w is the packed buffer, g.nleaves = P, g.ncg the
// column groups of 64.
template <int MR, int WAVES, int AHEAD>
__global__ void __launch_bounds__(64 * WAVES) gemv_packed_kernel(GemvArgs g, const float* __restrict__ x) {
  constexpr int LEAVES = 2 * WAVES;
  __shared__ float part[WAVES][MR][PK_COLS];
  __shared__ unsigned int last_flag;

  set_flush_inputs_mode();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the grid holds at most INT32_MAX workgroups (the host refuses more): a 32-bit split
  const int64_t cg = blockIdx.x % (uint32_t)g.ncg;
  const int64_t grp = blockIdx.x / (uint32_t)g.ncg;
  const int64_t t0 = grp * LEAVES + 2 * wave;  // this wave's first leaf
  const int m = (int)g.m;

  float y[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) y[r] = 0.f;

  if (t0 < g.nleaves) {
    // this lane's scale, its column clamped into [0, n) (columns past n are never stored)
    const int64_t j = cg * PK_COLS + lane;
    const float sc = g.scales[j < g.n ? j : g.n - 1];
    const int64_t slab = g.nleaves * g.ncg * 1024;  // bytes of one block of every leaf
    const int lstride = (int)(g.ncg * 1024);        // leaf t to t + 1 (the host keeps it < 2^31)
    const char* base = static_cast<const char*>(g.w) + (t0 * g.ncg + cg) * 1024;
    if (t0 + 1 < g.nleaves) {
      float acc[2][MR];
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[0][r] = acc[1][r] = 0.f;
      gv_leaves_packed<MR, 2, AHEAD>(acc, base, slab, lstride, lane, x + t0 * GV_CH, g.k, m, sc);
#pragma unroll
      for (int r = 0; r < MR; ++r) y[r] = acc[0][r] + acc[1][r];  // the level-1 pair
    } else {
      float acc[1][MR];
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[0][r] = 0.f;
      gv_leaves_packed<MR, 1, AHEAD>(acc, base, slab, lstride, lane, x + t0 * GV_CH, g.k, m, sc);
#pragma unroll
      for (int r = 0; r < MR; ++r) y[r] = acc[0][r];  // the odd last leaf, carried
    }
  }

#pragma unroll
  for (int r = 0; r < MR; ++r) part[wave][r][lane] = y[r];
  gv_finish<MR, PK_COLS, LEAVES, 64 * WAVES, true>(g, part, last_flag, tid, grp, cg, m);
}

hipError_t launch_int8w_pack(void* dst, const void* codes, int64_t k, int64_t n, hipStream_t stream) {
  const int64_t P = k / GV_CH, ncg = (n + PK_COLS - 1) / PK_COLS;
  const int64_t chunks = PK_BLOCKS * P * ncg * 64;
  const int64_t blocks = (chunks + PK_CHUNK_THREADS - 1) / PK_CHUNK_THREADS;
  if (blocks > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(int8w_pack_kernel, dim3((unsigned)blocks), dim3(PK_CHUNK_THREADS), 0, stream,
                     static_cast<u4*>(dst), static_cast<const uint8_t*>(codes), n, P, ncg, chunks);
  return hipGetLastError();
}

template <int MR>
static hipError_t launch_pk_mr(const GemvArgs& g, const float* x, int waves, dim3 grid, hipStream_t s) {
  switch (waves) {
    case PK_WAVES_WHOLE:  // m <= 2 and the launch fills the CUs: loads a few blocks ahead
      if constexpr (MR <= 2) {
        hipLaunchKernelGGL((gemv_packed_kernel<MR, PK_WAVES_WHOLE, PK_AHEAD>), grid, dim3(64 * PK_WAVES_WHOLE), 0,
                           s, g, x);
        break;
      }
      return hipErrorInvalidValue;
    case PK_WAVES_SPLIT:  // few waves: every block of both leaves requested at once
      hipLaunchKernelGGL((gemv_packed_kernel<MR, PK_WAVES_SPLIT, PK_BLOCKS>), grid, dim3(64 * PK_WAVES_SPLIT), 0, s,
                         g, x);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemv_packed(const GemvArgs& g, const float* x, int waves, dim3 grid, hipStream_t stream) {
  if (g.m <= 1) return launch_pk_mr<1>(g, x, waves, grid, stream);
  if (g.m <= 2) return launch_pk_mr<2>(g, x, waves, grid, stream);
  if (g.m <= 4) return launch_pk_mr<4>(g, x, waves, grid, stream);
  if (g.m <= 8) return launch_pk_mr<8>(g, x, waves, grid, stream);
  return launch_pk_mr<16>(g, x, waves, grid, stream);
}

}  // namespace mlg

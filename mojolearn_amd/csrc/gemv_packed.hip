// gfx950 decode GEMV on int8 weights in the decode-packed layout, and the kernel that packs them.
//
// The row-major decode kernel (gemv_nn_kernel) streams every leaf of a column at once: at any
// moment its 3584 waves (M = 1, N = 14336, K = 4096) read within all 32 leaves' row bands, the
// whole 58.7 MB, and a read-only pass in that order takes 12.1 us.  The packed layout puts the
// same wave's data where its neighbours in time read: code (p, j) -- leaf t = p / 128, octet
// o = (p % 128) / 8 (eight rows), row i = p % 8, column group cg = j / 128, lane l = (j % 128) / 2,
// code e = j % 2 -- lives at byte
//
//     ((o * P + t) * ncg + cg) * 1024 + l * 16 + i * 2 + e        (P leaves, ncg column groups),
//
// so octet o of every wave is one contiguous slab of P * ncg KB and the waves, which advance
// together, read one slab at a time (read-only 10.8 us for the same bytes), with one 16-byte
// load per lane per octet (eight rows of its two columns) instead of eight 16-bit ones.
// Columns past n are packed as zero codes and never stored.  The arithmetic and its order are
// gemv_nn_kernel's: each lane runs its two columns' leaf chains in VALU in step order, each
// workgroup folds its aligned subtree of leaves through LDS, and the completing workgroup
// folds the group roots (gv_finish), so the bits are the row-major product's.
#include "gemv_body.h"

namespace mlg {

constexpr int PK_COLS = 128;                // columns a group: 64 lanes x 2 codes
constexpr int PK_OCT = 8;                   // rows an octet: one 16-byte load a lane
constexpr int PK_OCTS = GV_CH / PK_OCT;     // 16 octets a 128-row leaf
constexpr int PK_AHEAD = 4;                 // octets requested ahead of the one consumed
constexpr int PK_CHUNK_THREADS = 256;

// One thread per 16-byte chunk (octet o, leaf t, group cg, lane l), chunk index
// ((o * P + t) * ncg + cg) * 64 + l: it gathers rows 8o .. 8o+7 of leaf t at columns
// 128 cg + 2l, +1 (zero past n) and writes them in row order, two codes a row.
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
  const int64_t o = r / P;
  const int64_t p0 = t * GV_CH + o * PK_OCT;
  const int64_t j0 = cg * PK_COLS + 2 * l;
  uint32_t w[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t v = 0;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint8_t* row = codes + (p0 + 2 * q + h) * n;
#pragma unroll
      for (int e = 0; e < 2; ++e)
        if (j0 + e < n) v |= (uint32_t)row[j0 + e] << (8 * (2 * h + e));
    }
    w[q] = v;
  }
  dst[chunk] = u4{w[0], w[1], w[2], w[3]};
}

// One leaf of one column group from the packed layout: `base` is octet 0 of this wave's block,
// octet o at base + o * slab.  x is read XB steps at a time (uniform loads), one batch ahead.
template <int MR>
__device__ __forceinline__ void gv_leaf_packed(float (&acc)[MR][2], const char* base, int64_t slab, int lane,
                                               const float* __restrict__ xl, int64_t k, int m, const float (&sc)[2]) {
  constexpr int XB = MR <= 2 ? PK_OCT : 16 / MR;  // x steps a batch: at most 16 values a batch
  auto oct_rs = [&](int o) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base) + o * slab, (short)0, 1024, RSRC_WORD3);
  };
  const float* xr[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) xr[r] = xl + (r < m ? r : m - 1) * k;  // rows past m: never stored
  u4 ring[PK_OCTS];
#pragma unroll
  for (int o = 0; o < PK_AHEAD; ++o) ring[o] = __builtin_amdgcn_raw_buffer_load_b128(oct_rs(o), lane * 16, 0, 0);
  float xc[MR][XB], xn[MR][XB];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < XB; ++q) xc[r][q] = xr[r][q];
#pragma unroll
  for (int o = 0; o < PK_OCTS; ++o) {
    if (o + PK_AHEAD < PK_OCTS) {
      __builtin_amdgcn_sched_barrier(0);
      ring[o + PK_AHEAD] = __builtin_amdgcn_raw_buffer_load_b128(oct_rs(o + PK_AHEAD), lane * 16, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i0 = 0; i0 < PK_OCT; i0 += XB) {
      const int s0 = o * PK_OCT + i0;  // the leaf step of this batch's first value
      if (s0 + XB < GV_CH) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
          for (int q = 0; q < XB; ++q) xn[r][q] = xr[r][s0 + XB + q];
      }
#pragma unroll
      for (int q = 0; q < XB; ++q) {
        const int i = i0 + q;
        const uint32_t u = ring[o][i >> 1] >> (16 * (i & 1));
        // f32(code) * scale, one rounding (the scale flushed on input by MODE.FP_DENORM = 2)
        const float w0 = (float)((int32_t)(u << 24) >> 24) * sc[0];
        const float w1 = (float)((int32_t)(u << 16) >> 24) * sc[1];
#pragma unroll
        for (int r = 0; r < MR; ++r) {
          acc[r][0] = __builtin_fmaf(xc[r][q], w0, acc[r][0]);
          acc[r][1] = __builtin_fmaf(xc[r][q], w1, acc[r][1]);
        }
      }
      if (s0 + XB < GV_CH) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
          for (int q = 0; q < XB; ++q) xc[r][q] = xn[r][q];
      }
    }
  }
}

// A wave per (leaf, column group); LEAVES leaves a workgroup (an aligned subtree).  g.w is the
// packed buffer, g.nleaves = P, g.ncg the column groups of 128.
template <int MR, int LEAVES>
__global__ void __launch_bounds__(64 * LEAVES) gemv_packed_kernel(GemvArgs g, const float* __restrict__ x) {
  __shared__ float part[LEAVES][MR][PK_COLS];
  __shared__ unsigned int last_flag;

  set_flush_inputs_mode();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the grid holds at most INT32_MAX workgroups (the host refuses more): a 32-bit split
  const int64_t cg = blockIdx.x % (uint32_t)g.ncg;
  const int64_t grp = blockIdx.x / (uint32_t)g.ncg;
  const int64_t t = grp * LEAVES + wave;  // this wave's leaf
  const int m = (int)g.m;

  float acc[MR][2];
#pragma unroll
  for (int r = 0; r < MR; ++r) acc[r][0] = acc[r][1] = 0.f;

  if (t < g.nleaves) {
    // this lane's scales, clamped into [0, n) (columns past n are never stored)
    const int64_t c0 = cg * PK_COLS + lane * 2;
    float sc[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) sc[e] = g.scales[c0 + e < g.n ? c0 + e : g.n - 1];
    const int64_t slab = g.nleaves * g.ncg * 1024;  // bytes of one octet of every wave
    const char* base = static_cast<const char*>(g.w) + (t * g.ncg + cg) * 1024;
    gv_leaf_packed<MR>(acc, base, slab, lane, x + t * GV_CH, g.k, m, sc);
  }

#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int e = 0; e < 2; ++e) part[wave][r][lane * 2 + e] = acc[r][e];
  gv_finish<MR, PK_COLS, LEAVES, 64 * LEAVES>(g, part, last_flag, tid, grp, cg, m);
}

hipError_t launch_int8w_pack(void* dst, const void* codes, int64_t k, int64_t n, hipStream_t stream) {
  const int64_t P = k / GV_CH, ncg = (n + PK_COLS - 1) / PK_COLS;
  const int64_t chunks = PK_OCTS * P * ncg * 64;
  const int64_t blocks = (chunks + PK_CHUNK_THREADS - 1) / PK_CHUNK_THREADS;
  if (blocks > INT32_MAX) return hipErrorInvalidValue;
  hipLaunchKernelGGL(int8w_pack_kernel, dim3((unsigned)blocks), dim3(PK_CHUNK_THREADS), 0, stream,
                     static_cast<u4*>(dst), static_cast<const uint8_t*>(codes), n, P, ncg, chunks);
  return hipGetLastError();
}

template <int MR>
static hipError_t launch_pk_mr(const GemvArgs& g, const float* x, int leaves, dim3 grid, hipStream_t s) {
  if (leaves == GV_WIDE_LEAVES) {
    if constexpr (MR <= 2) {
      hipLaunchKernelGGL((gemv_packed_kernel<MR, GV_WIDE_LEAVES>), grid, dim3(64 * GV_WIDE_LEAVES), 0, s, g, x);
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  if (leaves != GV_LEAVES) return hipErrorInvalidValue;
  hipLaunchKernelGGL((gemv_packed_kernel<MR, GV_LEAVES>), grid, dim3(64 * GV_LEAVES), 0, s, g, x);
  return hipGetLastError();
}

hipError_t launch_gemv_packed(const GemvArgs& g, const float* x, int leaves, dim3 grid, hipStream_t stream) {
  if (g.m <= 1) return launch_pk_mr<1>(g, x, leaves, grid, stream);
  if (g.m <= 2) return launch_pk_mr<2>(g, x, leaves, grid, stream);
  if (g.m <= 4) return launch_pk_mr<4>(g, x, leaves, grid, stream);
  if (g.m <= 8) return launch_pk_mr<8>(g, x, leaves, grid, stream);
  return launch_pk_mr<16>(g, x, leaves, grid, stream);
}

}  // namespace mlg

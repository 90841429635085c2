// gfx950 decode GEMV on int8 weights in the decode-packed layout, and the kernel that packs them.
//
// The row-major decode kernel (gemv_nn_kernel) cannot give one workgroup every leaf of its
// columns: a 64-column strip of a row-major int8 matrix is 64-byte row segments, which read at
// half the speed of 256-byte ones, so its workgroups hold 4 or 8 leaves of 128 columns and the
// leaf groups of a column meet through a cross-workgroup fold (roots to memory, a counter, the
// last workgroup reloading them).  The packed layout makes a 64-column group contiguous:
// code (p, j) -- leaf t = p / 128, block s = (p % 128) / 16 (sixteen rows), row i = p % 16,
// column group cg = j / 64, lane l = j % 64 -- lives, biased (the byte code + 128), at byte
//
//     ((s * P + t) * ncg + cg) * 1024 + l * 16 + i        (P leaves, ncg column groups),
//
// so one 16-byte load gives a lane sixteen rows of its column, the waves of a group read whole
// 1 KB chunks, and block s of every leaf is one contiguous slab of P * ncg KB that the waves,
// which advance together, read at the same time.  A workgroup of 16 waves, each running two
// adjacent leaves, then holds 32 leaves of 64 columns: at K = 4096 the whole contract tree of
// its columns, folded in LDS with no workspace, no counter and no second pass.  Columns past n
// are packed as zero codes and never stored.  The bias lets the dequant convert an unsigned byte
// (v_cvt_f32_ubyte, faster than the sign-extending convert) and fold the bias into one fma
// (pk_dequant).  The arithmetic and its order are gemv_nn_kernel's:
// per leaf the chain acc = fma(x, f32(code) * scale, acc) in step order from +0, the level-1
// pair of a wave's two leaves added in registers, the rest of the tree over the workgroup's
// pairs (gv_finish with two-leaf nodes), and past 32 leaves the group roots folded by the
// workgroup that completes the count -- so the bits are the row-major product's.  A launch too
// small for whole columns runs 4-leaf groups of four one-leaf waves, folded across workgroups;
// for 3 <= m <= 16 with x on the 16-byte grid the chains run on the matrix cores
// (gemv_packed_mfma_kernel below).
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
constexpr uint32_t PK_BIAS = 0x80808080u;  // code + 128 in each byte of a packed word

// f32(code) * scale with one rounding (the contract's dequant; the scale is flushed on input by
// MODE.FP_DENORM = 2) from byte `byte` of a packed word.  FAST: f32(u) * scale - 128 * scale is
// code * scale exactly, so one fma rounds it once, whenever 128 * scale is exact (nsc = -128 *
// scale, |scale| < 2^120 and not NaN: the caller's wave-uniform check).  Otherwise the code is
// unbiased, sign-extended and multiplied.  A zero weight's sign cannot reach a chain that
// starts at +0 (+0 + -0 is +0), so the forms agree on every bit that reaches the output.
template <bool FAST>
__device__ __forceinline__ float pk_dequant(uint32_t u, int byte, float sc, float nsc) {
  if constexpr (FAST) return __builtin_fmaf((float)((u >> (8 * byte)) & 0xFFu), sc, nsc);
  else return (float)((int32_t)((u ^ PK_BIAS) << (24 - 8 * byte)) >> 24) * sc;
}

// Whether every lane of the wave may take pk_dequant's fma form.
__device__ __forceinline__ bool pk_fast_scales(float sc) {
  return __builtin_amdgcn_ballot_w64(!(__builtin_fabsf(sc) < 0x1p120f)) == 0;
}

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
  dst[chunk] = u4{w[0] ^ PK_BIAS, w[1] ^ PK_BIAS, w[2] ^ PK_BIAS, w[3] ^ PK_BIAS};
}

// NL adjacent leaves of one lane's column from the packed layout: block s of leaf q at
// base + s * slab + q * lstride (+ lane * 16), AHEAD blocks requested ahead of the one
// consumed.  x is read XB steps at a time (uniform loads) one batch ahead.  acc[q][r] is leaf
// q's chain for row r.
template <int MR, int NL, int AHEAD, bool FAST>
__device__ __forceinline__ void gv_leaves_packed(float (&acc)[NL][MR], const char* base, int64_t slab,
                                                 int lstride, int lane, const float* __restrict__ xl, int64_t k,
                                                 int m, float sc) {
  const float nsc = -128.f * sc;  // exact for pk_dequant<true>
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
    // a block issues no loads once every block is in flight: the fence keeps its converts from
    // being hoisted into earlier blocks (all of them live at once: 55 -> 137 VGPRs at M = 1)
    if (s + AHEAD >= PK_BLOCKS) __builtin_amdgcn_sched_barrier(0);
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
          const float w = pk_dequant<FAST>(u, b & 3, sc, nsc);
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

// WAVES waves a workgroup, each running LPW adjacent leaves (two, or one when the launch is small
// and shorter chains on more waves pay) of the workgroup's 64 columns (LPW * WAVES leaves: an
// aligned subtree).  g.w is the packed buffer, g.nleaves = P, g.ncg the column groups of 64.
template <int MR, int WAVES, int AHEAD, int LPW = 2>
__global__ void __launch_bounds__(64 * WAVES) gemv_packed_kernel(GemvArgs g, const float* __restrict__ x) {
  static_assert(LPW == 1 || LPW == 2, "one or two leaves a wave");
  constexpr int LEAVES = LPW * WAVES;
  __shared__ float part[WAVES][MR][PK_COLS];
  __shared__ unsigned int last_flag;

  set_flush_inputs_mode();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the grid holds at most INT32_MAX workgroups (the host refuses more): a 32-bit split
  const int64_t cg = blockIdx.x % (uint32_t)g.ncg;
  const int64_t grp = blockIdx.x / (uint32_t)g.ncg;
  const int64_t t0 = grp * LEAVES + LPW * wave;  // this wave's first leaf
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
    if (LPW == 2 && t0 + 1 < g.nleaves) {
      float acc[2][MR];
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[0][r] = acc[1][r] = 0.f;
      if (pk_fast_scales(sc))
        gv_leaves_packed<MR, 2, AHEAD, true>(acc, base, slab, lstride, lane, x + t0 * GV_CH, g.k, m, sc);
      else
        gv_leaves_packed<MR, 2, AHEAD, false>(acc, base, slab, lstride, lane, x + t0 * GV_CH, g.k, m, sc);
#pragma unroll
      for (int r = 0; r < MR; ++r) y[r] = acc[0][r] + acc[1][r];  // the level-1 pair
    } else {
      float acc[1][MR];
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[0][r] = 0.f;
      if (pk_fast_scales(sc))
        gv_leaves_packed<MR, 1, AHEAD, true>(acc, base, slab, lstride, lane, x + t0 * GV_CH, g.k, m, sc);
      else
        gv_leaves_packed<MR, 1, AHEAD, false>(acc, base, slab, lstride, lane, x + t0 * GV_CH, g.k, m, sc);
#pragma unroll
      for (int r = 0; r < MR; ++r) y[r] = acc[0][r];  // one leaf, or the odd last leaf carried
    }
  }

#pragma unroll
  for (int r = 0; r < MR; ++r) part[wave][r][lane] = y[r];
  gv_finish<MR, PK_COLS, LEAVES, 64 * WAVES, LPW>(g, part, last_flag, tid, grp, cg, m);
}

// ---- 3 <= m <= 16 on the matrix cores, from the decode-packed layout.
//
// Lane l of a wave owns column 64 cg + l (the layout's lane) and feeds B = W[p][64 cg + l] to a
// K = 1 instruction (one fma_rn per output element: under MODE.FP_DENORM = 2 the contract's
// fma(ftz a, ftz b, ftz c), like v_fma_f32); A is x[row][p] for the row the shape gives the lane:
//  * SHAPE 16 (v_mfma_f32_16x16x1_4b_f32, 9 <= m <= 16): block b = l / 16 is the outer product
//    of lanes 16b .. 16b+15's values, so lane l feeds row l % 16 and gets back, in register
//    4 blk + i, row 4 (l / 16) + i of column 16 blk + l % 16;
//  * SHAPE 4 (v_mfma_f32_4x4x1_16b_f32, 3 <= m <= 8, G groups of four rows): lane l feeds row
//    4 g + l % 4 and gets back, in register r, row 4 g + r of its own column.
// A wave runs two adjacent leaves, one instruction per leaf per step.  Only one lane group
// needs each x value: the instruction's A broadcast (CBSZ, ABID) feeds every block from block
// ABID's lanes.  So the lanes hold different steps of x: with SHAPE 16, lane 16u + r holds
// x[r][steps 4u .. 4u+3 of the block] of one leaf (one 16-byte read a leaf a block, block u
// broadcast for steps 4u .. 4u+3); with SHAPE 4, lane 32g + 16q + 4u + r holds x[4g + r][steps
// 4u .. 4u+3] of leaf q (one read a block for both leaves and both groups, block 8g + 4q + u
// broadcast).  So each lane loads its own x chunks straight into registers, with the block's
// weights.  The workgroup and its fold are gemv_packed_kernel's.
template <int SHAPE, int G>
struct PkMf {
  static constexpr int MR = SHAPE == 16 ? 16 : 4 * G;  // rows the lane's instructions cover
  static constexpr int NA = SHAPE == 16 ? 1 : G;        // accumulators a leaf
  static constexpr int NI = SHAPE == 16 ? 2 : 1;        // x loads a block, 16 bytes a lane each
};
typedef float pk_v16f __attribute__((ext_vector_type(16)));
typedef float pk_v4f __attribute__((ext_vector_type(4)));
template <int SHAPE>
using PkV = typename std::conditional<SHAPE == 16, pk_v16f, pk_v4f>::type;

// The x chunk lane l of load h holds: leaf q, row r, steps 4u .. 4u+3 of the block (the
// broadcast layout above; with one group of four rows, lanes 32 .. 63 load nothing: no
// instruction takes their x).
template <int SHAPE, int G>
__device__ __forceinline__ void pk_xchunk(int h, int lane, int& q, int& r, int& u) {
  if constexpr (SHAPE == 16) {
    q = h;
    r = lane & 15;
    u = lane >> 4;
  } else {
    const int l = G == 1 ? (lane & 31) : lane;
    q = (l >> 4) & 1;
    u = (l >> 2) & 3;
    r = 4 * (l >> 5) + (l & 3);
  }
}

// f(integral_constant<int, I>) for I = B .. E-1: the block loop with its index a constant, so
// every wait count and register slot below is named at compile time.
template <int B, int E, typename F>
__device__ __forceinline__ void pk_static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    pk_static_for<B + 1, E>(f);
  }
}

// s_waitcnt vmcnt(N), other counters untouched
template <int N>
__device__ __forceinline__ void pk_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 0 .. 63");
  __builtin_amdgcn_s_waitcnt(((N & 15) | ((N >> 4) << 14)) | 0x0F70);
}

// NL adjacent leaves of one lane's column (block s of leaf q at base + s * slab + q * lstride,
// + lane * 16), AHEAD blocks in flight.  Issue order: blocks 0 .. AHEAD-1 (weights, then x) up
// front; in iteration s block s + AHEAD's weights and x before block s is consumed.  Both land
// in register rings of AHEAD + 1 blocks; a lane's x chunk is the one its own instructions take.
template <int SHAPE, int G, int NL, int AHEAD, bool FAST, typename V, int NA>
__device__ __forceinline__ void pk_leaves_mfma(V (&acc)[NL][NA], const char* base, int64_t slab, int lstride,
                                               int lane, __amdgpu_buffer_rsrc_t xrs,
                                               const uint32_t (&xvoff)[PkMf<SHAPE, G>::NI], float sc) {
  const float nsc = -128.f * sc;  // exact for pk_dequant<true>
  using S = PkMf<SHAPE, G>;
  static_assert(NA == S::NA, "accumulators a leaf");
  static_assert(AHEAD >= 1 && AHEAD <= PK_BLOCKS, "blocks in flight");
  constexpr int RING = AHEAD + 1 < PK_BLOCKS ? AHEAD + 1 : PK_BLOCKS;  // register blocks
  constexpr int LPG = S::NI + NL;                                    // loads a block
  auto block_rs = [&](int s) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base) + s * slab, (short)0, 0x7FFFFFFF, RSRC_WORD3);
  };
  u4 ring[RING][NL];
  u4 xr[RING][S::NI];
  // (with one group of four rows only lanes 0 .. 31 load x: the other half would repeat them)
  auto issue = [&](int s) {
#pragma unroll
    for (int q = 0; q < NL; ++q)
      ring[s % RING][q] = __builtin_amdgcn_raw_buffer_load_b128(block_rs(s), lane * 16, q * lstride, PK_AUX);
#pragma unroll
    for (int h = 0; h < S::NI; ++h)
      if (SHAPE == 16 || G == 2 || lane < 32)
        xr[s % RING][h] = __builtin_amdgcn_raw_buffer_load_b128(xrs, (int)xvoff[h], 64 * s, 0);
  };
  pk_static_for<0, AHEAD>([&](auto SC) { issue(decltype(SC)::value); });

  pk_static_for<0, PK_BLOCKS>([&](auto SC) {
    constexpr int s = decltype(SC)::value;
    if constexpr (s + AHEAD < PK_BLOCKS) {
      __builtin_amdgcn_sched_barrier(0);
      issue(s + AHEAD);
      __builtin_amdgcn_sched_barrier(0);
    }
    // block s landed; the blocks issued after it stay in flight
    constexpr int later = PK_BLOCKS - 1 - s < AHEAD ? PK_BLOCKS - 1 - s : AHEAD;
    pk_wait_vm<later * LPG>();
    __builtin_amdgcn_sched_barrier(0);
    f4 xq[S::NI];
#pragma unroll
    for (int h = 0; h < S::NI; ++h) xq[h] = __builtin_bit_cast(f4, xr[s % RING][h]);
    // the block's weights first, then its instructions back to back: with each weight formed just
    // before its instruction, every instruction waited on its own convert and fma (and the SIMD's
    // waves, running the same sequence, on theirs): M = 4 14.7 -> 13.2 us, M = 16 25.3 -> 23.7
    float wb[PK_RB][NL];
    pk_static_for<0, PK_RB>([&](auto BC) {
      constexpr int b = decltype(BC)::value;
      pk_static_for<0, NL>([&](auto QC) {
        constexpr int q = decltype(QC)::value;
        wb[b][q] = pk_dequant<FAST>(ring[s % RING][q][b >> 2], b & 3, sc, nsc);
      });
    });
    __builtin_amdgcn_sched_barrier(0);
    pk_static_for<0, PK_RB>([&](auto BC) {
      constexpr int b = decltype(BC)::value;  // byte of the chunk: row 16 s + b of the leaf
      pk_static_for<0, NL>([&](auto QC) {
        constexpr int q = decltype(QC)::value;
        const float w = wb[b][q];
        pk_static_for<0, NA>([&](auto GC) {
          constexpr int gg = decltype(GC)::value;
          const V c = (s == 0 && b == 0) ? V{} : acc[q][gg];
          if constexpr (SHAPE == 16)  // block b / 4 holds x of steps 4 (b / 4) .. +3 of leaf q
            acc[q][gg] = __builtin_amdgcn_mfma_f32_16x16x1f32(xq[q][b & 3], w, c, 2, b >> 2, 0);
          else  // block 8 gg + 4 q + b / 4 holds rows 4 gg .. 4 gg + 3 of those steps
            acc[q][gg] = __builtin_amdgcn_mfma_f32_4x4x1f32(xq[0][b & 3], w, c, 4, 8 * gg + 4 * q + (b >> 2), 0);
        });
      });
    });
  });
}

template <int SHAPE, int G, int WAVES, int AHEAD>
__global__ void __launch_bounds__(64 * WAVES) gemv_packed_mfma_kernel(GemvArgs g, const float* __restrict__ x) {
  using S = PkMf<SHAPE, G>;
  using V = PkV<SHAPE>;
  constexpr int MR = S::MR;
  constexpr int LEAVES = 2 * WAVES;
  __shared__ __attribute__((aligned(16))) float part[WAVES][MR][PK_COLS];
  __shared__ unsigned int last_flag;

  set_flush_inputs_mode();
  gv_fetch_args(g, x);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the grid holds at most INT32_MAX workgroups (the host refuses more): a 32-bit split
  const int64_t cg = blockIdx.x % (uint32_t)g.ncg;
  const int64_t grp = blockIdx.x / (uint32_t)g.ncg;
  const int64_t t0 = grp * LEAVES + 2 * wave;  // this wave's first leaf
  const int m = (int)g.m;

  V y[S::NA];
#pragma unroll
  for (int gg = 0; gg < S::NA; ++gg) y[gg] = V{};

  if (t0 < g.nleaves) {
    const int64_t j = cg * PK_COLS + lane;
    const float sc = g.scales[j < g.n ? j : g.n - 1];  // columns past n are never stored
    const int64_t slab = g.nleaves * g.ncg * 1024;
    const int lstride = (int)(g.ncg * 1024);
    const char* base = static_cast<const char*>(g.w) + (t0 * g.ncg + cg) * 1024;
    // x: one resource over the whole operand (rows past m read row m - 1; the host keeps
    // m * k * 4 < 2^31), this lane's chunk of each of a block's loads at a fixed offset, the
    // block's first step in the scalar offset
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), (short)0, (int)(g.m * g.k * 4), RSRC_WORD3);
    uint32_t xvoff[S::NI];
#pragma unroll
    for (int h = 0; h < S::NI; ++h) {
      int q, r, u;
      pk_xchunk<SHAPE, G>(h, lane, q, r, u);
      const int64_t row = r < m ? r : m - 1;
      xvoff[h] = (uint32_t)((row * g.k + (t0 + q) * GV_CH + 4 * u) * 4);
    }
    if (t0 + 1 < g.nleaves) {
      V acc[2][S::NA];
      if (pk_fast_scales(sc))
        pk_leaves_mfma<SHAPE, G, 2, AHEAD, true>(acc, base, slab, lstride, lane, xrs, xvoff, sc);
      else
        pk_leaves_mfma<SHAPE, G, 2, AHEAD, false>(acc, base, slab, lstride, lane, xrs, xvoff, sc);
#pragma unroll
      for (int gg = 0; gg < S::NA; ++gg) y[gg] = acc[0][gg] + acc[1][gg];  // the level-1 pair
    } else {
      V acc[1][S::NA];
      if (pk_fast_scales(sc))
        pk_leaves_mfma<SHAPE, G, 1, AHEAD, true>(acc, base, slab, lstride, lane, xrs, xvoff, sc);
      else
        pk_leaves_mfma<SHAPE, G, 1, AHEAD, false>(acc, base, slab, lstride, lane, xrs, xvoff, sc);
#pragma unroll
      for (int gg = 0; gg < S::NA; ++gg) y[gg] = acc[0][gg];  // the odd last leaf, carried
    }
  }

  if constexpr (SHAPE == 16) {
#pragma unroll
    for (int blk = 0; blk < 4; ++blk)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[wave][4 * (lane >> 4) + i][16 * blk + (lane & 15)] = y[0][4 * blk + i];
  } else {
#pragma unroll
    for (int gg = 0; gg < G; ++gg)
#pragma unroll
      for (int r = 0; r < 4; ++r) part[wave][4 * gg + r][lane] = y[gg][r];
  }
  gv_finish<MR, PK_COLS, LEAVES, 64 * WAVES, 2>(g, part, last_flag, tid, grp, cg, m);
}

template <int SHAPE, int G>
static hipError_t launch_pkmf(const GemvArgs& g, const float* x, int waves, dim3 grid, hipStream_t s) {
  switch (waves) {
    case PK_WAVES_WHOLE:
      hipLaunchKernelGGL((gemv_packed_mfma_kernel<SHAPE, G, PK_WAVES_WHOLE, PK_AHEAD>), grid,
                         dim3(64 * PK_WAVES_WHOLE), 0, s, g, x);
      break;
    case PK_WAVES_SPLIT:
      hipLaunchKernelGGL((gemv_packed_mfma_kernel<SHAPE, G, PK_WAVES_SPLIT, PK_BLOCKS>), grid,
                         dim3(64 * PK_WAVES_SPLIT), 0, s, g, x);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_gemv_packed_mfma(const GemvArgs& g, const float* x, int waves, dim3 grid, hipStream_t stream) {
  if (g.m <= 4) return launch_pkmf<4, 1>(g, x, waves, grid, stream);
  if (g.m <= 8) return launch_pkmf<4, 2>(g, x, waves, grid, stream);
  return launch_pkmf<16, 1>(g, x, waves, grid, stream);
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
    case PK_WAVES_SPLIT:  // a small launch: 4-leaf groups as four one-leaf waves, every block in flight
      hipLaunchKernelGGL((gemv_packed_kernel<MR, 2 * PK_WAVES_SPLIT, PK_BLOCKS, 1>), grid, dim3(128 * PK_WAVES_SPLIT),
                         0, s, g, x);
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

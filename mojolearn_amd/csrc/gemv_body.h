// Device body of the skinny-M kernels, shared by gemv_nn.hip and gemv_nt.hip.
#pragma once
#include "device_common.h"
#include "gemv.h"

namespace mlg {

// The arguments the first W loads depend on, named by an empty asm at a matrix-core skinny
// kernel's start: both lines of the argument block are then fetched in one round trip, not in
// dependent pieces around the workgroup index split and the leaf check (measured: M = 16
// decode 1.7% faster).  The asm is volatile, so the compiler can no longer prove memory
// unchanged since the kernel's start: a kernel that reads x with scalar loads (gemv_nn) would
// read it with vector loads after it, and does without it.
__device__ __forceinline__ void gv_fetch_args(const GemvArgs& g, const float* x) {
  __asm__ volatile("" ::"s"(g.w), "s"(g.scales), "s"(g.m), "s"(g.n), "s"(g.k), "s"(g.leaf), "s"(g.nleaves),
                   "s"(g.ncg), "s"(x));
}

// The contract's tree over a cell's P roots base[t * stride], read with agent-scope atomic
// loads issued up to GV_FOLD_BATCH at a time.
__device__ __forceinline__ float fold_roots(const float* base, int64_t P, int64_t stride) {
  StackF stk;
  int64_t t = 0;
  float last = 0.f;
  for (int64_t t0 = 0; t0 < P; t0 += GV_FOLD_BATCH) {
    float v[GV_FOLD_BATCH];
#pragma unroll
    for (int e = 0; e < GV_FOLD_BATCH; ++e)
      if (t0 + e < P) v[e] = __hip_atomic_load(base + (t0 + e) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int e = 0; e < GV_FOLD_BATCH; ++e) {
      if (t0 + e >= P) break;
      t = t0 + e;
      if (t + 1 < P) stk.push(v[e], (int)t);
      else last = v[e];
    }
  }
  return stk.root(last, (int)t);
}

// Load the words of rows k0 .. k0+GV_CH-1 (rows past `klast` read row `klast`: in bounds,
// and no chain step uses them).  VEC: buffer loads, the chunk's first row in a scalar
// resource, the row offset i*rowbytes in the scalar offset and the lane's byte offset
// `loff` in one VGPR (the host keeps GV_CH * rowbytes below 2^31).  Otherwise one load per
// element at the per-column offsets `coff`.
template <int BT, bool VEC>
__device__ __forceinline__ void gv_load(uint32_t (&buf)[GV_CH], const char* w, uint32_t loff, const uint32_t* coff,
                                        int64_t rowbytes, int64_t k0, int64_t klast) {
  const int64_t last = klast - k0;  // >= GV_CH - 1 for a full chunk
  if constexpr (VEC) {
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<char*>(w + k0 * rowbytes), (short)0, 0x7FFFFFFF, RSRC_WORD3);
#pragma unroll
    for (int i = 0; i < GV_CH; ++i) {
      const int ii = i <= last ? i : (int)last;
      buf[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)loff, ii * (int)rowbytes, 0);
    }
  } else {
    constexpr int CPL = GvCols<BT>::cpl;
#pragma unroll
    for (int i = 0; i < GV_CH; ++i) {
      const int64_t ii = i <= last ? i : last;
      const char* row = w + (k0 + ii) * rowbytes;
      uint32_t u = 0;
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        if constexpr (BT == T_F32) u = *reinterpret_cast<const uint32_t*>(row + coff[e]);
        else if constexpr (BT == T_BF16) u |= (uint32_t)*reinterpret_cast<const uint16_t*>(row + coff[e]) << (16 * e);
        else u |= (uint32_t)*reinterpret_cast<const uint8_t*>(row + coff[e]) << (8 * e);
      }
      buf[i] = u;
    }
  }
}

// x values for steps k0+i0 .. k0+i0+XB-1 of every row (uniform loads; a row past m reads
// row m-1 and a step past k reads step k-1 -- in bounds, and no chain step uses them).
template <int MR, int XB, bool FULL>
__device__ __forceinline__ void gv_load_x(float (&xv)[MR][XB], const float* __restrict__ x, int64_t k, int64_t k0,
                                          int i0, int m) {
#pragma unroll
  for (int r = 0; r < MR; ++r) {
    const float* xr = x + (r < m ? r : m - 1) * k;
#pragma unroll
    for (int q = 0; q < XB; ++q) {
      if constexpr (FULL) {
        xv[r][q] = xr[k0 + i0 + q];  // a full chunk lies inside the leaf
      } else {
        const int64_t kk = k0 + i0 + q < k ? k0 + i0 + q : k - 1;
        xv[r][q] = xr[kk];
      }
    }
  }
}

// Chain steps for rows k0 .. k0+nrows-1 (all GV_CH when FULL).  W[p, j] as float32: bf16
// widened exactly; int8 f32(code) * scale[j], one rounding (the scale flushed on input).
// x is read XB steps at a time, one batch ahead.
template <int BT, int MR, bool FULL>
__device__ __forceinline__ void gv_steps(float (&acc)[MR][GvCols<BT>::cpl], const uint32_t (&buf)[GV_CH],
                                         const float* __restrict__ x, int64_t k, int64_t k0, int nrows,
                                         int m, const float (&sc)[GvCols<BT>::cpl]) {
  constexpr int CPL = GvCols<BT>::cpl;
  constexpr int XB = MR >= 16 ? 1 : 16 / MR;
  float xc[MR][XB], xn[MR][XB];
  gv_load_x<MR, XB, FULL>(xc, x, k, k0, 0, m);
#pragma unroll
  for (int b = 0; b < GV_CH / XB; ++b) {
    if (b + 1 < GV_CH / XB) gv_load_x<MR, XB, FULL>(xn, x, k, k0, (b + 1) * XB, m);
#pragma unroll
    for (int q = 0; q < XB; ++q) {
      const int i = b * XB + q;
      if (!FULL && i >= nrows) continue;  // uniform
      const uint32_t u = buf[i];
      float wv[CPL];
      if constexpr (BT == T_F32) {
        wv[0] = __uint_as_float(u);
      } else if constexpr (BT == T_BF16) {
        wv[0] = __uint_as_float(u << 16);
        wv[1] = __uint_as_float(u & 0xFFFF0000u);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) wv[e] = (float)((int32_t)(u << (24 - 8 * e)) >> 24) * sc[e];
      }
      // rows past m (MR rounds m up) run on row m-1's x and are never stored
#pragma unroll
      for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int e = 0; e < CPL; ++e) acc[r][e] = __builtin_fmaf(xc[r][q], wv[e], acc[r][e]);
    }
    if (b + 1 < GV_CH / XB) {
#pragma unroll
      for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int q = 0; q < XB; ++q) xc[r][q] = xn[r][q];
    }
  }
}

// One whole 128-row leaf (the decode shapes: L = 128, k a multiple of 128), straight-line:
// the rows travel in blocks of GV_RB through a ring of GV_AHEAD + 1 register blocks, GV_AHEAD
// blocks requested ahead of the one being consumed, so the wave keeps loads in flight while
// it computes on the rows that have landed.  x is read XB steps at a time, one batch ahead.
// `wleaf` is the leaf's first row; rows are `rowbytes` apart (GV_CH * rowbytes < 2^31).  A
// lane's word is 32 bits, or 16 (two int8 codes) where GvCols<BT, false, true> says so.
constexpr int GV_RB = 16;
constexpr int GV_AHEAD = 3;

template <int BT, int CPL>
__device__ __forceinline__ void gv_weights(uint32_t u, const float (&sc)[CPL], float (&wv)[CPL]) {
  if constexpr (BT == T_F32) {
    wv[0] = __uint_as_float(u);
  } else if constexpr (BT == T_BF16) {
    wv[0] = __uint_as_float(u << 16);
    wv[1] = __uint_as_float(u & 0xFFFF0000u);
  } else {
#pragma unroll
    for (int e = 0; e < CPL; ++e) wv[e] = (float)((int32_t)(u << (24 - 8 * e)) >> 24) * sc[e];
  }
}

template <int BT, int MR, int CPL>
__device__ __forceinline__ void gv_leaf_full(float (&acc)[MR][CPL], const char* wleaf, uint32_t loff, int rowbytes,
                                             const float* __restrict__ xl, int64_t k, int m,
                                             const float (&sc)[CPL]) {
  static_assert(CPL == GvCols<BT, false, true>::cpl, "a whole-leaf lane's columns");
  constexpr bool HALF = CPL * Elem<BT>::bytes == 2;  // 16-bit words
  constexpr int NBLK = GV_CH / GV_RB;
  constexpr int RING = GV_AHEAD + 1;
  constexpr int XB = MR <= 16 ? 16 / MR : 1;  // 16 x values a batch: two batches fit the scalar file
  // Each block of GV_RB rows gets a resource based at its first row, so the scalar offsets
  // are the GV_RB values i * rowbytes shared by every block (not GV_CH values held at once).
  auto block_rs = [&](int b) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(wleaf) + (int64_t)b * GV_RB * rowbytes, (short)0,
                                             0x7FFFFFFF, RSRC_WORD3);
  };
  // non-temporal (cache policy nt): a wave's loads of a row take whole lines, nothing is read
  // twice (M=1 int8 decode 15.05 -> 14.5 us, fp32 GEMV 1x14336x4096 45.3 -> 43.2 us; the
  // matrix-core kernels keep the default policy: M=16 31.7 -> 32.9 us with it)
  auto load_word = [&](__amdgpu_buffer_rsrc_t rs, int soff) -> uint32_t {
    if constexpr (HALF) return __builtin_amdgcn_raw_buffer_load_b16(rs, (int)loff, soff, GV_NT);
    else return __builtin_amdgcn_raw_buffer_load_b32(rs, (int)loff, soff, GV_NT);
  };
  const float* xr[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) xr[r] = xl + (r < m ? r : m - 1) * k;  // rows past m: never stored

  uint32_t ring[RING][GV_RB];
#pragma unroll
  for (int b = 0; b < GV_AHEAD; ++b) {
    const __amdgpu_buffer_rsrc_t rs = block_rs(b);
    int rb = rowbytes;
    // With more than one row of x the offsets are recomputed per block, never held across
    // blocks (held, they overflow the scalar file next to x).
    if constexpr (MR > 1) __asm__ volatile("" : "+s"(rb));
#pragma unroll
    for (int i = 0; i < GV_RB; ++i) ring[b][i] = load_word(rs, i * rb);
  }
  float xc[MR][XB], xn[MR][XB];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < XB; ++q) xc[r][q] = xr[r][q];

#pragma unroll
  for (int b = 0; b < NBLK; ++b) {
    if (b + GV_AHEAD < NBLK) {
      __builtin_amdgcn_sched_barrier(0);
      const __amdgpu_buffer_rsrc_t rs = block_rs(b + GV_AHEAD);
      int rb = rowbytes;
      if constexpr (MR > 1) __asm__ volatile("" : "+s"(rb));
#pragma unroll
      for (int i = 0; i < GV_RB; ++i) ring[(b + GV_AHEAD) % RING][i] = load_word(rs, i * rb);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q0 = 0; q0 < GV_RB; q0 += XB) {
      const int s0 = b * GV_RB + q0;
      if (s0 + XB < GV_CH) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
          for (int q = 0; q < XB; ++q) xn[r][q] = xr[r][s0 + XB + q];
      }
#pragma unroll
      for (int q = 0; q < XB; ++q) {
        float wv[CPL];
        gv_weights<BT, CPL>(ring[b % RING][q0 + q], sc, wv);
#pragma unroll
        for (int r = 0; r < MR; ++r)
#pragma unroll
          for (int e = 0; e < CPL; ++e) acc[r][e] = __builtin_fmaf(xc[r][q], wv[e], acc[r][e]);
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

// OP_NT (the LM layout W[n][k]): lane l owns output column j0 + l and walks its own W row,
// contiguous in k, 16 bytes per load (VEC: 4 / 8 / 16 steps per load for f32 / bf16 / int8) or one
// element per load.  A piece of up to S steps of the leaf (64 with 16-byte loads, 128 otherwise)
// is requested with one buffer resource starting at row j0, step p0 (bounded by the operand's end:
// rows past n read zeros) and immediate offsets, then consumed in order.  x is read XB steps at a
// time, one batch ahead.
template <int BT, int MR, bool VEC, bool FULL, int S = GV_CH>
__device__ __forceinline__ void gv_steps_nt(float (&acc)[MR][1], const uint32_t (&buf)[VEC ? S * Elem<BT>::bytes / 4 : S],
                                            const float* __restrict__ x, int64_t k, int64_t p0, int nrow, int m,
                                            float sc) {
  constexpr int EB = Elem<BT>::bytes;
  constexpr int XB = MR <= 2 ? 16 : 32 / MR;
  float xc[MR][XB], xn[MR][XB];
  gv_load_x<MR, XB, FULL>(xc, x, k, p0, 0, m);
#pragma unroll
  for (int b = 0; b < S / XB; ++b) {
    if (b + 1 < S / XB) gv_load_x<MR, XB, FULL>(xn, x, k, p0, (b + 1) * XB, m);
#pragma unroll
    for (int q = 0; q < XB; ++q) {
      const int i = b * XB + q;
      if (!FULL && i >= nrow) continue;  // uniform
      float wv;
      if constexpr (VEC) {
        const uint32_t u = buf[i * EB / 4];
        if constexpr (BT == T_F32) wv = __uint_as_float(u);
        else if constexpr (BT == T_BF16) wv = __uint_as_float((i & 1) ? (u & 0xFFFF0000u) : (u << 16));
        else wv = (float)((int32_t)(u << (24 - 8 * (i & 3))) >> 24) * sc;
      } else {
        const uint32_t u = buf[i];
        if constexpr (BT == T_F32) wv = __uint_as_float(u);
        else if constexpr (BT == T_BF16) wv = __uint_as_float(u << 16);
        else wv = (float)(int32_t)(int8_t)(uint8_t)u * sc;
      }
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[r][0] = __builtin_fmaf(xc[r][q], wv, acc[r][0]);
    }
    if (b + 1 < S / XB) {
#pragma unroll
      for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int q = 0; q < XB; ++q) xc[r][q] = xn[r][q];
    }
  }
}

template <int BT, int MR, bool VEC>
__device__ __forceinline__ void gv_leaf_nt(float (&acc)[MR][1], const char* w, int64_t n, int64_t k, int64_t j0,
                                           int64_t kb, int64_t ke, const float* __restrict__ x, int m, float sc,
                                           int lane) {
  constexpr int EB = Elem<BT>::bytes;
  // 64-step pieces with 16-byte loads: half the registers of a whole leaf (fp32: 2 -> 5 waves a
  // SIMD; the 1 x 14336 x 4096 product 50.8 -> 48.8 us, 8-row products up to 28 % faster)
  constexpr int PC = VEC ? 64 : GV_CH;
  constexpr int NW = VEC ? PC * EB / 4 : GV_CH;  // words per piece
  const int64_t total = n * k * EB;
  const int voff = (int)(lane * k * EB);  // the host keeps 64 * k * bytes below 2^31
  for (int64_t p0 = kb; p0 < ke; p0 += PC) {
    const int64_t off = (j0 * k + p0) * EB;
    const int64_t rem = total - off;
    const int nrec = rem <= 0 ? 0 : (rem > 0x7FFFFFFF ? 0x7FFFFFFF : (int)rem);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(w + (rem > 0 ? off : 0)), (short)0, nrec, RSRC_WORD3);
    uint32_t buf[NW];
    if constexpr (VEC) {
#pragma unroll
      for (int l = 0; l < NW / 4; ++l) {
        const u4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff + l * 16, 0, 0);
        buf[4 * l] = v[0]; buf[4 * l + 1] = v[1]; buf[4 * l + 2] = v[2]; buf[4 * l + 3] = v[3];
      }
    } else {
#pragma unroll
      for (int i = 0; i < GV_CH; ++i) {
        if constexpr (BT == T_F32) buf[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff + i * 4, 0, 0);
        else if constexpr (BT == T_BF16) buf[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, voff + i * 2, 0, 0);
        else buf[i] = __builtin_amdgcn_raw_buffer_load_b8(rs, voff + i, 0, 0);
      }
    }
    const int64_t nrow = ke - p0;
    if (nrow >= PC) gv_steps_nt<BT, MR, VEC, true, PC>(acc, buf, x, k, p0, PC, m, sc);
    else gv_steps_nt<BT, MR, VEC, false, PC>(acc, buf, x, k, p0, (int)nrow, m, sc);
  }
}

// The completing workgroup's fold when the group count NG is a power of two (the decode shapes:
// 32 leaves in groups of 8 or 4): the rest of the contract's tree is then complete -- adjacent
// pairs, level by level -- and every root of up to 8 of this thread's cells is requested at once.
template <int NG, int MR, int COLS, int THREADS, int CPT>
__device__ __forceinline__ void gv_fold_pow2(const GemvArgs& g, int tid, int64_t cg, int m) {
  constexpr int CB = CPT < 8 ? CPT : 8;
#pragma unroll
  for (int c0 = 0; c0 < CPT; c0 += CB) {
    float v[CB][NG];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const int cell = tid + (c0 + c) * THREADS;
      const int r = cell / COLS, col = cell % COLS;
      const int64_t j = cg * COLS + col;
      if (c0 + c >= CPT || cell >= MR * COLS || r >= m || j >= g.n) continue;
#pragma unroll
      for (int e = 0; e < NG; ++e)
        v[c][e] = __hip_atomic_load(g.ws + (e * g.m + r) * g.n + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int c = 0; c < CB; ++c) {
      const int cell = tid + (c0 + c) * THREADS;
      const int r = cell / COLS, col = cell % COLS;
      const int64_t j = cg * COLS + col;
      if (c0 + c >= CPT || cell >= MR * COLS || r >= m || j >= g.n) continue;
#pragma unroll
      for (int w = NG; w > 1; w /= 2)
#pragma unroll
        for (int q = 0; q < w / 2; ++q) v[c][q] = v[c][2 * q] + v[c][2 * q + 1];
      float y = v[c][0];
      if (g.bias) y = y + g.bias[j];
      g.c[r * g.n + j] = store_word(y);
    }
  }
}

// The end of a skinny product, once every wave has written its leaf partial into
// part[wave][row][col]: the workgroup's root (the tree over its up to LEAVES leaves),
// then either the store (one group) or the count and, in the workgroup that completes it,
// the fold of every group's root (the rest of the contract's tree), bias and store.
//
// LPN (leaves per node) 2 or 4: each wave ran LPN adjacent leaves (an aligned subtree) and
// wrote that subtree's node -- for the last, partial subtree the contract's tree over the leaves
// it has, the odd one carried -- so part holds LEAVES / LPN nodes, and the tree over them is the
// rest of the contract's tree over the workgroup's leaves.
template <int MR, int COLS, int LEAVES = GV_LEAVES, int THREADS = GV_THREADS, int LPN = 1>
__device__ __forceinline__ void gv_finish(const GemvArgs& g, float (&part)[LEAVES / LPN][MR][COLS],
                                          unsigned int& last_flag, int tid, int64_t grp, int64_t cg, int m) {
  constexpr int NODES = LEAVES / LPN;
  static_assert(LPN == 1 || LPN == 2 || LPN == 4, "a node is a subtree of 1, 2 or 4 leaves");
  static_assert(NODES == 2 || NODES == 4 || NODES == 8 || NODES == 16, "a workgroup folds 2 .. 16 nodes");
  static_assert(LPN > 1 || LEAVES == 4 || LEAVES == 8, "workgroups of single-leaf nodes fold 4 or 8 leaves");
  __syncthreads();
  const int64_t left = g.nleaves - grp * LEAVES;
  const int cntl = left < LEAVES ? (int)left : LEAVES;
  const int cnt = (cntl + LPN - 1) / LPN;  // nodes written
  constexpr int CPT = (MR * COLS + THREADS - 1) / THREADS;  // cells per thread
  constexpr int LB = CPT < 4 ? CPT : 4;                      // cells per batch of LDS reads
  // this thread's cells tid + c * THREADS of rows < m, LB at a time: every partial of a
  // batch read before any add
#pragma unroll
  for (int c0 = 0; c0 < CPT; c0 += LB) {
    float p[NODES][LB];
#pragma unroll
    for (int c = 0; c < LB; ++c) {
      const int cell = tid + (c0 + c) * THREADS;
      const int r = cell / COLS, col = cell % COLS;
      if (c0 + c >= CPT || cell >= MR * COLS || r >= m) continue;
#pragma unroll
      for (int l = 0; l < NODES; ++l)
        if (l < cnt) p[l][c] = part[l][r][col];
    }
#pragma unroll
    for (int c = 0; c < LB; ++c) {
      const int cell = tid + (c0 + c) * THREADS;
      const int r = cell / COLS, col = cell % COLS;
      const int64_t j = cg * COLS + col;
      if (c0 + c >= CPT || cell >= MR * COLS || r >= m || j >= g.n) continue;
      float y;
      if (cnt == NODES) {
        // the complete aligned subtree: adjacent pairs, level by level
        float v[NODES];
#pragma unroll
        for (int l = 0; l < NODES; ++l) v[l] = p[l][c];
#pragma unroll
        for (int w = NODES; w > 1; w /= 2)
#pragma unroll
          for (int q = 0; q < w / 2; ++q) v[q] = v[2 * q] + v[2 * q + 1];
        y = v[0];
      } else {
        // the tail of the tree (the last group, fewer leaves): the odd one carried up
        float v[NODES];
#pragma unroll
        for (int l = 0; l < NODES; ++l) v[l] = l < cnt ? p[l][c] : 0.f;
        int w = cnt;
#pragma unroll 1
        while (w > 1) {
#pragma unroll
          for (int q = 0; q < NODES / 2; ++q)
            if (q < w / 2) v[q] = v[2 * q] + v[2 * q + 1];
#pragma unroll
          for (int q = 0; q < NODES / 2; ++q)
            if ((w & 1) && q == w / 2) v[q] = v[w - 1];
          w = (w + 1) / 2;
        }
        y = v[0];
      }
      if (g.ngroups == 1) {
        if (g.bias) y = y + g.bias[j];  // ftz(C) + ftz(b) by the input flush
        g.c[r * g.n + j] = store_word(y);
      } else {
        __hip_atomic_store(&g.ws[(grp * g.m + r) * g.n + j], y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  if (g.ngroups == 1) return;

  // Count this group's roots in; the workgroup that completes the count folds.  The hand-off
  // is ordered at the ISA level, on words that are all agent-scope atomics:
  //  - each root is an agent-scope atomic store (global_store ... sc1): written through to the
  //    device's coherence point, never left dirty in one XCD's L2;
  //  - s_waitcnt vmcnt(0), then the barrier: every root store of the workgroup is acknowledged
  //    before thread 0 issues the count;
  //  - the count is an agent-scope read-modify-write, performed at the coherence point, so the
  //    workgroup that reads ngroups - 1 comes after every other group's count;
  //  - that workgroup reads the roots with agent-scope atomic loads (sc1), at the coherence point.
  // A C++ release/acquire pair would order the same steps, but its release compiles to
  // buffer_wbl2 sc1 (a writeback of the XCD's whole L2) in every workgroup: measured on the
  // decode GEMV at M = 1, 16.1 -> 27.5 us.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  if (tid == 0) {
    const unsigned int prev = __hip_atomic_fetch_add(&g.counter[cg], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev + 1 == (unsigned int)g.ngroups ? 1u : 0u;
  }
  __syncthreads();
  if (!last_flag) return;
  const int64_t stride = g.m * g.n;
  if (g.ngroups == 2) {
    gv_fold_pow2<2, MR, COLS, THREADS, CPT>(g, tid, cg, m);
  } else if (g.ngroups == 4) {
    gv_fold_pow2<4, MR, COLS, THREADS, CPT>(g, tid, cg, m);
  } else if (g.ngroups == 8) {
    gv_fold_pow2<8, MR, COLS, THREADS, CPT>(g, tid, cg, m);
  } else if (g.ngroups <= GV_FEW_GROUPS) {
    // every root of up to 8 cells of this thread requested at once, then folded
    constexpr int CB = CPT < 8 ? CPT : 8;
#pragma unroll
    for (int c0 = 0; c0 < CPT; c0 += CB) {
      float v[CB][GV_FEW_GROUPS];
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        const int cell = tid + (c0 + c) * THREADS;
        const int r = cell / COLS, col = cell % COLS;
        const int64_t j = cg * COLS + col;
        if (c0 + c >= CPT || cell >= MR * COLS || r >= m || j >= g.n) continue;
#pragma unroll
        for (int e = 0; e < GV_FEW_GROUPS; ++e)
          if (e < g.ngroups)
            v[c][e] = __hip_atomic_load(g.ws + (e * g.m + r) * g.n + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
#pragma unroll
      for (int c = 0; c < CB; ++c) {
        const int cell = tid + (c0 + c) * THREADS;
        const int r = cell / COLS, col = cell % COLS;
        const int64_t j = cg * COLS + col;
        if (c0 + c >= CPT || cell >= MR * COLS || r >= m || j >= g.n) continue;
        StackF stk;
        const int P = (int)g.ngroups;
#pragma unroll
        for (int e = 0; e + 1 < GV_FEW_GROUPS; ++e)
          if (e + 1 < P) stk.push(v[c][e], e);
        float y = v[c][0];
#pragma unroll
        for (int e = 1; e < GV_FEW_GROUPS; ++e)
          if (e == P - 1) y = v[c][e];
        y = stk.root(y, P - 1);
        if (g.bias) y = y + g.bias[j];
        g.c[r * g.n + j] = store_word(y);
      }
    }
  } else {
#pragma unroll 1
    for (int cell = tid; cell < MR * COLS; cell += THREADS) {
      const int r = cell / COLS, col = cell % COLS;
      const int64_t j = cg * COLS + col;
      if (r >= m || j >= g.n) continue;
      float y = fold_roots(g.ws + r * g.n + j, g.ngroups, stride);
      if (g.bias) y = y + g.bias[j];
      g.c[r * g.n + j] = store_word(y);
    }
  }
  if (tid == 0) __hip_atomic_store(&g.counter[cg], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One skinny product: OP_NN (W[k][n], FULLLEAF: every leaf exactly 128 rows) or OP_NT (W[n][k]),
// LEAVES leaves (waves) a workgroup.  The argument block is taken by value: the compiler then
// requests both of its cache lines before the workgroup index split (measured 1-2% at M <= 2).
template <int BT, int MR, bool VEC, bool FULLLEAF, bool NT, int LEAVES = GV_LEAVES>
__device__ __forceinline__ void gemv_body(GemvArgs g, const float* __restrict__ x) {
  constexpr int CPL = GvCols<BT, NT, FULLLEAF>::cpl;
  constexpr int COLS = GvCols<BT, NT, FULLLEAF>::cols;
  constexpr int EB = Elem<BT>::bytes;
  static_assert(LEAVES == GV_LEAVES || (FULLLEAF && !NT), "wide workgroups take whole leaves");
  __shared__ float part[LEAVES][MR][COLS];
  __shared__ unsigned int last_flag;

  set_flush_inputs_mode();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: leaf and k range too
  // the grid holds at most INT32_MAX workgroups (the host refuses more): a 32-bit split
  const int64_t cg = blockIdx.x % (uint32_t)g.ncg;
  const int64_t grp = blockIdx.x / (uint32_t)g.ncg;
  const int64_t t = grp * LEAVES + wave;  // this wave's leaf
  const int m = (int)g.m;

  float acc[MR][CPL];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int e = 0; e < CPL; ++e) acc[r][e] = 0.f;

  if constexpr (NT) {
    if (t < g.nleaves) {
      const int64_t j0 = cg * COLS;
      float sc = 1.f;
      if constexpr (BT == T_I8) sc = g.scales[j0 + lane < g.n ? j0 + lane : g.n - 1];
      const int64_t kb = t * g.leaf;
      const int64_t ke = kb + g.leaf < g.k ? kb + g.leaf : g.k;
      gv_leaf_nt<BT, MR, VEC>(acc, static_cast<const char*>(g.w), g.n, g.k, j0, kb, ke, x, m, sc, lane);
    }
  } else if (t < g.nleaves) {
    // this lane's columns, clamped into the operand (their cells are never stored)
    int64_t c0 = cg * COLS + lane * CPL;
    uint32_t coff[CPL];
    float sc[CPL];
    if constexpr (VEC) {
      if (c0 >= g.n) c0 = g.n - CPL;
#pragma unroll
      for (int e = 0; e < CPL; ++e) coff[e] = (uint32_t)((c0 + e) * EB);
    } else {
#pragma unroll
      for (int e = 0; e < CPL; ++e) coff[e] = (uint32_t)((c0 + e < g.n ? c0 + e : g.n - 1) * EB);
    }
#pragma unroll
    for (int e = 0; e < CPL; ++e) {
      sc[e] = 1.f;
      if constexpr (BT == T_I8) sc[e] = g.scales[coff[e]];  // EB == 1: the offset is the column
    }
    const char* w = static_cast<const char*>(g.w);
    const uint32_t loff = coff[0];
    const int64_t rowbytes = g.n * EB;
    const int64_t kb = t * g.leaf;
    const int64_t ke = kb + g.leaf < g.k ? kb + g.leaf : g.k;
    const int64_t klast = ke - 1;

    if constexpr (FULLLEAF) {
      gv_leaf_full<BT, MR>(acc, w + kb * rowbytes, loff, (int)rowbytes, x + kb, g.k, m, sc);
    } else {
      // The general case: the leaf's rows in pieces of GV_CH (one piece unless the leaf is
      // longer than 128); every row of a piece is requested before its first step, and the
      // steps consume them in order as they land.
      uint32_t buf[GV_CH];
      for (int64_t p0 = kb; p0 < ke; p0 += GV_CH) {
        const int64_t nrow = ke - p0;
        gv_load<BT, VEC>(buf, w, loff, coff, rowbytes, p0, klast);
        if (nrow >= GV_CH) gv_steps<BT, MR, true>(acc, buf, x, g.k, p0, GV_CH, m, sc);
        else gv_steps<BT, MR, false>(acc, buf, x, g.k, p0, (int)nrow, m, sc);
      }
    }
  }

  // The group's root: the tree over its (up to LEAVES) leaf partials, through LDS.
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int e = 0; e < CPL; ++e) part[wave][r][lane * CPL + e] = acc[r][e];
  gv_finish<MR, COLS, LEAVES, 64 * LEAVES>(g, part, last_flag, tid, grp, cg, m);
}

}  // namespace mlg

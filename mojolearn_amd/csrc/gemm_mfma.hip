// gfx950 MFMA GEMM kernel of mojolearn.identical.gemm.fp32.v1 (any m, n, k; NN, NT, TN; f32, bf16, int8).
#include "act.h"
#include "device_common.h"
#include "lds_stage.h"
#include "mfma.h"

namespace mlg {

__device__ __forceinline__ v32f vadd(const v32f& x, const v32f& y) {
  v32f r;
#pragma unroll
  for (int e = 0; e < 32; ++e) r[e] = x[e] + y[e];
  return r;
}

// Register-stack fold of up to 32 leaf partials per output cell.  Slots 0-3 are named
// registers (every access static); slot 4, written once per 16 leaves and read once per
// 32, lives in this wave's private LDS area as [32 elements / 4][64 lanes][4].
struct Stack32 {
  v32f s0, s1, s2, s3;
  f4* s4;  // this lane's first f4 of the wave's LDS slot

  __device__ __forceinline__ void put4(const v32f& x) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      f4 v = {x[4 * e], x[4 * e + 1], x[4 * e + 2], x[4 * e + 3]};
      s4[e * 64] = v;
    }
  }
  __device__ __forceinline__ v32f get4() const {
    v32f x;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const f4 v = s4[e * 64];
      x[4 * e] = v[0]; x[4 * e + 1] = v[1]; x[4 * e + 2] = v[2]; x[4 * e + 3] = v[3];
    }
    return x;
  }
  // Push partial number t (0-based, t <= 30): merge slot l while bit l of t is 1, then
  // store into the first slot whose bit is 0.  x is used as the running sum (its value is
  // not needed afterwards).
  __device__ __forceinline__ void push(v32f& x, int t) {
    if (!(t & 1)) { s0 = x; return; }
    x = vadd(s0, x);
    if (!(t & 2)) { s1 = x; return; }
    x = vadd(s1, x);
    if (!(t & 4)) { s2 = x; return; }
    x = vadd(s2, x);
    if (!(t & 8)) { s3 = x; return; }
    x = vadd(s3, x);
    put4(x);
  }
  // The last partial (number t <= 31): the group's root, combining slot l for every set
  // bit l of t, lowest level first.
  __device__ __forceinline__ v32f root(v32f x, int t) const {
    if (t & 1) x = vadd(s0, x);
    if (t & 2) x = vadd(s1, x);
    if (t & 4) x = vadd(s2, x);
    if (t & 8) x = vadd(s3, x);
    if (t & 16) x = vadd(get4(), x);
    return x;
  }
};

// MFMA steps s0 .. s1-1 of one staged slice, in ascending order.  The slice is walked in
// aligned groups of 4 steps whose operands are read from LDS one group ahead; unless FULL,
// a step outside [s0, s1) is skipped by a uniform branch.  The scheduling fences keep the
// compiler from hoisting every LDS read of the slice, which would not fit beside the
// accumulator and the fold slots.
template <int OP, int AT, int BT, bool FULL, bool FRESH = false>
__device__ __forceinline__ void mfma_steps(v32f& acc, const char* la, const char* lb, int s0, int s1,
                                           int arow, int bcol, float scale) {
  constexpr bool A_IMAJ = (OP != OP_TN);
  constexpr bool B_IMAJ = (OP == OP_NT);
  f4 a4 = read4<AT, A_IMAJ>(la, arow, 0, 1.f);
  f4 b4 = read4<BT, B_IMAJ>(lb, bcol, 0, scale);
#pragma unroll
  for (int s = 0; s < KT; s += 4) {
    f4 an, bn;
    if (s + 4 < KT) {
      an = read4<AT, A_IMAJ>(la, arow, s + 4, 1.f);
      bn = read4<BT, B_IMAJ>(lb, bcol, s + 4, scale);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      // FRESH: the slice starts a leaf, whose chain starts from +0 (the MFMA's C operand)
      if (FRESH && s + q == 0) acc = __builtin_amdgcn_mfma_f32_32x32x1f32(a4[q], b4[q], v32f{}, 0, 0, 0);
      else if (FULL || (s + q >= s0 && s + q < s1)) acc = __builtin_amdgcn_mfma_f32_32x32x1f32(a4[q], b4[q], acc, 0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    if (s + 4 < KT) { a4 = an; b4 = bn; }
  }
}

// ACT: the store applies an activation follower (GemmArgs::epi 4 or 5; an instantiation of its
// own, so the other products' kernels carry none of its code).
template <int OP, int AT, int BT, bool ACT = false>
__global__ void __launch_bounds__(NTHREADS) gemm_mfma_kernel(GemmArgs g) {
  constexpr bool A_IMAJ = (OP != OP_TN);
  constexpr bool B_IMAJ = (OP == OP_NT);
  // three slice buffers [A, B], separate objects so the compiler can tell them apart
  __shared__ __attribute__((aligned(1024))) char lds0[2][SLICE_BYTES];
  __shared__ __attribute__((aligned(1024))) char lds1[2][SLICE_BYTES];
  __shared__ __attribute__((aligned(1024))) char lds2[2][SLICE_BYTES];

  __shared__ f4 slot4[NWAVES][8][64];  // fold slot 4, per wave

  set_flush_inputs_mode();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 2;  // 0..1: rows wr*64 .. +63
  const int wc = wave & 3;   // 0..3: cols wc*32 .. +31

  const int tile = tile_of(blockIdx.x, gridDim.x, g.tiles_m, g.tiles_n);
  const int64_t i0 = (int64_t)(tile / g.tiles_n) * BM;
  const int64_t j0 = (int64_t)(tile % g.tiles_n) * BN;
  const int64_t grp = blockIdx.y;

  const int64_t t_first = grp * g.group;
  int64_t t_last = t_first + g.group;
  if (t_last > g.nleaves) t_last = g.nleaves;
  const int cnt = (int)(t_last - t_first);
  const int64_t kb = t_first * g.leaf;
  int64_t ke = t_last * g.leaf;
  if (ke > g.k) ke = g.k;

  const int64_t kt_first = kb / KT;
  const int64_t kt_last = (ke - 1) / KT;

  DirectLoader<AT, A_IMAJ> lda;
  DirectLoader<BT, B_IMAJ> ldb;
  lda.init(g.a_pitch, wave, lane);
  ldb.init(g.b_pitch, wave, lane);
  // loads per slice per wave: every wave issues the same count, so vmcnt(LPS) waits for all
  // but the most recent slice's loads
  constexpr int LPS = Slice<AT, A_IMAJ>::PER_WAVE + Slice<BT, B_IMAJ>::PER_WAVE;
  constexpr int WAIT_ONE_BEHIND = (LPS & 0xF) | ((LPS >> 4) << 14) | (0x7 << 4) | (0xF << 8);
  // Slices are loaded unconditionally, two ahead: one past the group's last slice reads
  // zeros or bytes no step uses (the resource bounds keep it inside the operand).
  lda.issue(lds0[0], g.a, g.a_bytes, g.a_pitch, i0, kt_first * KT, wave);
  ldb.issue(lds0[1], g.b, g.b_bytes, g.b_pitch, j0, kt_first * KT, wave);
  lda.issue(lds1[0], g.a, g.a_bytes, g.a_pitch, i0, (kt_first + 1) * KT, wave);
  ldb.issue(lds1[1], g.b, g.b_bytes, g.b_pitch, j0, (kt_first + 1) * KT, wave);

  const int arow = wr * 64 + lane;
  const int bcol = wc * 32 + (lane & 31);
  float scale = 1.f;
  if constexpr (BT == T_I8) {
    int64_t j = j0 + bcol;
    if (j >= g.n) j = g.n - 1;
    scale = g.scales[j];
  }

  v32f acc;
#pragma unroll
  for (int e = 0; e < 32; ++e) acc[e] = 0.f;
  Stack32 stk;
  stk.s4 = &slot4[wave][0][lane];

  int t = 0;  // leaf number within the group
  int64_t leaf_end = (t_first + 1) * g.leaf;
  if (leaf_end > g.k) leaf_end = g.k;

  // the first slice has landed (the second may still be in flight)
  __builtin_amdgcn_s_waitcnt(WAIT_ONE_BEHIND);
  lds_barrier();

  // One slice: fill buffer FILL with slice kt + 2 (it was last read before the previous
  // slice's barrier), run slice kt's steps out of buffer CUR (pushing each finished leaf;
  // after the group's last leaf acc holds the group's root), wait for slice kt + 1.  The
  // loop below is unrolled by NBUF, so every step names its buffers as distinct objects and
  // the compiler does not make the reads of slice kt wait for the loads of slice kt + 2.
#define MLG_SLICE_STEP(CUR, FILL) \
  do { \
    lda.issue(FILL[0], g.a, g.a_bytes, g.a_pitch, i0, (kt + 2) * KT, wave); \
    ldb.issue(FILL[1], g.b, g.b_bytes, g.b_pitch, j0, (kt + 2) * KT, wave); \
    const char* la = CUR[0]; \
    const char* lb = CUR[1]; \
    const int64_t tbase = kt * KT; \
    int64_t pos = tbase > kb ? tbase : kb; \
    int64_t hi = tbase + KT; \
    if (hi > ke) hi = ke; \
    while (pos < hi) { \
      const int64_t seg = hi < leaf_end ? hi : leaf_end; \
      if (pos == tbase && seg == tbase + KT) \
        mfma_steps<OP, AT, BT, true>(acc, la, lb, 0, KT, arow, bcol, scale); \
      else \
        mfma_steps<OP, AT, BT, false>(acc, la, lb, (int)(pos - tbase), (int)(seg - tbase), arow, bcol, scale); \
      pos = seg; \
      if (pos == leaf_end) { \
        if (t + 1 < cnt) { \
          stk.push(acc, t); \
          _Pragma("unroll") for (int e = 0; e < 32; ++e) acc[e] = 0.f; \
          ++t; \
          leaf_end = (t_first + t + 1) * g.leaf; \
          if (leaf_end > g.k) leaf_end = g.k; \
        } else { \
          acc = stk.root(acc, t); \
        } \
      } \
    } \
    __builtin_amdgcn_s_waitcnt(WAIT_ONE_BEHIND); \
    lds_barrier(); \
  } while (0)
  // The regular case (every decoder shape: leaves of whole slices, k a multiple of KT):
  // every slice runs all KT steps, and a leaf ends after exactly `spl` slices.
#define MLG_REGULAR_STEP(CUR, FILL) \
  do { \
    lda.issue(FILL[0], g.a, g.a_bytes, g.a_pitch, i0, (kt + 2) * KT, wave); \
    ldb.issue(FILL[1], g.b, g.b_bytes, g.b_pitch, j0, (kt + 2) * KT, wave); \
    if (sl == 0) mfma_steps<OP, AT, BT, true, true>(acc, CUR[0], CUR[1], 0, KT, arow, bcol, scale); \
    else mfma_steps<OP, AT, BT, true>(acc, CUR[0], CUR[1], 0, KT, arow, bcol, scale); \
    if (++sl == spl) { \
      sl = 0; \
      if (t + 1 < cnt) { \
        stk.push(acc, t); \
        ++t; \
      } else { \
        acc = stk.root(acc, t); \
      } \
    } \
    __builtin_amdgcn_s_waitcnt(WAIT_ONE_BEHIND); \
    lds_barrier(); \
  } while (0)
  static_assert(NBUF == 3, "the slice loop is unrolled by NBUF");
  if (!g.seed && g.leaf % KT == 0 && ke % KT == 0) {
    const int spl = (int)(g.leaf / KT);
    int sl = 0;
    for (int64_t kt = kt_first; kt <= kt_last;) {
      MLG_REGULAR_STEP(lds0, lds2);
      if (++kt > kt_last) break;
      MLG_REGULAR_STEP(lds1, lds0);
      if (++kt > kt_last) break;
      MLG_REGULAR_STEP(lds2, lds1);
      ++kt;
    }
  } else {
    if (g.seed) {
      // one leaf: the chain starts from the old C cell (flushed as the first step's C input)
      const int64_t col = j0 + bcol;
      if (col < g.n) {
#pragma unroll
        for (int e = 0; e < 32; ++e) {
          const int blk = e >> 4, rr = e & 15;
          const int64_t row = i0 + wr * 64 + 32 * blk + (rr & 3) + 8 * (rr >> 2) + 4 * (lane >> 5);
          if (row < g.m) acc[e] = g.c[row * g.ldc + col];
        }
      }
    }
    for (int64_t kt = kt_first; kt <= kt_last;) {
      MLG_SLICE_STEP(lds0, lds2);
      if (++kt > kt_last) break;
      MLG_SLICE_STEP(lds1, lds0);
      if (++kt > kt_last) break;
      MLG_SLICE_STEP(lds2, lds1);
      ++kt;
    }
  }
#undef MLG_REGULAR_STEP
#undef MLG_SLICE_STEP
  // no load into LDS may outlive the workgroup
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  // acc holds the group root.  Element e -> block b = e/16, row (e%4) + 8*((e%16)/4) + 4*(lane/32) within it.
  const int64_t col = j0 + bcol;
  if (col < g.n) {
    if (ACT && g.ngroups == 1) {
      // the activation followers: the root staged through this wave's fold slot (free now),
      // then one cell at a time (a rolled loop: the activation's code once, not 32 times)
      stk.put4(acc);
      const float* staged = reinterpret_cast<const float*>(stk.s4);
#pragma unroll 1
      for (int e = 0; e < 32; ++e) {
        const int blk = e >> 4, rr = e & 15;
        const int64_t row = i0 + wr * 64 + 32 * blk + (rr & 3) + 8 * (rr >> 2) + 4 * (lane >> 5);
        if (row < g.m) {
          const float y = staged[(e >> 2) * 64 * 4 + (e & 3)];
          const float q = g.epi == EPI_ACT_BWD ? g.epi_p[row * g.n + col] : g.epi_p[col];
          g.c[row * g.ldc + col] = store_word(follow_one(act_ftz(y), g.epi, q, g.act));
        }
      }
    } else if (g.ngroups == 1) {
      const float bj = g.epi == EPI_PLUS_BIAS ? g.epi_p[col] : 0.f;
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        const int blk = e >> 4, rr = e & 15;
        const int64_t row = i0 + wr * 64 + 32 * blk + (rr & 3) + 8 * (rr >> 2) + 4 * (lane >> 5);
        if (row < g.m) {
          float y = acc[e];
          if (g.epi == EPI_PLUS_BIAS) y = y + bj;  // ftz(C) + ftz(b) by the input flush
          g.c[row * g.ldc + col] = store_word(y);
        }
      }
    } else {
      float* wsg = g.ws + grp * g.m * g.n;
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        const int blk = e >> 4, rr = e & 15;
        const int64_t row = i0 + wr * 64 + 32 * blk + (rr & 3) + 8 * (rr >> 2) + 4 * (lane >> 5);
        if (row < g.m) wsg[row * g.n + col] = acc[e];
      }
    }
  }
}

// Copy a stored operand [rows][cols] of `eb`-byte elements into [rows][pitch] (pitch a
// multiple of 16 bytes, zero padding), so that the product kernel's 16-byte loads are
// aligned and never straddle a row end.
__global__ void repack_rows_kernel(char* dst, const char* src, int64_t rows, int64_t cols, int64_t pitch,
                                   int eb, int64_t s_r, int64_t s_c) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * pitch) return;
  const int64_t r = i / pitch, cidx = i % pitch;
  const int64_t from = r * s_r + cidx * s_c;
  if (eb == 4) {
    reinterpret_cast<uint32_t*>(dst)[i] = cidx < cols ? reinterpret_cast<const uint32_t*>(src)[from] : 0u;
  } else if (eb == 2) {
    reinterpret_cast<uint16_t*>(dst)[i] = cidx < cols ? reinterpret_cast<const uint16_t*>(src)[from] : (uint16_t)0;
  } else {
    dst[i] = cidx < cols ? src[from] : (char)0;
  }
}

__global__ void __launch_bounds__(256) fold_groups_kernel(float* c, int64_t ldc, const float* ws, int64_t m, int64_t n,
                                                          int64_t ngroups, int epi, const float* epi_p, int act) {
  set_flush_inputs_mode();
  const int64_t cell = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t cells = m * n;
  if (cell >= cells) return;
  float y = 0.f;  // k == 0: +0.0
  if (ngroups > 0) {
    StackF stk;
    int64_t t = 0;
    for (; t + 1 < ngroups; ++t) stk.push(ws[t * cells + cell], (int)t);
    y = stk.root(ws[t * cells + cell], (int)t);
  }
  const int64_t row = cell / n, col = cell - row * n;
  if (epi != EPI_NONE) {
    const float q = epi == EPI_ACT_BWD ? epi_p[row * n + col] : epi_p[col];
    y = follow_one(act_ftz(y), epi, q, act);
  }
  c[row * ldc + col] = store_word(y);
}

template <int OP, int AT, int BT, bool ACT = false>
static hipError_t launch_one(const GemmArgs& g, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((gemm_mfma_kernel<OP, AT, BT, ACT>), grid, dim3(NTHREADS), 0, stream, g);
  return hipGetLastError();
}

template <int OP>
static hipError_t launch_types(const GemmArgs& g, int at, int bt, dim3 grid, hipStream_t s) {
  if (g.epi >= EPI_BIAS_ACT && g.ngroups == 1) {
    // the activation followers (the sequence word: float32 operands only)
    if (at != T_F32 || bt != T_F32) return hipErrorInvalidValue;
    return launch_one<OP, T_F32, T_F32, true>(g, grid, s);
  }
  if (at == T_F32) {
    if (bt == T_F32) return launch_one<OP, T_F32, T_F32>(g, grid, s);
    if (bt == T_BF16) return launch_one<OP, T_F32, T_BF16>(g, grid, s);
    return launch_one<OP, T_F32, T_I8>(g, grid, s);
  }
  if (bt == T_BF16) return launch_one<OP, T_BF16, T_BF16>(g, grid, s);
  return hipErrorInvalidValue;
}

hipError_t launch_mfma(const GemmArgs& g, int op, int a_type, int b_type, dim3 grid, hipStream_t stream) {
  if (op == OP_NN) return launch_types<OP_NN>(g, a_type, b_type, grid, stream);
  if (op == OP_NT) return launch_types<OP_NT>(g, a_type, b_type, grid, stream);
  return launch_types<OP_TN>(g, a_type, b_type, grid, stream);
}

hipError_t launch_repack(char* dst, const char* src, int64_t rows, int64_t cols, int64_t pitch, int eb,
                         int64_t s_r, int64_t s_c, hipStream_t stream) {
  const int64_t total = rows * pitch;
  hipLaunchKernelGGL(repack_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, dst, src,
                     rows, cols, pitch, eb, s_r, s_c);
  return hipGetLastError();
}

hipError_t launch_fold_groups(float* c, int64_t ldc, const float* ws, int64_t m, int64_t n, int64_t ngroups, int epi,
                              const float* epi_p, int act, hipStream_t stream) {
  const int64_t cells = m * n;
  hipLaunchKernelGGL(fold_groups_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, stream, c, ldc, ws, m,
                     n, ngroups, epi, epi_p, act);
  return hipGetLastError();
}

}  // namespace mlg

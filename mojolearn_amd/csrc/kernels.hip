// gfx950 kernels for mojolearn.identical.gemm.fp32.v1.
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
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "contract.h"
#include "kernels.h"

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

// ---------------------------------------------------------------------------
// Tiling: 512 threads = 8 waves (2 per SIMD); workgroup tile 128 x 128 cells; each
// wave owns 64 rows x 32 columns = one v_mfma_f32_32x32x1_2b_f32 (block 0 = rows 0-31,
// block 1 = rows 32-63, both against the same 32 columns).  K is staged through LDS
// in KT = 32 slices, double buffered.
constexpr int NTHREADS = 512;
constexpr int BM = 128;
constexpr int BN = 128;
constexpr int KT = 32;
constexpr int IP = KT + 4;    // pitch of an index-major slice [128][KT] (k contiguous)
constexpr int KP = BM + 4;    // pitch of a k-major slice [KT][128] (index contiguous)
constexpr int SLICE = BM * IP;  // floats per operand slice buffer (>= KT * KP)
constexpr int MAX_GROUP_LEAVES = 32;  // one group's leaves fold in registers

static_assert(KT * KP <= SLICE, "slice buffer");

// Operand staging for one KT slice of a stored row-major operand [rows][cols] of element
// type T: 4096 elements = 1024 chunks of 4 consecutive elements along `cols`, two chunks
// per thread.  Index-major (IMAJ) slices are [BM indices][KT k] (the operand stores k
// contiguously); k-major slices are [KT k][BM indices].  The per-thread pointers are
// fixed for the whole k loop (a slice only adds a uniform k offset); chunk coordinates
// are recomputed from the thread id, which costs VALU slots the MFMA loop leaves idle
// rather than registers it needs.
template <int T>
struct ElemBytes { static constexpr int v = T == T_F32 ? 4 : (T == T_BF16 ? 2 : 1); };

template <bool IMAJ>
__device__ __forceinline__ void chunk_coords(int q, int64_t idx0, int64_t& idx, int& koff) {
  if constexpr (IMAJ) { idx = idx0 + (q >> 3); koff = (q & 7) << 2; }
  else { idx = idx0 + ((q & 31) << 2); koff = q >> 5; }
}

template <int T, bool IMAJ>
struct Stager {
  const char* ptr[2];  // the chunk's first element at k = 0
  f4 reg[2];

  __device__ __forceinline__ void init(const void* base, int64_t cols, int64_t idx0, int tid) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int64_t idx; int koff;
      chunk_coords<IMAJ>(tid + NTHREADS * h, idx0, idx, koff);
      const int64_t off = IMAJ ? idx * cols + koff : (int64_t)koff * cols + idx;
      ptr[h] = static_cast<const char*>(base) + off * ElemBytes<T>::v;
    }
  }

  // Load the slice starting at k0 (uniform).  Elements outside the operand read as 0;
  // no k step ever uses one (the step count is exact) and no store reads one (index masks).
  __device__ __forceinline__ void load(int64_t rows, int64_t cols, int64_t idx0, int64_t k0,
                                       bool vec, const float* scales, int tid) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      int64_t idx; int koff;
      chunk_coords<IMAJ>(tid + NTHREADS * h, idx0, idx, koff);
      const int64_t kk = k0 + koff;
      bool ok;
      int64_t left;  // elements of the chunk inside the operand's row
      const char* p;
      if constexpr (IMAJ) {
        ok = idx < rows && kk < cols;
        left = cols - kk;
        p = ptr[h] + k0 * ElemBytes<T>::v;
      } else {
        ok = idx < cols && kk < rows;
        left = cols - idx;
        p = ptr[h] + k0 * cols * ElemBytes<T>::v;
      }
      f4 v = {0.f, 0.f, 0.f, 0.f};
      if (ok) {
        const bool full = vec && left >= 4;
        if constexpr (T == T_F32) {
          const float* fp = reinterpret_cast<const float*>(p);
          if (full) {
            v = *reinterpret_cast<const f4*>(fp);
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (e < left) v[e] = fp[e];
          }
        } else if constexpr (T == T_BF16) {
          const uint16_t* hp = reinterpret_cast<const uint16_t*>(p);
          uint32_t w[4] = {0u, 0u, 0u, 0u};
          if (full) {
            const uint2 u = *reinterpret_cast<const uint2*>(hp);
            w[0] = u.x & 0xFFFFu; w[1] = u.x >> 16; w[2] = u.y & 0xFFFFu; w[3] = u.y >> 16;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (e < left) w[e] = hp[e];
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = __uint_as_float(w[e] << 16);
        } else {
          const int8_t* bp = reinterpret_cast<const int8_t*>(p);
          int32_t code[4] = {0, 0, 0, 0};
          if (full) {
            const uint32_t u = *reinterpret_cast<const uint32_t*>(bp);
#pragma unroll
            for (int e = 0; e < 4; ++e) code[e] = (int32_t)(int8_t)(u >> (8 * e));
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (e < left) code[e] = bp[e];
          }
          // B_eff = fl32(f32(code) * ftz(scale[j])): MODE.FP_DENORM = 2 flushes the scale on
          // input, and the MFMA's input flush applies ftz to the product.  j is the chunk's
          // row for an [n][k] operand and its column for a [k][n] operand.
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float sc = IMAJ ? scales[idx] : scales[idx + (e < left ? e : 0)];
            v[e] = (float)code[e] * sc;
          }
        }
      }
      reg[h] = v;
    }
  }

  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int q = tid + NTHREADS * h;
      int o;
      if constexpr (IMAJ) o = (q >> 3) * IP + ((q & 7) << 2);
      else o = (q >> 5) * KP + ((q & 31) << 2);
      *reinterpret_cast<f4*>(lds + o) = reg[h];
    }
  }
};

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
  // store into the first slot whose bit is 0.
  __device__ __forceinline__ void push(v32f x, int t) {
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

struct GemmArgs {
  float* c;
  const void* a;
  const void* b;
  const float* scales;
  const float* bias;
  float* ws;          // group roots [ngroups][m][n] when ngroups > 1
  int64_t m, n, k;
  int64_t leaf;       // L
  int64_t nleaves;    // P
  int64_t group;      // leaves per group (power of two, <= 32)
  int64_t ngroups;
  int64_t a_rows, a_cols, b_rows, b_cols;  // stored shapes
  int tiles_n;
  int a_vec, b_vec;
};

template <int OP>
__device__ __forceinline__ void load_group(f4& a4, f4& b4, const float* la, const float* lb, int s,
                                           int arow, int bcol) {
  constexpr bool A_IMAJ = (OP != OP_TN);
  constexpr bool B_IMAJ = (OP == OP_NT);
  if constexpr (A_IMAJ) {
    a4 = *reinterpret_cast<const f4*>(la + arow * IP + s);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) a4[q] = la[(s + q) * KP + arow];
  }
  if constexpr (B_IMAJ) {
    b4 = *reinterpret_cast<const f4*>(lb + bcol * IP + s);
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) b4[q] = lb[(s + q) * KP + bcol];
  }
}

// MFMA steps s0 .. s1-1 of one staged K slice, in ascending order.  One code path for
// full and ragged slices (a separate loop for ragged ones gets its own copy of the
// accumulator): the slice is walked in aligned groups of 4 steps whose operands are
// read from LDS one group ahead, and a step outside [s0, s1) is skipped by a uniform
// branch.  The scheduling fences keep the compiler from hoisting every LDS read of the
// slice, which would not fit beside the accumulator and the fold slots.
template <int OP>
__device__ __forceinline__ void mfma_steps(v32f& acc, const float* la, const float* lb, int s0,
                                           int s1, int arow, int bcol) {
  f4 a4, b4;
  load_group<OP>(a4, b4, la, lb, 0, arow, bcol);
#pragma unroll
  for (int s = 0; s < KT; s += 4) {
    f4 an, bn;
    if (s + 4 < KT) load_group<OP>(an, bn, la, lb, s + 4, arow, bcol);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      if (s + q >= s0 && s + q < s1) acc = __builtin_amdgcn_mfma_f32_32x32x1f32(a4[q], b4[q], acc, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 4 < KT) { a4 = an; b4 = bn; }
  }
}

template <int OP, int AT, int BT>
__global__ void __launch_bounds__(NTHREADS) gemm_mfma_kernel(GemmArgs g) {
  constexpr bool A_IMAJ = (OP != OP_TN);
  constexpr bool B_IMAJ = (OP == OP_NT);
  __shared__ float lds[2][2][SLICE];  // [buffer][A,B][slice]
  __shared__ f4 slot4[NTHREADS / 64][8][64];  // fold slot 4, per wave

  set_flush_inputs_mode();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wr = wave >> 2;  // 0..1: rows wr*64 .. +63
  const int wc = wave & 3;   // 0..3: cols wc*32 .. +31

  const int tile = blockIdx.x;
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

  Stager<AT, A_IMAJ> sa;
  Stager<BT, B_IMAJ> sb;
  sa.init(g.a, g.a_cols, i0, tid);
  sb.init(g.b, g.b_cols, j0, tid);
  sa.load(g.a_rows, g.a_cols, i0, kt_first * KT, g.a_vec != 0, nullptr, tid);
  sb.load(g.b_rows, g.b_cols, j0, kt_first * KT, g.b_vec != 0, g.scales, tid);
  sa.store(lds[0][0], tid);
  sb.store(lds[0][1], tid);
  __syncthreads();

  const int arow = wr * 64 + lane;
  const int bcol = wc * 32 + (lane & 31);

  v32f acc;
#pragma unroll
  for (int e = 0; e < 32; ++e) acc[e] = 0.f;
  Stack32 stk;
  stk.s4 = &slot4[wave][0][lane];

  int t = 0;  // leaf number within the group
  int64_t leaf_end = (t_first + 1) * g.leaf;
  if (leaf_end > g.k) leaf_end = g.k;

  int buf = 0;
  for (int64_t kt = kt_first; kt <= kt_last; ++kt) {
    const bool more = kt < kt_last;
    if (more) {
      sa.load(g.a_rows, g.a_cols, i0, (kt + 1) * KT, g.a_vec != 0, nullptr, tid);
      sb.load(g.b_rows, g.b_cols, j0, (kt + 1) * KT, g.b_vec != 0, g.scales, tid);
    }
    const float* la = lds[buf][0];
    const float* lb = lds[buf][1];
    const int64_t tbase = kt * KT;
    int64_t pos = tbase > kb ? tbase : kb;
    int64_t hi = tbase + KT;
    if (hi > ke) hi = ke;
    while (pos < hi) {
      const int64_t seg = hi < leaf_end ? hi : leaf_end;
      mfma_steps<OP>(acc, la, lb, (int)(pos - tbase), (int)(seg - tbase), arow, bcol);
      pos = seg;
      if (pos == leaf_end) {
        if (t + 1 < cnt) {
          stk.push(acc, t);
#pragma unroll
          for (int e = 0; e < 32; ++e) acc[e] = 0.f;
          ++t;
          leaf_end = (t_first + t + 1) * g.leaf;
          if (leaf_end > g.k) leaf_end = g.k;
        } else {
          acc = stk.root(acc, t);  // the group's root; no step follows the last leaf
        }
      }
    }
    if (more) {
      sa.store(lds[buf ^ 1][0], tid);
      sb.store(lds[buf ^ 1][1], tid);
    }
    __syncthreads();
    buf ^= 1;
  }

  // acc holds the group root.  Store: acc element e -> block b = e/16, row (e%4) + 8*((e%16)/4) + 4*(lane/32) within it.
  const int64_t col = j0 + bcol;
  if (col < g.n) {
    if (g.ngroups == 1) {
      const float bj = g.bias ? g.bias[col] : 0.f;
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        const int blk = e >> 4, rr = e & 15;
        const int64_t row = i0 + wr * 64 + 32 * blk + (rr & 3) + 8 * (rr >> 2) + 4 * (lane >> 5);
        if (row < g.m) {
          float y = acc[e];
          if (g.bias) y = y + bj;  // ftz(C) + ftz(b) by the input flush
          g.c[row * g.n + col] = store_word(y);
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

// Upper tree levels: fold `ngroups` group roots per cell (a subtree per aligned group,
// so the rest of the contract's tree is the same rule applied to the roots).
// The same rule for up to 1024 scalar partials (ten levels), slots named.
struct StackF {
  float s0, s1, s2, s3, s4, s5, s6, s7, s8, s9;
#define MLG_PUSH_LEVEL(L)                      \
  if (!((t >> L) & 1)) { s##L = x; return; } \
  x = s##L + x;
  __device__ __forceinline__ void push(float x, int t) {
    MLG_PUSH_LEVEL(0) MLG_PUSH_LEVEL(1) MLG_PUSH_LEVEL(2) MLG_PUSH_LEVEL(3) MLG_PUSH_LEVEL(4)
    MLG_PUSH_LEVEL(5) MLG_PUSH_LEVEL(6) MLG_PUSH_LEVEL(7) MLG_PUSH_LEVEL(8)
    s9 = x;
  }
#undef MLG_PUSH_LEVEL
#define MLG_ROOT_LEVEL(L) \
  if ((t >> L) & 1) x = s##L + x;
  __device__ __forceinline__ float root(float x, int t) const {
    MLG_ROOT_LEVEL(0) MLG_ROOT_LEVEL(1) MLG_ROOT_LEVEL(2) MLG_ROOT_LEVEL(3) MLG_ROOT_LEVEL(4)
    MLG_ROOT_LEVEL(5) MLG_ROOT_LEVEL(6) MLG_ROOT_LEVEL(7) MLG_ROOT_LEVEL(8) MLG_ROOT_LEVEL(9)
    return x;
  }
#undef MLG_ROOT_LEVEL
};

__global__ void __launch_bounds__(256) fold_groups_kernel(float* c, const float* ws, const float* bias,
                                                          int64_t m, int64_t n, int64_t ngroups) {
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
  if (bias) y = y + bias[cell % n];
  c[cell] = store_word(y);
}

// ---------------------------------------------------------------------------
// Skinny-M product (decode GEMV), OP_NN: X[M x K] . W[K x N], M <= 16.
//
// Work is split into tasks: (block of 256 output columns, one k-leaf).  A persistent grid of
// 256-thread workgroups walks its tasks leaf chunk by leaf chunk through one continuous
// pipeline: the 256 threads stream the next chunk of W (R rows x 256 columns, 16-byte loads,
// 32 KB) and of x into registers while the current chunk's chains run out of LDS, so HBM sees
// a steady stream regardless of how the serial chains are owned.  Thread c runs the chain of
// column c: a VALU FMA per step under MODE.FP_DENORM = 2 (v_fma_f32 is fma(ftz a, ftz b,
// ftz acc), like the K=1 MFMA), for all M rows.  A finished leaf partial is published with
// agent-scope atomic stores (device coherent, so no cache writeback is needed: the stores only
// have to be complete before the count), counted on its column block's counter, and the task
// that completes a block folds its P partials with the contract's tree, writes the output and
// resets the counter.  One launch computes the whole product.
constexpr int GV_THREADS = 256;
constexpr int GV_COLS = 256;                // columns per task: one per thread
constexpr int GV_MAXM = 16;
constexpr int GV_CHUNK = 32768;             // bytes of W per LDS buffer
constexpr int GV_FOLD_BATCH = 32;           // partial loads in flight while folding

template <int T>
struct GvElem {
  static constexpr int bytes = T == T_F32 ? 4 : (T == T_BF16 ? 2 : 1);
  static constexpr int rows = GV_CHUNK / (GV_COLS * bytes);  // rows per chunk: 128 / 64 / 32
};

struct GemvArgs {
  float* c;
  const float* x;
  const void* w;
  const float* scales;
  const float* bias;
  float* ws;              // [nleaves][m][n] leaf partials when nleaves > 1
  unsigned int* counter;  // [column blocks], zero between launches
  int64_t m, n, k, leaf, nleaves;
  int64_t ncb;            // column blocks
  int64_t ntasks;         // ncb * nleaves
  int chunks;             // chunks per leaf: ceil(leaf / rows)
};

// Issue every global read of one chunk into registers; `store` writes them to LDS.  A
// segment no chain step reads (a row outside the leaf, columns past n) is read from the
// operand's first bytes instead -- an in-bounds address -- so the loads carry no branch and
// are all in flight together; those LDS bytes only reach cells that are never stored.
template <int T, int MR, bool VEC>
struct GvStager {
  static constexpr int EB = GvElem<T>::bytes;
  static constexpr int R = GvElem<T>::rows;
  static constexpr int SEGS = GV_COLS * EB / 16;           // 16-byte segments per row
  static constexpr int PER = R * SEGS / GV_THREADS;        // segments per thread: 8
  static constexpr int XPER = (R * MR + GV_THREADS - 1) / GV_THREADS;
  u4 wv[PER];
  float xv[XPER];

  __device__ __forceinline__ void load(const GemvArgs& g, int64_t j0, int64_t t, int ch, int tid) {
    const char* wb = static_cast<const char*>(g.w);
    const int64_t kb = t * g.leaf + (int64_t)ch * R;
    int64_t kend = (t + 1) * g.leaf;
    if (kend > g.k) kend = g.k;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int q = tid + i * GV_THREADS;
      const int rr = q / SEGS;
      const int sg = q % SEGS;
      const int64_t kk = kb + rr;
      const int64_t col = j0 + (int64_t)sg * (16 / EB);
      if constexpr (VEC) {
        const bool ok = kk < kend && col < g.n;
        wv[i] = *reinterpret_cast<const u4*>(ok ? wb + (kk * g.n + col) * EB : wb);
      } else {
        u4 v = {0u, 0u, 0u, 0u};
        if (kk < kend) {
          const char* src = wb + (kk * g.n + col) * EB;
          char* d = reinterpret_cast<char*>(&v);
#pragma unroll
          for (int e = 0; e < 16 / EB; ++e)
            if (col + e < g.n) {
              if constexpr (EB == 4) reinterpret_cast<float*>(d)[e] = reinterpret_cast<const float*>(src)[e];
              else if constexpr (EB == 2) reinterpret_cast<uint16_t*>(d)[e] = reinterpret_cast<const uint16_t*>(src)[e];
              else d[e] = src[e];
            }
        }
        wv[i] = v;
      }
    }
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
      const int q = tid + i * GV_THREADS;
      const int rr = q / MR;
      const int r = q % MR;
      const int64_t kk = kb + rr;
      const bool ok = q < R * MR && kk < kend && r < g.m;
      xv[i] = *(ok ? g.x + r * g.k + kk : g.x);  // rows past m feed cells that are never stored
    }
  }

  __device__ __forceinline__ void store(char* buf, float* xbuf, int tid) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int q = tid + i * GV_THREADS;
      *reinterpret_cast<u4*>(buf + (q / SEGS) * GV_COLS * EB + (q % SEGS) * 16) = wv[i];
    }
#pragma unroll
    for (int i = 0; i < XPER; ++i) {
      const int q = tid + i * GV_THREADS;
      if (q < R * MR) xbuf[q] = xv[i];
    }
  }
};

// The contract's tree over a cell's P leaf partials ws[t * stride], read with agent-scope
// atomic loads issued GV_FOLD_BATCH at a time.
__device__ __forceinline__ float fold_partials(const float* base, int64_t P, int64_t stride) {
  StackF stk;
  int64_t t = 0;
  float last = 0.f;
  for (int64_t t0 = 0; t0 < P; t0 += GV_FOLD_BATCH) {
    float v[GV_FOLD_BATCH];
#pragma unroll
    for (int e = 0; e < GV_FOLD_BATCH; ++e) {
      const int64_t tt = t0 + e < P ? t0 + e : P - 1;
      v[e] = __hip_atomic_load(base + tt * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
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

// The task that completed column block `cb`: fold each cell's P partials, write the output,
// reset the block's counter.
template <int MR>
__device__ __forceinline__ void gv_finish(const GemvArgs& g, int64_t cb, int tid) {
  const int64_t col = cb * GV_COLS + tid;
  if (col < g.n) {
    const int64_t stride = g.m * g.n;
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      if (r >= g.m) continue;
      float y = fold_partials(g.ws + r * g.n + col, g.nleaves, stride);
      if (g.bias) y = y + g.bias[col];
      g.c[r * g.n + col] = store_word(y);
    }
  }
  if (tid == 0) __hip_atomic_store(&g.counter[cb], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int BT, int MR, bool VEC>
__global__ void __launch_bounds__(GV_THREADS) gemv_nn_kernel(GemvArgs g) {
  constexpr int EB = GvElem<BT>::bytes;
  constexpr int R = GvElem<BT>::rows;
  __shared__ __attribute__((aligned(16))) char wbuf[2][GV_CHUNK];
  __shared__ __attribute__((aligned(16))) float xbuf[2][R * MR];
  __shared__ unsigned int last_flag;
  set_flush_inputs_mode();
  const int tid = threadIdx.x;

  // this workgroup's items: (task, chunk), task = blockIdx.x + i * gridDim.x, leaf-major
  // tasks (consecutive tasks are neighbouring column blocks of one leaf)
  const int64_t my_tasks = g.ntasks > blockIdx.x ? (g.ntasks - 1 - blockIdx.x) / gridDim.x + 1 : 0;
  const int64_t items = my_tasks * g.chunks;
  if (items == 0) return;  // uniform

  GvStager<BT, MR, VEC> st;
  auto task_of = [&](int64_t it) { return (int64_t)blockIdx.x + (it / g.chunks) * (int64_t)gridDim.x; };
  {
    const int64_t task = task_of(0);
    st.load(g, (task % g.ncb) * GV_COLS, task / g.ncb, 0, tid);
    st.store(wbuf[0], xbuf[0], tid);
  }
  __syncthreads();

  float acc[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) acc[r] = 0.f;
  int64_t pending_cb = -1;        // column block of this workgroup's last counted task
  unsigned int pending_prev = 0;  // (thread 0) the count before that task's increment

  for (int64_t it = 0; it < items; ++it) {
    const int64_t task = task_of(it);
    const int ch = (int)(it % g.chunks);
    const int64_t cb = task % g.ncb;
    const int64_t t = task / g.ncb;
    const int64_t col = cb * GV_COLS + tid;
    if (it + 1 < items) {
      const int64_t nt = task_of(it + 1);
      st.load(g, (nt % g.ncb) * GV_COLS, nt / g.ncb, (int)((it + 1) % g.chunks), tid);
    }
    // this chunk's chain steps
    int64_t kend = (t + 1) * g.leaf;
    if (kend > g.k) kend = g.k;
    int s_end = (int)(kend - (t * g.leaf + (int64_t)ch * R));
    if (s_end > R) s_end = R;
    const char* cur = wbuf[it & 1] + tid * EB;
    const float* xc = xbuf[it & 1];
    const float sc = (BT == T_I8 && col < g.n) ? g.scales[col] : 0.f;
    for (int s = 0; s < s_end; ++s) {
      float wv;
      if constexpr (BT == T_F32) wv = reinterpret_cast<const float*>(cur)[s * GV_COLS];
      else if constexpr (BT == T_BF16)
        wv = __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(cur)[s * GV_COLS] << 16);
      else wv = (float)(int32_t)reinterpret_cast<const int8_t*>(cur)[s * GV_COLS] * sc;
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[r] = __builtin_fmaf(xc[s * MR + r], wv, acc[r]);
    }
    if (ch + 1 == g.chunks) {
      // the leaf is complete: acc is its partial
      const bool live = col < g.n;
      if (g.nleaves == 1) {
        if (live) {
          const float bj = g.bias ? g.bias[col] : 0.f;
#pragma unroll
          for (int r = 0; r < MR; ++r)
            if (r < g.m) g.c[r * g.n + col] = store_word(g.bias ? acc[r] + bj : acc[r]);
        }
      } else {
        if (live) {
#pragma unroll
          for (int r = 0; r < MR; ++r)
            if (r < g.m)
              __hip_atomic_store(&g.ws[(t * g.m + r) * g.n + col], acc[r], __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
        }
        // the agent-scope stores above are complete (device coherent) before the count
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
        // the count of the previous completed task has long returned: act on it now
        if (tid == 0) last_flag = pending_prev + 1 == (unsigned int)g.nleaves ? 1u : 0u;
        __syncthreads();
        if (pending_cb >= 0 && last_flag) gv_finish<MR>(g, pending_cb, tid);
        if (tid == 0)
          pending_prev = __hip_atomic_fetch_add(&g.counter[cb], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        pending_cb = cb;
      }
#pragma unroll
      for (int r = 0; r < MR; ++r) acc[r] = 0.f;
    }
    if (it + 1 < items) st.store(wbuf[(it + 1) & 1], xbuf[(it + 1) & 1], tid);
    __syncthreads();
  }
  if (pending_cb >= 0) {
    if (tid == 0) last_flag = pending_prev + 1 == (unsigned int)g.nleaves ? 1u : 0u;
    __syncthreads();
    if (last_flag) gv_finish<MR>(g, pending_cb, tid);
  }
}

// ---------------------------------------------------------------------------
// host side

static bool aligned(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }
static int elem_bytes(int t) { return t == T_F32 ? 4 : (t == T_BF16 ? 2 : 1); }

static int pick_group(int64_t nleaves, int64_t tiles, int num_cus) {
  // Largest power-of-two group <= 32 leaves; split further (aligned subtrees) while the
  // grid is smaller than two workgroups per CU and groups still hold >= 4 leaves.
  int64_t gsz = 32;
  while (gsz > 1 && gsz / 2 >= nleaves) gsz /= 2;
  auto groups = [&](int64_t s) { return (nleaves + s - 1) / s; };
  while (gsz > 4 && tiles * groups(gsz) < 2 * (int64_t)num_cus) gsz /= 2;
  return (int)gsz;
}

// The skinny-M path takes OP_NN products with at most GV_MAXM float32 rows.
static bool use_gemv(const GemmProblem& p) {
  return p.op == OP_NN && p.a_type == T_F32 && p.m >= 1 && p.m <= GV_MAXM;
}

int64_t gemm_workspace_floats(const GemmProblem& p, int num_cus) {
  const int64_t L = p.leaf > 0 ? p.leaf : leaf_size(p.k);
  const int64_t P = leaf_count(p.k, L);
  if (P <= 1 || p.m <= 0 || p.n <= 0) return 0;
  if (use_gemv(p)) return P > 1 ? P * p.m * p.n : 0;
  const int64_t tiles = ((p.m + BM - 1) / BM) * ((p.n + BN - 1) / BN);
  const int64_t gsz = pick_group(P, tiles, num_cus);
  const int64_t ng = (P + gsz - 1) / gsz;
  return ng > 1 ? ng * p.m * p.n : 0;
}

int64_t gemm_counter_count(const GemmProblem& p) {
  const int64_t L = p.leaf > 0 ? p.leaf : leaf_size(p.k);
  const int64_t P = leaf_count(p.k, L);
  if (!use_gemv(p) || p.n <= 0 || P <= 1) return 0;
  return (p.n + GV_COLS - 1) / GV_COLS;
}

template <int BT, int MR>
static hipError_t launch_gemv_mr(const GemvArgs& g, bool vec, dim3 grid, hipStream_t s) {
  if (vec) hipLaunchKernelGGL((gemv_nn_kernel<BT, MR, true>), grid, dim3(GV_THREADS), 0, s, g);
  else hipLaunchKernelGGL((gemv_nn_kernel<BT, MR, false>), grid, dim3(GV_THREADS), 0, s, g);
  return hipGetLastError();
}

template <int BT>
static hipError_t launch_gemv_m(const GemvArgs& g, int64_t m, bool vec, dim3 grid, hipStream_t s) {
  if (m <= 1) return launch_gemv_mr<BT, 1>(g, vec, grid, s);
  if (m <= 2) return launch_gemv_mr<BT, 2>(g, vec, grid, s);
  if (m <= 4) return launch_gemv_mr<BT, 4>(g, vec, grid, s);
  if (m <= 8) return launch_gemv_mr<BT, 8>(g, vec, grid, s);
  return launch_gemv_mr<BT, 16>(g, vec, grid, s);
}

static hipError_t launch_gemv_bt(const GemvArgs& g, int bt, int64_t m, bool vec, dim3 grid, hipStream_t s) {
  if (bt == T_F32) return launch_gemv_m<T_F32>(g, m, vec, grid, s);
  if (bt == T_BF16) return launch_gemv_m<T_BF16>(g, m, vec, grid, s);
  return launch_gemv_m<T_I8>(g, m, vec, grid, s);
}

template <int OP, int AT, int BT>
static hipError_t launch_gemm(const GemmArgs& g, dim3 grid, hipStream_t stream) {
  hipLaunchKernelGGL((gemm_mfma_kernel<OP, AT, BT>), grid, dim3(NTHREADS), 0, stream, g);
  return hipGetLastError();
}

template <int OP>
static hipError_t launch_gemm_types(const GemmArgs& g, int at, int bt, dim3 grid, hipStream_t s) {
  if (at == T_F32) {
    if (bt == T_F32) return launch_gemm<OP, T_F32, T_F32>(g, grid, s);
    if (bt == T_BF16) return launch_gemm<OP, T_F32, T_BF16>(g, grid, s);
    return launch_gemm<OP, T_F32, T_I8>(g, grid, s);
  }
  if (bt == T_BF16) return launch_gemm<OP, T_BF16, T_BF16>(g, grid, s);
  return hipErrorInvalidValue;
}


hipError_t run_gemm(const GemmProblem& p, float* ws, unsigned int* counters, int num_cus,
                    hipStream_t stream) {
  if (p.m <= 0 || p.n <= 0) return hipSuccess;
  const int64_t L = p.leaf > 0 ? p.leaf : leaf_size(p.k);
  const int64_t P = leaf_count(p.k, L);
  if (P == 0) {
    const int64_t cells = p.m * p.n;
    hipLaunchKernelGGL(fold_groups_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0,
                       stream, p.c, (const float*)nullptr, p.bias, p.m, p.n, (int64_t)0);
    return hipGetLastError();
  }
  if (use_gemv(p)) {
    GemvArgs v;
    v.c = p.c; v.x = static_cast<const float*>(p.a); v.w = p.b; v.scales = p.scales; v.bias = p.bias;
    v.ws = ws; v.counter = counters;
    v.m = p.m; v.n = p.n; v.k = p.k; v.leaf = L; v.nleaves = P;
    if (P > 1 && (ws == nullptr || counters == nullptr)) return hipErrorInvalidValue;
    const int eb = elem_bytes(p.b_type);
    const int rows = GV_CHUNK / (GV_COLS * eb);
    v.chunks = (int)((L + rows - 1) / rows);
    v.ncb = (p.n + GV_COLS - 1) / GV_COLS;
    v.ntasks = v.ncb * P;
    const bool vec = ((p.n * eb) % 16 == 0) && aligned(p.b, 16);
    // persistent grid: as many 256-thread workgroups as are resident at once (LDS: 64 KB of W
    // buffers plus x's two buffers each, two per CU while that fits in 160 KB)
    const int64_t lds = 2 * (int64_t)GV_CHUNK + 2 * (int64_t)rows * (p.m <= 1 ? 1 : p.m <= 2 ? 2 : p.m <= 4 ? 4 : p.m <= 8 ? 8 : 16) * 4;
    int64_t grid = (lds * 2 <= 160 * 1024 ? 2 : 1) * (int64_t)num_cus;
    if (grid > v.ntasks) grid = v.ntasks;
    return launch_gemv_bt(v, p.b_type, p.m, vec, dim3((unsigned)grid), stream);
  }
  GemmArgs g;
  g.c = p.c; g.a = p.a; g.b = p.b; g.scales = p.scales; g.bias = p.bias; g.ws = ws;
  g.m = p.m; g.n = p.n; g.k = p.k; g.leaf = L; g.nleaves = P;
  if (p.op == OP_TN) { g.a_rows = p.k; g.a_cols = p.m; } else { g.a_rows = p.m; g.a_cols = p.k; }
  if (p.op == OP_NT) { g.b_rows = p.n; g.b_cols = p.k; } else { g.b_rows = p.k; g.b_cols = p.n; }
  const int ea = elem_bytes(p.a_type), eb = elem_bytes(p.b_type);
  g.a_vec = (g.a_cols % 4 == 0) && aligned(p.a, 4 * ea);
  g.b_vec = (g.b_cols % 4 == 0) && aligned(p.b, 4 * eb);
  const int64_t tm = (p.m + BM - 1) / BM, tn = (p.n + BN - 1) / BN;
  g.tiles_n = (int)tn;
  const int64_t gsz = P > 1 ? pick_group(P, tm * tn, num_cus) : 1;
  g.group = gsz;
  g.ngroups = (P + gsz - 1) / gsz;
  if (g.ngroups > 1 && ws == nullptr) return hipErrorInvalidValue;
  dim3 grid((unsigned)(tm * tn), (unsigned)g.ngroups);
  hipError_t e;
  if (p.op == OP_NN) e = launch_gemm_types<OP_NN>(g, p.a_type, p.b_type, grid, stream);
  else if (p.op == OP_NT) e = launch_gemm_types<OP_NT>(g, p.a_type, p.b_type, grid, stream);
  else e = launch_gemm_types<OP_TN>(g, p.a_type, p.b_type, grid, stream);
  if (e != hipSuccess || g.ngroups == 1) return e;
  const int64_t cells = p.m * p.n;
  hipLaunchKernelGGL(fold_groups_kernel, dim3((unsigned)((cells + 255) / 256)), dim3(256), 0, stream,
                     p.c, (const float*)ws, p.bias, p.m, p.n, g.ngroups);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// bf16 conversions (gemm/IDENTICAL_LOWBIT_CONTRACT.md L-1, L-2; checks/numerics.mojo:1548-1574)

__global__ void bf16_widen_kernel(float* out, const uint16_t* in, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) out[i] = __uint_as_float((uint32_t)in[i] << 16);
}

__global__ void bf16_narrow_kernel(uint16_t* out, const float* in, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  uint32_t b = __float_as_uint(in[i]);
  if ((b & 0x7F800000u) == 0u) b &= 0x80000000u;  // ftz first
  if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0u) {
    out[i] = (uint16_t)((b >> 16) | 0x0040u);  // NaN stays a quiet NaN
    return;
  }
  const uint32_t lsb = (b >> 16) & 1u;
  out[i] = (uint16_t)((b + 0x7FFFu + lsb) >> 16);
}

hipError_t run_bf16_widen(float* out, const uint16_t* in, int64_t count, hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(bf16_widen_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream,
                     out, in, count);
  return hipGetLastError();
}

hipError_t run_bf16_narrow(uint16_t* out, const float* in, int64_t count, hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(bf16_narrow_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream,
                     out, in, count);
  return hipGetLastError();
}

}  // namespace mlg

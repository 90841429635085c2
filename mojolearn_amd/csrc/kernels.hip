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
// wave owns 64 rows x 32 columns = one v_mfma_f32_32x32x1_2b_f32 per k step (block 0 =
// rows 0-31, block 1 = rows 32-63, both against the same 32 columns).  K is staged
// through LDS in KT = 32-step slices, three buffers (loads issued two slices ahead).  Operands travel global -> LDS
// with global_load_lds_dwordx4 (16 bytes per lane, straight into LDS, no registers) in
// their stored element type; bf16 widening and int8 x column-scale dequantisation
// happen when a lane reads its MFMA operand out of LDS.
constexpr int NTHREADS = 512;
constexpr int NWAVES = NTHREADS / 64;
constexpr int BM = 128;
constexpr int BN = 128;
constexpr int KT = 32;
constexpr int SLICE_BYTES = BM * KT * 4;  // one operand slice at float32: 16 KB
constexpr int NBUF = 3;                   // slices in LDS: loads run two slices ahead
constexpr int MAX_GROUP_LEAVES = 32;      // one group's leaves fold in registers + one LDS slot

typedef __attribute__((address_space(3))) void* lds_vptr;
typedef __attribute__((address_space(1))) void* gbl_vptr;

template <int T>
struct Elem {
  static constexpr int bytes = T == T_F32 ? 4 : (T == T_BF16 ? 2 : 1);
  static constexpr int per16 = 16 / bytes;  // elements per 16-byte chunk
};

// One staged slice (BM indices x KT steps) of an operand of element type T, as
// NCH = BM*KT*bytes/16 chunks of 16 bytes, chunk position p loaded by lane p % 64 of
// load instruction p / 64 (a load instruction fills 1 KB of LDS, lane L at L*16).
//  * index-major (the operand stores k contiguously: A in NN/NT, B in NT): index r owns
//    CR = KT*bytes/16 chunks; its chunk c sits at position r*CR + (c ^ swz(r)), so the
//    lanes of one read (consecutive r, same c) land in different banks.
//  * k-major (the operand stores indices contiguously: B in NN/TN, A in TN): step s owns
//    RC = BM*bytes/16 chunks holding the BM indices in order.
template <int T, bool IMAJ>
struct Slice {
  static constexpr int EB = Elem<T>::bytes;
  static constexpr int CE = Elem<T>::per16;
  static constexpr int NCH = BM * KT * EB / 16;  // 1024 / 512 / 256
  static constexpr int NI = NCH / 64;            // load instructions per slice: 16 / 8 / 4
  static constexpr int CR = KT * EB / 16;        // 8 / 4 / 2
  static constexpr int RC = BM * EB / 16;        // 32 / 16 / 8
  static constexpr int PER_WAVE = (NI + NWAVES - 1) / NWAVES;

  __device__ static __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & (CR - 1); }

  // Chunk position p -> (index offset, step offset) of its first element.
  __device__ static __forceinline__ void coords(int p, int& di, int& dk) {
    if constexpr (IMAJ) {
      const int r = p / CR;
      di = r;
      dk = ((p % CR) ^ swz(r)) * CE;
    } else {
      di = (p % RC) * CE;
      dk = p / RC;
    }
  }
};

// Word 3 of a raw buffer resource on gfx9-family targets (32-bit data format, no swizzle).
constexpr int RSRC_WORD3 = 0x00020000;

// The global side of one operand: this lane's share of every slice's load instructions, as
// buffer loads straight into LDS.  Load instruction q of a slice covers RPI consecutive
// stored rows; its scalar resource starts at the first of them and ends at the operand's
// end, and the lane's byte offset within it is fixed for the whole k loop.  A chunk past
// the operand's end reads as zeros (the resource's record bound); a chunk past a row's
// end reads the next row's bytes.  Neither reaches a stored cell: indices past m or n are
// never stored, steps past k are never executed.  The host keeps RPI * pitch * bytes
// below 2^31.
template <int T, bool IMAJ>
struct DirectLoader {
  using S = Slice<T, IMAJ>;
  static constexpr int RPI = IMAJ ? 64 / S::CR : 64 / S::RC;  // stored rows per instruction
  uint32_t voff[S::PER_WAVE];

  __device__ __forceinline__ void init(int64_t pitch, int wave, int lane) {
#pragma unroll
    for (int h = 0; h < S::PER_WAVE; ++h) {
      const int q = (wave + NWAVES * h) % S::NI;
      int di, dk;
      S::coords(q * 64 + lane, di, dk);
      if constexpr (IMAJ) voff[h] = (uint32_t)(((di - q * RPI) * pitch + dk) * S::EB);
      else voff[h] = (uint32_t)(((dk - q * RPI) * pitch + di) * S::EB);
    }
  }

  // Issue this wave's PER_WAVE loads of the slice that starts at step k0 into `slice` (when
  // a slice has fewer load instructions than waves, the extra waves repeat an earlier
  // wave's chunk -- the same bytes to the same place -- so every wave issues the same
  // count and can wait on it with one vmcnt).  `wave` must be wave-uniform.
  __device__ __forceinline__ void issue(char* slice, const void* base, int64_t total_bytes, int64_t pitch,
                                        int64_t idx0, int64_t k0, int wave) const {
#pragma unroll
    for (int h = 0; h < S::PER_WAVE; ++h) {
      const int q = (wave + NWAVES * h) % S::NI;
      const int64_t off = IMAJ ? ((idx0 + q * RPI) * pitch + k0) * S::EB : ((k0 + q * RPI) * pitch + idx0) * S::EB;
      const int64_t rem = total_bytes - off;
      const int nrec = rem <= 0 ? 0 : (rem > 0x7FFFFFFF ? 0x7FFFFFFF : (int)rem);
      const char* first = static_cast<const char*>(base) + (rem > 0 ? off : 0);
      const __amdgpu_buffer_rsrc_t rs =
          __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(first), (short)0, nrec, RSRC_WORD3);
#if defined(__HIP_DEVICE_COMPILE__)
      // (the host pass compiles kernel bodies only for their launch stubs; with this builtin
      // in a kernel template it drops the stubs of every instantiation after the first)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_vptr)(slice + q * 1024), 16, voff[h], 0, 0, 0);
#else
      (void)rs;
#endif
    }
  }
};

// A workgroup barrier for LDS hand-off only: no wait on this wave's outstanding global
// loads (the k loop waits for exactly the slice it needs), a compiler fence on each side.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// A lane's MFMA operand values for steps s .. s+3 of a staged slice, as float32: index
// `idx` of the slice.  bf16 widens exactly (bits << 16); int8 is f32(code) * scale, one
// rounding, the scale flushed on input by MODE.FP_DENORM = 2 (and the product by the
// MFMA's input flush), i.e. ftz(f32(code) * ftz(scale)).
template <int T, bool IMAJ>
__device__ __forceinline__ f4 read4(const char* slice, int idx, int s, float scale) {
  using S = Slice<T, IMAJ>;
  f4 v;
  if constexpr (IMAJ) {
    const int c = s * S::EB / 16;              // chunk holding step s
    const int sub = (s * S::EB) % 16;          // byte offset of step s in it
    const char* p = slice + (idx * S::CR + (c ^ S::swz(idx))) * 16 + sub;
    if constexpr (T == T_F32) {
      v = *reinterpret_cast<const f4*>(p);
    } else if constexpr (T == T_BF16) {
      const uint2 u = *reinterpret_cast<const uint2*>(p);
      v[0] = __uint_as_float(u.x << 16); v[1] = __uint_as_float(u.x & 0xFFFF0000u);
      v[2] = __uint_as_float(u.y << 16); v[3] = __uint_as_float(u.y & 0xFFFF0000u);
    } else {
      const uint32_t u = *reinterpret_cast<const uint32_t*>(p);
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = (float)(int32_t)(int8_t)(u >> (8 * e)) * scale;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const char* p = slice + ((s + e) * BM + idx) * S::EB;
      if constexpr (T == T_F32) v[e] = *reinterpret_cast<const float*>(p);
      else if constexpr (T == T_BF16) v[e] = __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
      else v[e] = (float)*reinterpret_cast<const int8_t*>(p) * scale;
    }
  }
  return v;
}

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
  int tiles_n;
};

// MFMA steps s0 .. s1-1 of one staged slice, in ascending order.  The slice is walked in
// aligned groups of 4 steps whose operands are read from LDS one group ahead; unless FULL,
// a step outside [s0, s1) is skipped by a uniform branch.  The scheduling fences keep the
// compiler from hoisting every LDS read of the slice, which would not fit beside the
// accumulator and the fold slots.
template <int OP, int AT, int BT, bool FULL>
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
    for (int q = 0; q < 4; ++q)
      if (FULL || (s + q >= s0 && s + q < s1)) acc = __builtin_amdgcn_mfma_f32_32x32x1f32(a4[q], b4[q], acc, 0, 0, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (s + 4 < KT) { a4 = an; b4 = bn; }
  }
}

template <int OP, int AT, int BT>
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
  static_assert(NBUF == 3, "the slice loop is unrolled by NBUF");
  for (int64_t kt = kt_first; kt <= kt_last;) {
    MLG_SLICE_STEP(lds0, lds2);
    if (++kt > kt_last) break;
    MLG_SLICE_STEP(lds1, lds0);
    if (++kt > kt_last) break;
    MLG_SLICE_STEP(lds2, lds1);
    ++kt;
  }
#undef MLG_SLICE_STEP
  // no load into LDS may outlive the workgroup
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)

  // acc holds the group root.  Element e -> block b = e/16, row (e%4) + 8*((e%16)/4) + 4*(lane/32) within it.
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

// Copy a stored operand [rows][cols] of `eb`-byte elements into [rows][pitch] (pitch a
// multiple of 16 bytes, zero padding), so that the product kernel's 16-byte loads are
// aligned and never straddle a row end.
__global__ void repack_rows_kernel(char* dst, const char* src, int64_t rows, int64_t cols, int64_t pitch,
                                   int eb) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * pitch) return;
  const int64_t r = i / pitch, cidx = i % pitch;
  if (eb == 4) {
    reinterpret_cast<uint32_t*>(dst)[i] = cidx < cols ? reinterpret_cast<const uint32_t*>(src)[r * cols + cidx] : 0u;
  } else if (eb == 2) {
    reinterpret_cast<uint16_t*>(dst)[i] = cidx < cols ? reinterpret_cast<const uint16_t*>(src)[r * cols + cidx] : (uint16_t)0;
  } else {
    dst[i] = cidx < cols ? src[r * cols + cidx] : (char)0;
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
// A wave owns one k-leaf of one column group.  Each lane owns CPL = 4 / bytes consecutive
// columns: one 32-bit word of W per k row (4 int8 codes, 2 bf16 or 1 float32), so the 64
// lanes read 256 contiguous bytes of every W row.  The leaf's rows stream into registers
// GV_CH at a time, two buffers requested before the first arithmetic (a whole 128-row leaf
// is in flight at once), and each lane runs CPL x M serial chains in VALU (v_fma_f32 under
// MODE.FP_DENORM = 2 is fma(ftz a, ftz b, ftz acc), like the K=1 MFMA).  x is the same for
// every lane and is read with uniform loads.  A 256-thread workgroup is one column group's
// aligned group of GV_LEAVES leaves -- a subtree of the fold -- whose root it forms through
// LDS.  With more than one group, the roots go to the workspace with agent-scope atomic
// stores and are counted on the column group's counter; the workgroup that completes the
// count folds them (the rest of the contract's tree), writes the output and resets the
// counter.  One launch computes the whole product.
constexpr int GV_THREADS = 256;
constexpr int GV_LEAVES = GV_THREADS / 64;  // leaves per workgroup: an aligned subtree
constexpr int GV_MAXM = 16;
constexpr int GV_CH = 128;                  // W rows per register buffer: a whole contract leaf
constexpr int GV_FOLD_BATCH = 32;           // root loads in flight while folding
constexpr int GV_FEW_GROUPS = 8;            // up to this many groups: all roots loaded at once

template <int T>
struct GvCols {
  static constexpr int cpl = 4 / Elem<T>::bytes;  // columns per lane
  static constexpr int cols = 64 * cpl;           // columns per group
};

struct GemvArgs {
  float* c;
  const void* w;
  const float* scales;
  const float* bias;
  float* ws;              // [ngroups][m][n] group roots when ngroups > 1
  unsigned int* counter;  // [ncg], zero between launches (ngroups > 1)
  int64_t m, n, k, leaf, nleaves;
  int64_t ngroups;        // ceil(nleaves / GV_LEAVES)
  int64_t ncg;            // column groups
};

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
// `wleaf` is the leaf's first row; rows are `rowbytes` apart (GV_CH * rowbytes < 2^31).
constexpr int GV_RB = 16;
constexpr int GV_AHEAD = 3;

template <int BT>
__device__ __forceinline__ void gv_weights(uint32_t u, const float (&sc)[GvCols<BT>::cpl], float (&wv)[GvCols<BT>::cpl]) {
  if constexpr (BT == T_F32) {
    wv[0] = __uint_as_float(u);
  } else if constexpr (BT == T_BF16) {
    wv[0] = __uint_as_float(u << 16);
    wv[1] = __uint_as_float(u & 0xFFFF0000u);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) wv[e] = (float)((int32_t)(u << (24 - 8 * e)) >> 24) * sc[e];
  }
}

template <int BT, int MR>
__device__ __forceinline__ void gv_leaf_full(float (&acc)[MR][GvCols<BT>::cpl], const char* wleaf, uint32_t loff,
                                             int rowbytes, const float* __restrict__ xl, int64_t k, int m,
                                             const float (&sc)[GvCols<BT>::cpl]) {
  constexpr int CPL = GvCols<BT>::cpl;
  constexpr int NBLK = GV_CH / GV_RB;
  constexpr int RING = GV_AHEAD + 1;
  constexpr int XB = MR <= 2 ? 16 : 32 / MR;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(wleaf), (short)0, 0x7FFFFFFF, RSRC_WORD3);
  const float* xr[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r) xr[r] = xl + (r < m ? r : m - 1) * k;  // rows past m: never stored

  uint32_t ring[RING][GV_RB];
#pragma unroll
  for (int b = 0; b < GV_AHEAD; ++b)
#pragma unroll
    for (int i = 0; i < GV_RB; ++i)
      ring[b][i] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)loff, (b * GV_RB + i) * rowbytes, 0);
  float xc[MR][XB], xn[MR][XB];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int q = 0; q < XB; ++q) xc[r][q] = xr[r][q];

#pragma unroll
  for (int b = 0; b < NBLK; ++b) {
    if (b + GV_AHEAD < NBLK) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < GV_RB; ++i)
        ring[(b + GV_AHEAD) % RING][i] =
            __builtin_amdgcn_raw_buffer_load_b32(rs, (int)loff, ((b + GV_AHEAD) * GV_RB + i) * rowbytes, 0);
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
        gv_weights<BT>(ring[b % RING][q0 + q], sc, wv);
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

template <int BT, int MR, bool VEC, bool FULLLEAF>
__global__ void __launch_bounds__(GV_THREADS) gemv_nn_kernel(GemvArgs g, const float* __restrict__ x) {
  constexpr int CPL = GvCols<BT>::cpl;
  constexpr int COLS = GvCols<BT>::cols;
  constexpr int EB = Elem<BT>::bytes;
  __shared__ float part[GV_LEAVES][MR][COLS];
  __shared__ unsigned int last_flag;

  set_flush_inputs_mode();

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: leaf and k range too
  const int64_t cg = blockIdx.x % g.ncg;
  const int64_t grp = blockIdx.x / g.ncg;
  const int64_t t = grp * GV_LEAVES + wave;  // this wave's leaf
  const int m = (int)g.m;

  float acc[MR][CPL];
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int e = 0; e < CPL; ++e) acc[r][e] = 0.f;

  if (t < g.nleaves) {
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

  // The group's root: the tree over its (up to GV_LEAVES) leaf partials, through LDS.
#pragma unroll
  for (int r = 0; r < MR; ++r)
#pragma unroll
    for (int e = 0; e < CPL; ++e) part[wave][r][lane * CPL + e] = acc[r][e];
  __syncthreads();
  const int64_t left = g.nleaves - grp * GV_LEAVES;
  const int cnt = left < GV_LEAVES ? (int)left : GV_LEAVES;
  for (int cell = tid; cell < MR * COLS; cell += GV_THREADS) {
    const int r = cell / COLS, col = cell % COLS;
    const int64_t j = cg * COLS + col;
    if (r >= m || j >= g.n) continue;
    float y = part[0][r][col];
    if (cnt >= 2) y = y + part[1][r][col];           // leaves 0,1 paired
    if (cnt == 3) y = y + part[2][r][col];           // leaf 2 carried, then joined
    if (cnt == 4) y = y + (part[2][r][col] + part[3][r][col]);
    if (g.ngroups == 1) {
      if (g.bias) y = y + g.bias[j];  // ftz(C) + ftz(b) by the input flush
      g.c[r * g.n + j] = store_word(y);
    } else {
      __hip_atomic_store(&g.ws[(grp * g.m + r) * g.n + j], y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if (g.ngroups == 1) return;

  // Count this group's roots in; the workgroup that completes the count folds.  The roots
  // are device-coherent stores, complete (vmcnt) before the count is published.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  __syncthreads();
  if (tid == 0) {
    const unsigned int prev = __hip_atomic_fetch_add(&g.counter[cg], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev + 1 == (unsigned int)g.ngroups ? 1u : 0u;
  }
  __syncthreads();
  if (!last_flag) return;
  const int64_t stride = g.m * g.n;
  constexpr int CPT = (MR * COLS + GV_THREADS - 1) / GV_THREADS;  // cells per thread
  if (g.ngroups <= GV_FEW_GROUPS) {
    // every root of every cell of this thread requested at once, then folded
    float v[CPT][GV_FEW_GROUPS];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int cell = tid + c * GV_THREADS;
      const int r = cell / COLS, col = cell % COLS;
      const int64_t j = cg * COLS + col;
      if (cell >= MR * COLS || r >= m || j >= g.n) continue;
#pragma unroll
      for (int e = 0; e < GV_FEW_GROUPS; ++e)
        if (e < g.ngroups)
          v[c][e] = __hip_atomic_load(g.ws + (e * g.m + r) * g.n + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int cell = tid + c * GV_THREADS;
      const int r = cell / COLS, col = cell % COLS;
      const int64_t j = cg * COLS + col;
      if (cell >= MR * COLS || r >= m || j >= g.n) continue;
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
  } else {
    for (int cell = tid; cell < MR * COLS; cell += GV_THREADS) {
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

// ---------------------------------------------------------------------------
// host side

static bool aligned(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }
static int elem_bytes(int t) { return t == T_F32 ? 4 : (t == T_BF16 ? 2 : 1); }

static int pick_group(int64_t nleaves, int64_t tiles, int num_cus) {
  // Largest power-of-two group <= 32 leaves; split further (aligned subtrees) while the
  // grid has fewer workgroups than CUs (one 160 KB workgroup fits a CU).
  int64_t gsz = 32;
  while (gsz > 1 && gsz / 2 >= nleaves) gsz /= 2;
  auto groups = [&](int64_t s) { return (nleaves + s - 1) / s; };
  while (gsz > 1 && tiles * groups(gsz) < (int64_t)num_cus) gsz /= 2;
  return (int)gsz;
}

static int64_t gemv_groups(int64_t P) { return (P + GV_LEAVES - 1) / GV_LEAVES; }
static int64_t gemv_cols(int bt) { return 64 * (4 / elem_bytes(bt)); }

// The skinny-M path takes OP_NN products with at most GV_MAXM float32 rows.
static bool use_gemv(const GemmProblem& p) {
  return p.op == OP_NN && p.a_type == T_F32 && p.m >= 1 && p.m <= GV_MAXM;
}

// Stored shape of an operand of the MFMA path: [rows][cols] elements.
static void stored_shape(const GemmProblem& p, bool is_a, int64_t& rows, int64_t& cols) {
  if (is_a) {
    if (p.op == OP_TN) { rows = p.k; cols = p.m; } else { rows = p.m; cols = p.k; }
  } else {
    if (p.op == OP_NT) { rows = p.n; cols = p.k; } else { rows = p.k; cols = p.n; }
  }
}

// Floats of workspace the MFMA path needs to repack an operand whose base is not 16-byte
// aligned or whose rows are not a multiple of 16 bytes (0 when it is loaded in place).
static int64_t repack_floats(const GemmProblem& p, bool is_a) {
  int64_t rows, cols;
  stored_shape(p, is_a, rows, cols);
  const int eb = elem_bytes(is_a ? p.a_type : p.b_type);
  const void* base = is_a ? p.a : p.b;
  if ((cols * eb) % 16 == 0 && (base == nullptr || aligned(base, 16))) return 0;
  const int64_t ce = 16 / eb;
  const int64_t pitch = (cols + ce - 1) / ce * ce;
  return (rows * pitch * eb + 255) / 256 * 64;  // 256-byte granules
}

static int64_t round_floats(int64_t f) { return (f + 63) / 64 * 64; }

int64_t gemm_workspace_floats(const GemmProblem& p, int num_cus) {
  const int64_t L = p.leaf > 0 ? p.leaf : leaf_size(p.k);
  const int64_t P = leaf_count(p.k, L);
  if (P < 1 || p.m <= 0 || p.n <= 0) return 0;
  if (use_gemv(p)) return gemv_groups(P) > 1 ? gemv_groups(P) * p.m * p.n : 0;
  const int64_t tiles = ((p.m + BM - 1) / BM) * ((p.n + BN - 1) / BN);
  const int64_t gsz = P > 1 ? pick_group(P, tiles, num_cus) : 1;
  const int64_t ng = (P + gsz - 1) / gsz;
  return (ng > 1 ? round_floats(ng * p.m * p.n) : 0) + repack_floats(p, true) + repack_floats(p, false);
}

int64_t gemm_counter_count(const GemmProblem& p) {
  const int64_t L = p.leaf > 0 ? p.leaf : leaf_size(p.k);
  const int64_t P = leaf_count(p.k, L);
  if (!use_gemv(p) || p.n <= 0 || gemv_groups(P) <= 1) return 0;
  return (p.n + gemv_cols(p.b_type) - 1) / gemv_cols(p.b_type);
}

// vec: 0 element loads, 1 word (buffer) loads, 2 word loads of whole 128-row leaves
template <int BT, int MR>
static hipError_t launch_gemv_mr(const GemvArgs& g, const float* x, int vec, dim3 grid, hipStream_t s) {
  if (vec == 2) hipLaunchKernelGGL((gemv_nn_kernel<BT, MR, true, true>), grid, dim3(GV_THREADS), 0, s, g, x);
  else if (vec == 1) hipLaunchKernelGGL((gemv_nn_kernel<BT, MR, true, false>), grid, dim3(GV_THREADS), 0, s, g, x);
  else hipLaunchKernelGGL((gemv_nn_kernel<BT, MR, false, false>), grid, dim3(GV_THREADS), 0, s, g, x);
  return hipGetLastError();
}

template <int BT>
static hipError_t launch_gemv_m(const GemvArgs& g, const float* x, int64_t m, int vec, dim3 grid, hipStream_t s) {
  if (m <= 1) return launch_gemv_mr<BT, 1>(g, x, vec, grid, s);
  if (m <= 2) return launch_gemv_mr<BT, 2>(g, x, vec, grid, s);
  if (m <= 4) return launch_gemv_mr<BT, 4>(g, x, vec, grid, s);
  if (m <= 8) return launch_gemv_mr<BT, 8>(g, x, vec, grid, s);
  return launch_gemv_mr<BT, 16>(g, x, vec, grid, s);
}

static hipError_t launch_gemv_bt(const GemvArgs& g, const float* x, int bt, int64_t m, int vec, dim3 grid,
                                 hipStream_t s) {
  if (bt == T_F32) return launch_gemv_m<T_F32>(g, x, m, vec, grid, s);
  if (bt == T_BF16) return launch_gemv_m<T_BF16>(g, x, m, vec, grid, s);
  return launch_gemv_m<T_I8>(g, x, m, vec, grid, s);
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
    v.c = p.c; v.w = p.b; v.scales = p.scales; v.bias = p.bias;
    v.ws = ws; v.counter = counters;
    v.m = p.m; v.n = p.n; v.k = p.k; v.leaf = L; v.nleaves = P;
    v.ngroups = gemv_groups(P);
    v.ncg = (p.n + gemv_cols(p.b_type) - 1) / gemv_cols(p.b_type);
    if (v.ngroups > 1 && (ws == nullptr || counters == nullptr)) return hipErrorInvalidValue;
    const int eb = elem_bytes(p.b_type);
    // word loads need 4-byte rows and base, and GV_CH rows within a 31-bit buffer offset
    int vec = ((p.n * eb) % 4 == 0) && aligned(p.b, 4) && (int64_t)GV_CH * p.n * eb < (int64_t(1) << 31) ? 1 : 0;
    if (vec && L == GV_CH && p.k % GV_CH == 0) vec = 2;
    const int64_t grid = v.ncg * v.ngroups;
    return launch_gemv_bt(v, static_cast<const float*>(p.a), p.b_type, p.m, vec, dim3((unsigned)grid), stream);
  }
  GemmArgs g;
  g.c = p.c; g.a = p.a; g.b = p.b; g.scales = p.scales; g.bias = p.bias; g.ws = ws;
  g.m = p.m; g.n = p.n; g.k = p.k; g.leaf = L; g.nleaves = P;
  const int64_t tm = (p.m + BM - 1) / BM, tn = (p.n + BN - 1) / BN;
  g.tiles_n = (int)tn;
  const int64_t gsz = P > 1 ? pick_group(P, tm * tn, num_cus) : 1;
  g.group = gsz;
  g.ngroups = (P + gsz - 1) / gsz;
  // workspace: [group roots][A repacked][B repacked], each part 256-byte aligned
  float* wsp = ws + (g.ngroups > 1 ? round_floats(g.ngroups * p.m * p.n) : 0);
  const int64_t ra = repack_floats(p, true), rb = repack_floats(p, false);
  if ((g.ngroups > 1 || ra > 0 || rb > 0) && ws == nullptr) return hipErrorInvalidValue;
  for (int which = 0; which < 2; ++which) {
    const bool is_a = which == 0;
    int64_t rows, cols;
    stored_shape(p, is_a, rows, cols);
    const int eb = elem_bytes(is_a ? p.a_type : p.b_type);
    const int64_t ce = 16 / eb;
    const int64_t pitch = (cols + ce - 1) / ce * ce;
    const void* src = is_a ? p.a : p.b;
    if ((is_a ? ra : rb) > 0) {
      const int64_t total = rows * pitch;
      hipLaunchKernelGGL(repack_rows_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                         (char*)wsp, (const char*)src, rows, cols, pitch, eb);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      src = wsp;
      wsp += is_a ? ra : rb;
    }
    if (is_a) { g.a = src; g.a_pitch = pitch; g.a_bytes = rows * pitch * eb; }
    else { g.b = src; g.b_pitch = pitch; g.b_bytes = rows * pitch * eb; }
    // one load instruction spans at most 32 stored rows (int8, index-major)
    if ((32 * pitch + KT) * eb >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  }
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

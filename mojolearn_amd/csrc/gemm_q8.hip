// gfx950 kernels of the integer profiles mojolearn.identical.gemm.int8i32.v1
// (gemm/IDENTICAL_LOWBIT_CONTRACT.md L-3..L-7) and int15i64.v1 (section 6, W-1..W-7): the row
// quantizers, the dequantizers and the OP_NT products on the integer matrix unit.
//
// The product's only arithmetic before the store is an integer sum of int8 x int8 products in an
// Int32 that cannot overflow (k <= 131072), so the order in which the matrix unit adds them is
// scheduling (L-9's construction): v_mfma_i32_32x32x32_i8 gives the same Int32 as the oracle's
// ascending loop.  Codes past k are masked to zero (a zero code adds nothing).  The float steps,
// L-5's split conversion and L-6's power-of-two multiply and flush, run once per cell at the store.
#include "device_common.h"
#include "lds_stage.h"
#include "mfma.h"
#include "q8.h"

namespace mlg {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// checks/numerics.mojo:1589-1598 pow2_f32: 2^e from its exponent field; above 127 the infinity,
// below -126 +0.0.
__device__ __forceinline__ float q8_pow2(int64_t e) {
  if (e > 127) return __uint_as_float(0x7F800000u);
  if (e < -126) return 0.f;
  return __uint_as_float((uint32_t)(e + 127) << 23);
}

// checks/numerics.mojo:262-268: a subnormal becomes the zero of its own sign.
__device__ __forceinline__ float q8_ftz(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x7F800000u) == 0u ? __uint_as_float(u & 0x80000000u) : x;
}

// checks/numerics.mojo:1609-1630 i32_to_f32_pinned (L-5): two exact conversions (a 20-bit high
// part, a 12-bit low part), an exact scaling by 2^12, one IEEE addition.
__device__ __forceinline__ float q8_i32_to_f32(int32_t v) {
  const bool neg = v < 0;
  const uint32_t mag = neg ? (uint32_t)(-(int64_t)v) : (uint32_t)v;
  const float hi = (float)(mag >> 12);
  const float lo = (float)(mag & 0xFFFu);
  const float r = hi * 4096.0f + lo;
  return neg ? -r : r;
}

// checks/numerics.mojo:1671-1677 dequant_int8_pinned (L-6), then the store's NaN canonicalisation.
__device__ __forceinline__ float q8_dequant(int32_t acc, int64_t e_sum) {
  return store_word(q8_ftz(q8_i32_to_f32(acc) * q8_pow2(e_sum)));
}

// ---------------------------------------------------------------------------
// Quantizer (L-3, L-4; checks/numerics.mojo:1638-1668, gemm/host/gemm_lowbit_oracle.mojo:171-198):
// one 256-thread workgroup per row.  The absmax is a maximum (exact, order-free), so a tree
// reduction gives the oracle's value; a NaN never wins a comparison.
constexpr int Q8_THREADS = 256;

__device__ __forceinline__ float q8_absmax_step(float best, float x) {
  float v = q8_ftz(x);
  if (v < 0.f) v = -v;
  return v > best ? v : best;
}

__device__ __forceinline__ int8_t q8_code(float x, int e) {
  if (x != x) return 0;
  const float s = q8_ftz(q8_ftz(x) * q8_pow2(-(int64_t)e));
  const float magic = 12582912.0f;  // checks/numerics.mojo:1577-1586 f32_round_half_even
  float r = s >= 0.f ? (s + magic) - magic : (s - magic) + magic;
  if (r != r) return 0;  // 0 * 2^-e with 2^-e infinite (absmax below 2^-121): the reference's Int(NaN) -> 0
  if (r > 127.f) r = 127.f;
  if (r < -127.f) r = -127.f;
  return (int8_t)(int)r;
}

__global__ void __launch_bounds__(Q8_THREADS) q8_quantize_kernel(int8_t* codes, int32_t* exps, const float* x,
                                                                 int64_t cols) {
  __shared__ float wbest[Q8_THREADS / 64];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * cols;
  float best = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += Q8_THREADS) best = q8_absmax_step(best, xr[c]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(best, off, 64);
    best = o > best ? o : best;
  }
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
  __syncthreads();
  best = wbest[0];
#pragma unroll
  for (int w = 1; w < Q8_THREADS / 64; ++w) best = wbest[w] > best ? wbest[w] : best;
  // int8_row_exponent: floor(log2 absmax) - 6 from the exponent field; 0 for a zero row
  const float a = q8_ftz(best);
  const int e = (a == 0.f || a != a) ? 0 : (int)((__float_as_uint(a) >> 23) & 0xFFu) - 127 - 6;
  if (threadIdx.x == 0) exps[row] = e;
  int8_t* cr = codes + row * cols;
  for (int64_t c = threadIdx.x; c < cols; c += Q8_THREADS) cr[c] = q8_code(xr[c], e);
}

__global__ void q8_dequantize_kernel(float* out, const int8_t* codes, const int32_t* exps, int64_t rows,
                                     int64_t cols) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * cols) return;
  out[i] = q8_dequant((int32_t)codes[i], exps[i / cols]);
}

// ---------------------------------------------------------------------------
// The product.  Tiling as the fp32 MFMA kernel: 512 threads, a 128 x 128 cell tile, wave (wr, wc)
// owns rows wr*64 .. +63 (two 32-row blocks) and columns wc*32 .. +31.  Both operands store k
// contiguously (OP_NT), so a slice of 128 codes per row is staged exactly like an index-major
// float32 slice of 32 words (16-byte chunks, swizzled rows) and read 16 codes per lane: lane l of
// v_mfma_i32_32x32x32_i8 gives row / column l % 32 and codes 16 (l / 32) .. +15 of the 32-code
// step, the same k range for both operands.
struct Q8Args {
  float* c;
  const void* qa;      // [m][pitch] codes (pitch a multiple of 16 bytes)
  const void* qb;      // [n][pitch]
  const int32_t* ea;
  const int32_t* eb;
  int64_t m, n, k;
  int64_t pitch_words;  // pitch / 4
  int64_t a_bytes, b_bytes;
  int32_t* part;        // split k: [splits][m][n] Int32 partial sums, else nullptr
  int64_t sps;          // 128-code slices per split (blockIdx.y)
  int tiles_m, tiles_n;
};

constexpr int Q8_KS = KT * 4;  // codes per slice: 128

template <bool MASK>
__device__ __forceinline__ void q8_slice(v16i (&acc)[2], const char* la, const char* lb, int wr, int lane,
                                         int bcol, int64_t valid) {
#pragma unroll
  for (int q = 0; q < Q8_KS / 32; ++q) {
    const int s = 8 * q + 4 * (lane >> 5);  // word offset of this lane's 16 codes in the row
    const v4i b4 = __builtin_bit_cast(v4i, read4<T_F32, true>(lb, bcol, s, 1.f));
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      v4i a4 = __builtin_bit_cast(v4i, read4<T_F32, true>(la, wr * 64 + 32 * blk + (lane & 31), s, 1.f));
      if constexpr (MASK) {
        // codes at or past k are zero (they may hold the next row's bytes); 0 < valid < 128 here
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int d = (int)valid - 4 * (s + w);  // codes of this word below k
          const uint32_t keep = d >= 4 ? 0xFFFFFFFFu : (d <= 0 ? 0u : 0xFFFFFFFFu >> (8 * (4 - d)));
          a4[w] = (int)((uint32_t)a4[w] & keep);
        }
      }
      acc[blk] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a4, b4, acc[blk], 0, 0, 0);
    }
  }
}

__global__ void __launch_bounds__(NTHREADS) q8_gemm_kernel(Q8Args g) {
  __shared__ __attribute__((aligned(1024))) char lds0[2][SLICE_BYTES];
  __shared__ __attribute__((aligned(1024))) char lds1[2][SLICE_BYTES];
  __shared__ __attribute__((aligned(1024))) char lds2[2][SLICE_BYTES];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 2;
  const int wc = wave & 3;
  // the XCD-aware tile order (integer sums are exact: the order never changes a word)
  const int tile = tile_of(blockIdx.x, gridDim.x, g.tiles_m, g.tiles_n);
  const int64_t i0 = (int64_t)(tile / g.tiles_n) * BM;
  const int64_t j0 = (int64_t)(tile % g.tiles_n) * BN;
  const int64_t nslices = (g.k + Q8_KS - 1) / Q8_KS;
  const int64_t kt0 = (int64_t)blockIdx.y * g.sps;
  const int64_t kt1 = kt0 + g.sps < nslices ? kt0 + g.sps : nslices;

  DirectLoader<T_F32, true> lda, ldb;
  lda.init(g.pitch_words, wave, lane);
  ldb.init(g.pitch_words, wave, lane);
  constexpr int LPS = 2 * Slice<T_F32, true>::PER_WAVE;
  constexpr int WAIT_ONE_BEHIND = (LPS & 0xF) | ((LPS >> 4) << 14) | (0x7 << 4) | (0xF << 8);
  lda.issue(lds0[0], g.qa, g.a_bytes, g.pitch_words, i0, kt0 * KT, wave);
  ldb.issue(lds0[1], g.qb, g.b_bytes, g.pitch_words, j0, kt0 * KT, wave);
  lda.issue(lds1[0], g.qa, g.a_bytes, g.pitch_words, i0, (kt0 + 1) * KT, wave);
  ldb.issue(lds1[1], g.qb, g.b_bytes, g.pitch_words, j0, (kt0 + 1) * KT, wave);

  const int bcol = wc * 32 + (lane & 31);
  v16i acc[2];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[blk][e] = 0;

  __builtin_amdgcn_s_waitcnt(WAIT_ONE_BEHIND);
  lds_barrier();

  // Slice kt out of buffer CUR while slice kt + 2 loads into FILL (unrolled by three so the
  // compiler sees distinct buffers); the last slice masks the codes past k.
#define MLG_Q8_STEP(CUR, FILL)                                                                   \
  do {                                                                                           \
    lda.issue(FILL[0], g.qa, g.a_bytes, g.pitch_words, i0, (kt + 2) * KT, wave);                 \
    ldb.issue(FILL[1], g.qb, g.b_bytes, g.pitch_words, j0, (kt + 2) * KT, wave);                 \
    const int64_t valid = g.k - kt * Q8_KS;                                                      \
    if (valid >= Q8_KS) q8_slice<false>(acc, CUR[0], CUR[1], wr, lane, bcol, valid);             \
    else q8_slice<true>(acc, CUR[0], CUR[1], wr, lane, bcol, valid);                             \
    __builtin_amdgcn_s_waitcnt(WAIT_ONE_BEHIND);                                                 \
    lds_barrier();                                                                               \
  } while (0)
  for (int64_t kt = kt0; kt < kt1;) {
    MLG_Q8_STEP(lds0, lds2);
    if (++kt >= kt1) break;
    MLG_Q8_STEP(lds1, lds0);
    if (++kt >= kt1) break;
    MLG_Q8_STEP(lds2, lds1);
    ++kt;
  }
#undef MLG_Q8_STEP
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no load into LDS outlives the workgroup

  const int64_t col = j0 + bcol;
  if (col >= g.n) return;
  if (g.part != nullptr) {  // split k: the exact partial sums, folded by q8_reduce_kernel
    int32_t* pr = g.part + (int64_t)blockIdx.y * g.m * g.n;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = i0 + wr * 64 + 32 * blk + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
        if (row < g.m) pr[row * g.n + col] = acc[blk][r];
      }
    }
    return;
  }
  const int64_t eb = g.eb[col];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = i0 + wr * 64 + 32 * blk + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
      if (row < g.m) g.c[row * g.n + col] = q8_dequant(acc[blk][r], (int64_t)g.ea[row] + eb);
    }
  }
}

// The split-k fold: Int32 addition is exact and associative (every partial and every running
// sum is bounded by 16129 * k < 2^31), so adding the splits in order gives the one-pass sum.
__global__ void q8_reduce_kernel(float* c, const int32_t* part, const int32_t* ea, const int32_t* eb, int64_t m,
                                 int64_t n, int splits) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= m * n) return;
  int32_t acc = 0;
  for (int s = 0; s < splits; ++s) acc += part[s * m * n + i];
  c[i] = q8_dequant(acc, (int64_t)ea[i / n] + eb[i % n]);
}

// ---------------------------------------------------------------------------
// Few rows of A (m <= 4): a streaming dot product per cell.  Each wave owns QV_ROWS rows of B
// (qb[n][k], contiguous in k) and every row of A; lane l reads bytes 16 l .. 16 l + 15 of each
// 1024-byte chunk of those rows (a row's chunk is one coalesced 1 KB read) and accumulates them
// with v_dot4_i32_i8, then the 64 lane sums of a cell are added across the wave.  An Int32 sum of
// int8 products below k = 131072 is exact in any order, so the cell is the oracle's Int32.  The
// rows are bounded by their buffer resources (bytes past k read as zero codes).
constexpr int QV_THREADS = 256;
constexpr int QV_ROWS = 4;
constexpr int QV_MAXM = 4;  // beyond, the matrix-unit tiles are faster (t8 rows)

template <int MR>
__global__ void __launch_bounds__(QV_THREADS) q8_gemv_kernel(float* c, const int8_t* qa, const int32_t* ea,
                                                             const int8_t* qb, const int32_t* eb, int64_t m,
                                                             int64_t n, int64_t k) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (QV_THREADS / 64) + (threadIdx.x >> 6);
  const int64_t j0 = wave * QV_ROWS;
  if (j0 >= n) return;  // whole waves only: nothing after this point synchronizes
  __amdgpu_buffer_rsrc_t rb[QV_ROWS], ra[MR];
#pragma unroll
  for (int r = 0; r < QV_ROWS; ++r) {
    const int64_t j = j0 + r < n ? j0 + r : n - 1;  // rows past n: loaded, never stored
    rb[r] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(qb + j * k), (short)0, (int)k, RSRC_WORD3);
  }
#pragma unroll
  for (int i = 0; i < MR; ++i) {
    const int64_t ii = i < m ? i : m - 1;  // rows past m: computed, never stored
    ra[i] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(qa + ii * k), (short)0, (int)k, RSRC_WORD3);
  }
  int32_t acc[MR][QV_ROWS];
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int r = 0; r < QV_ROWS; ++r) acc[i][r] = 0;
  for (int kc = 0; kc < (int)k; kc += 1024) {
    const int off = kc + 16 * lane;
    v4i w[QV_ROWS], a[MR];
#pragma unroll
    for (int r = 0; r < QV_ROWS; ++r) w[r] = __builtin_amdgcn_raw_buffer_load_b128(rb[r], off, 0, 0);
#pragma unroll
    for (int i = 0; i < MR; ++i) a[i] = __builtin_amdgcn_raw_buffer_load_b128(ra[i], off, 0, 0);
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
      for (int r = 0; r < QV_ROWS; ++r)
#pragma unroll
        for (int d = 0; d < 4; ++d) acc[i][r] = __builtin_amdgcn_sdot4(a[i][d], w[r][d], acc[i][r], false);
  }
  // the wave's sum of each cell, then lane i * QV_ROWS + r stores cell (i, j0 + r)
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int r = 0; r < QV_ROWS; ++r) {
      int32_t v = acc[i][r];
#pragma unroll
      for (int sh = 32; sh >= 1; sh >>= 1) v += __shfl_xor(v, sh, 64);
      acc[i][r] = v;
    }
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int r = 0; r < QV_ROWS; ++r)
      if (lane == i * QV_ROWS + r && i < m && j0 + r < n)
        c[i * n + j0 + r] = q8_dequant(acc[i][r], (int64_t)ea[i] + eb[j0 + r]);
}

__global__ void q8_repack_kernel(int8_t* dst, const int8_t* src, int64_t rows, int64_t k, int64_t pitch) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * pitch) return;
  const int64_t r = i / pitch, c = i % pitch;
  dst[i] = c < k ? src[r * k + c] : (int8_t)0;
}

// ---------------------------------------------------------------------------
// Profile mojolearn.identical.gemm.int15i64.v1 (contract section 6, W-1..W-7): codes in
// [-16383, 16383] kept as two int8 planes, hi = floor(c / 128) in [-128, 127] and lo = c mod 128
// in [0, 127].  The product runs the planes on the same integer matrix unit: three exact Int32
// sums per cell, HH = sum ah bh, MID = sum (ah bl + al bh) (one accumulator, exact for
// k <= 66052) and LL = sum al bl, recombined in Int64 as HH 2^14 + MID 2^7 + LL (W-4, W-5), then
// W-6's pinned conversion and W-7's scale.  All three sums are integer, so their order is
// scheduling, as for int8i32.

constexpr int64_t INT15_MAX_K_DEV = 65536;

// checks/numerics_int15.mojo:123-163 i64_to_f32_pinned (W-6): two exact 24-bit conversions and
// one IEEE addition below 2^48; above, the low sixteen bits folded into a sticky bit and an
// exact scaling by 2^16.
__device__ __forceinline__ float q15_i64_to_f32(int64_t v) {
  const bool neg = v < 0;
  uint64_t mag = (uint64_t)v;
  if (neg) mag = (uint64_t)0 - mag;
  bool reduced = false;
  if (mag >= ((uint64_t)1 << 48)) {
    const uint64_t lost = mag & 0xFFFFu;
    mag >>= 16;
    if (lost) mag |= 1u;
    reduced = true;
  }
  const float hi = (float)(int32_t)(mag >> 24);
  const float lo = (float)(int32_t)(mag & 0xFFFFFFu);
  float r = hi * 16777216.0f + lo;
  if (reduced) r = r * 65536.0f;
  return neg ? -r : r;
}

// checks/numerics_int15.mojo:166-172 (W-7), then the store's NaN canonicalisation.
__device__ __forceinline__ float q15_dequant(int64_t acc, int64_t e_sum) {
  return store_word(q8_ftz(q15_i64_to_f32(acc) * q8_pow2(e_sum)));
}

// checks/numerics_int15.mojo:66-93 quantize_int15_value (W-2): a NaN codes to 0 before the
// scaling and after it.
__device__ __forceinline__ int q15_code(float x, int e) {
  if (x != x) return 0;
  const float s = q8_ftz(q8_ftz(x) * q8_pow2(-(int64_t)e));
  if (s != s) return 0;
  const float magic = 12582912.0f;  // checks/numerics.mojo:1577-1586 f32_round_half_even
  float r = s >= 0.f ? (s + magic) - magic : (s - magic) + magic;
  if (r > 16383.f) r = 16383.f;
  if (r < -16383.f) r = -16383.f;
  return (int)r;
}

// W-1..W-3 per row (gemm/host/gemm_int15_oracle.mojo:116-131, :160-168): int8i32's absmax,
// e = floor(log2 absmax) - 13, the codes straight to their planes.
__global__ void __launch_bounds__(Q8_THREADS) q15_quantize_kernel(int8_t* hi, int8_t* lo, int32_t* exps,
                                                                  const float* x, int64_t cols) {
  __shared__ float wbest[Q8_THREADS / 64];
  const int64_t row = blockIdx.x;
  const float* xr = x + row * cols;
  float best = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += Q8_THREADS) best = q8_absmax_step(best, xr[c]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float o = __shfl_xor(best, off, 64);
    best = o > best ? o : best;
  }
  if ((threadIdx.x & 63) == 0) wbest[threadIdx.x >> 6] = best;
  __syncthreads();
  best = wbest[0];
#pragma unroll
  for (int w = 1; w < Q8_THREADS / 64; ++w) best = wbest[w] > best ? wbest[w] : best;
  // checks/numerics_int15.mojo:54-63 int15_row_exponent
  const float a = q8_ftz(best);
  const int e = (a == 0.f || a != a) ? 0 : (int)((__float_as_uint(a) >> 23) & 0xFFu) - 127 - 13;
  if (threadIdx.x == 0) exps[row] = e;
  for (int64_t c = threadIdx.x; c < cols; c += Q8_THREADS) {
    const int q = q15_code(xr[c], e);
    hi[row * cols + c] = (int8_t)(q >> 7);   // int15_piece_hi: the arithmetic shift
    lo[row * cols + c] = (int8_t)(q & 127);  // int15_piece_lo: the low seven bits
  }
}

// gemm/host/gemm_int15_oracle.mojo:147-157 with :170-176: ftz(f32(hi * 128 + lo) * 2^e).
__global__ void q15_dequantize_kernel(float* out, const int8_t* hi, const int8_t* lo, const int32_t* exps,
                                      int64_t rows, int64_t cols) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * cols) return;
  out[i] = q15_dequant((int64_t)hi[i] * 128 + (int64_t)lo[i], exps[i / cols]);
}

// W-5 and the store of one cell.
__device__ __forceinline__ float q15_cell(int32_t hh, int32_t mid, int32_t ll, int64_t e_sum) {
  const int64_t s = ((int64_t)hh << 14) + ((int64_t)mid << 7) + (int64_t)ll;
  return q15_dequant(s, e_sum);
}

struct Q15Args {
  float* c;
  const void* ah;  // [m][pitch] planes (pitch a multiple of Q15_KS codes, zero codes past k)
  const void* al;
  const void* bh;  // [n][pitch]
  const void* bl;
  const int32_t* ea;
  const int32_t* eb;
  int64_t m, n, k;
  int64_t pitch_words;
  int64_t a_bytes, b_bytes;
  int32_t* part;  // split k: [splits][3][m][n] Int32 partial sums (HH, MID, LL), else nullptr
  int64_t sps;    // slices per split
  int tiles_m, tiles_n;
};

constexpr int Q15_SK = KT / 2;        // words per row per slice: 64 codes
constexpr int Q15_KS = Q15_SK * 4;    // codes per slice
constexpr int Q15_PLANE = BM * Q15_SK * 4;  // bytes of one plane's slice: 8 KB

// The four products of one 64-code slice.  Every row is stored at a pitch of whole slices with
// zero codes past k (the host repacks otherwise), so no code past k reaches a product.
__device__ __forceinline__ void q15_slice(v16i (&hh)[2], v16i (&mid)[2], v16i (&ll)[2], const char* lah,
                                          const char* lal, const char* lbh, const char* lbl, int wr, int lane,
                                          int bcol) {
#pragma unroll
  for (int q = 0; q < Q15_KS / 32; ++q) {
    const int s = 8 * q + 4 * (lane >> 5);  // word offset of this lane's 16 codes in the row
    const v4i bh4 = __builtin_bit_cast(v4i, read4<T_F32, true, Q15_SK>(lbh, bcol, s, 1.f));
    const v4i bl4 = __builtin_bit_cast(v4i, read4<T_F32, true, Q15_SK>(lbl, bcol, s, 1.f));
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
      const int arow = wr * 64 + 32 * blk + (lane & 31);
      const v4i ah4 = __builtin_bit_cast(v4i, read4<T_F32, true, Q15_SK>(lah, arow, s, 1.f));
      const v4i al4 = __builtin_bit_cast(v4i, read4<T_F32, true, Q15_SK>(lal, arow, s, 1.f));
      hh[blk] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah4, bh4, hh[blk], 0, 0, 0);
      mid[blk] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ah4, bl4, mid[blk], 0, 0, 0);
      mid[blk] = __builtin_amdgcn_mfma_i32_32x32x32_i8(al4, bh4, mid[blk], 0, 0, 0);
      ll[blk] = __builtin_amdgcn_mfma_i32_32x32x32_i8(al4, bl4, ll[blk], 0, 0, 0);
    }
  }
}

__global__ void __launch_bounds__(NTHREADS) q15_gemm_kernel(Q15Args g) {
  __shared__ __attribute__((aligned(1024))) char lds0[4][Q15_PLANE];
  __shared__ __attribute__((aligned(1024))) char lds1[4][Q15_PLANE];
  __shared__ __attribute__((aligned(1024))) char lds2[4][Q15_PLANE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave >> 2;
  const int wc = wave & 3;
  // the XCD-aware tile order (integer sums are exact: the order never changes a word)
  const int tile = tile_of(blockIdx.x, gridDim.x, g.tiles_m, g.tiles_n);
  const int64_t i0 = (int64_t)(tile / g.tiles_n) * BM;
  const int64_t j0 = (int64_t)(tile % g.tiles_n) * BN;
  const int64_t nslices = (g.k + Q15_KS - 1) / Q15_KS;
  const int64_t kt0 = (int64_t)blockIdx.y * g.sps;
  const int64_t kt1 = kt0 + g.sps < nslices ? kt0 + g.sps : nslices;

  DirectLoader<T_F32, true, Q15_SK> lah, lal, lbh, lbl;
  lah.init(g.pitch_words, wave, lane);
  lal.init(g.pitch_words, wave, lane);
  lbh.init(g.pitch_words, wave, lane);
  lbl.init(g.pitch_words, wave, lane);
  constexpr int LPS = 4 * Slice<T_F32, true, Q15_SK>::PER_WAVE;
  constexpr int WAIT_ONE_BEHIND = (LPS & 0xF) | ((LPS >> 4) << 14) | (0x7 << 4) | (0xF << 8);
#define MLG_Q15_ISSUE(BUF, KTI)                                                         \
  do {                                                                                  \
    lah.issue(BUF[0], g.ah, g.a_bytes, g.pitch_words, i0, (KTI) * Q15_SK, wave);        \
    lal.issue(BUF[1], g.al, g.a_bytes, g.pitch_words, i0, (KTI) * Q15_SK, wave);        \
    lbh.issue(BUF[2], g.bh, g.b_bytes, g.pitch_words, j0, (KTI) * Q15_SK, wave);        \
    lbl.issue(BUF[3], g.bl, g.b_bytes, g.pitch_words, j0, (KTI) * Q15_SK, wave);        \
  } while (0)
  MLG_Q15_ISSUE(lds0, kt0);
  MLG_Q15_ISSUE(lds1, kt0 + 1);

  const int bcol = wc * 32 + (lane & 31);
  v16i hh[2], mid[2], ll[2];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk)
#pragma unroll
    for (int e = 0; e < 16; ++e) hh[blk][e] = mid[blk][e] = ll[blk][e] = 0;

  __builtin_amdgcn_s_waitcnt(WAIT_ONE_BEHIND);
  lds_barrier();

#define MLG_Q15_STEP(CUR, FILL)                                                                    \
  do {                                                                                             \
    MLG_Q15_ISSUE(FILL, kt + 2);                                                                   \
    q15_slice(hh, mid, ll, CUR[0], CUR[1], CUR[2], CUR[3], wr, lane, bcol);                        \
    __builtin_amdgcn_s_waitcnt(WAIT_ONE_BEHIND);                                                   \
    lds_barrier();                                                                                 \
  } while (0)
  // whole rotations of the three buffers, then the zero to two slices left (single entry
  // and exit, so the accumulators keep their registers across the loop)
  int64_t kt = kt0;
  for (const int64_t kr = kt0 + (kt1 - kt0) / 3 * 3; kt < kr; kt += 3) {
    MLG_Q15_STEP(lds0, lds2);
    ++kt;
    MLG_Q15_STEP(lds1, lds0);
    ++kt;
    MLG_Q15_STEP(lds2, lds1);
    kt -= 2;
  }
  if (kt < kt1) {
    MLG_Q15_STEP(lds0, lds2);
    ++kt;
    if (kt < kt1) MLG_Q15_STEP(lds1, lds0);
  }
#undef MLG_Q15_STEP
#undef MLG_Q15_ISSUE
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): no load into LDS outlives the workgroup

  const int64_t col = j0 + bcol;
  if (col >= g.n) return;
  if (g.part != nullptr) {  // split k: the three exact partial sums, folded by q15_reduce_kernel
    int32_t* pr = g.part + (int64_t)blockIdx.y * 3 * g.m * g.n;
    const int64_t mn = g.m * g.n;
#pragma unroll
    for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = i0 + wr * 64 + 32 * blk + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
        if (row < g.m) {
          pr[row * g.n + col] = hh[blk][r];
          pr[mn + row * g.n + col] = mid[blk][r];
          pr[2 * mn + row * g.n + col] = ll[blk][r];
        }
      }
    }
    return;
  }
  const int64_t eb = g.eb[col];
#pragma unroll
  for (int blk = 0; blk < 2; ++blk) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t row = i0 + wr * 64 + 32 * blk + (r & 3) + 8 * (r >> 2) + 4 * (lane >> 5);
      if (row < g.m) g.c[row * g.n + col] = q15_cell(hh[blk][r], mid[blk][r], ll[blk][r], (int64_t)g.ea[row] + eb);
    }
  }
}

// The split-k fold of the three sums (each exact in Int32 for k <= 65536, every running sum
// bounded like the whole), then W-5..W-7.
__global__ void q15_reduce_kernel(float* c, const int32_t* part, const int32_t* ea, const int32_t* eb, int64_t m,
                                  int64_t n, int splits) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t mn = m * n;
  if (i >= mn) return;
  int32_t hh = 0, mid = 0, ll = 0;
  for (int s = 0; s < splits; ++s) {
    hh += part[(3 * s) * mn + i];
    mid += part[(3 * s + 1) * mn + i];
    ll += part[(3 * s + 2) * mn + i];
  }
  c[i] = q15_cell(hh, mid, ll, (int64_t)ea[i / n] + eb[i % n]);
}

// ---------------------------------------------------------------------------
// host side

static bool q8_in_place(const void* p, int64_t k) { return k % 16 == 0 && ((uintptr_t)p % 16u) == 0; }
static int64_t q8_pitch(int64_t k) { return (k + 15) / 16 * 16; }

// Split k when the output tiles leave CUs idle (the skinny decode rows): about two workgroups
// per CU, at least two slices per split, the partial sums capped at 64 MB.
static int64_t q8_splits(int64_t m, int64_t n, int64_t k, int num_cus, int64_t* sps, int ks = Q8_KS,
                         int64_t part_words = 1) {
  const int64_t tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  const int64_t nslices = (k + ks - 1) / ks;
  int64_t want = tiles >= num_cus ? 1 : (2 * (int64_t)num_cus + tiles - 1) / tiles;
  if (want > nslices / 2) want = nslices / 2;
  while (want > 1 && want * part_words * m * n * 4 > (int64_t(64) << 20)) --want;
  if (want < 1) want = 1;
  *sps = (nslices + want - 1) / want;
  return (nslices + *sps - 1) / *sps;
}

static int64_t round256(int64_t b) { return (b + 255) / 256 * 256; }

int64_t q8_workspace_bytes(const void* qa, const void* qb, int64_t m, int64_t n, int64_t k, int num_cus) {
  if (m <= QV_MAXM && q8_in_place(qa, k) && q8_in_place(qb, k)) return 0;  // the streaming kernel
  int64_t bytes = 0;
  if (!q8_in_place(qa, k)) bytes += round256(m * q8_pitch(k));
  if (!q8_in_place(qb, k)) bytes += round256(n * q8_pitch(k));
  int64_t sps;
  const int64_t splits = q8_splits(m, n, k, num_cus, &sps);
  if (splits > 1) bytes += round256(splits * m * n * 4);
  return bytes;
}

hipError_t run_q8_quantize(int8_t* codes, int32_t* exps, const float* x, int64_t rows, int64_t cols,
                           hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  hipLaunchKernelGGL(q8_quantize_kernel, dim3((unsigned)rows), dim3(Q8_THREADS), 0, stream, codes, exps, x, cols);
  return hipGetLastError();
}

hipError_t run_q8_dequantize(float* out, const int8_t* codes, const int32_t* exps, int64_t rows, int64_t cols,
                             hipStream_t stream) {
  const int64_t total = rows * cols;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(q8_dequantize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, out, codes,
                     exps, rows, cols);
  return hipGetLastError();
}

hipError_t run_q8_gemm(float* c, const int8_t* qa, const int32_t* ea, const int8_t* qb, const int32_t* eb,
                       int64_t m, int64_t n, int64_t k, void* ws, int num_cus, hipStream_t stream) {
  if (m <= 0 || n <= 0 || k <= 0 || k > INT8_MAX_K) return hipErrorInvalidValue;
  if (m <= QV_MAXM && q8_in_place(qa, k) && q8_in_place(qb, k)) {
    const unsigned grid = (unsigned)((n + QV_ROWS * (QV_THREADS / 64) - 1) / (QV_ROWS * (QV_THREADS / 64)));
#define MLG_QV(MR) hipLaunchKernelGGL(q8_gemv_kernel<MR>, dim3(grid), dim3(QV_THREADS), 0, stream, c, \
                                      static_cast<const int8_t*>(qa), ea, static_cast<const int8_t*>(qb), eb, m, n, k)
    if (m == 1) MLG_QV(1);
    else if (m == 2) MLG_QV(2);
    else MLG_QV(4);
#undef MLG_QV
    return hipGetLastError();
  }
  const int64_t pitch = q8_pitch(k);
  if (32 * pitch + Q8_KS >= (int64_t(1) << 30)) return hipErrorInvalidValue;
  char* wsp = static_cast<char*>(ws);
  const void* ops[2] = {qa, qb};
  const int64_t rows[2] = {m, n};
  for (int w = 0; w < 2; ++w) {
    if (q8_in_place(ops[w], k)) continue;
    if (wsp == nullptr) return hipErrorInvalidValue;
    const int64_t total = rows[w] * pitch;
    hipLaunchKernelGGL(q8_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<int8_t*>(wsp), static_cast<const int8_t*>(ops[w]), rows[w], k, pitch);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    ops[w] = wsp;
    wsp += round256(total);
  }
  int64_t sps;
  const int64_t splits = q8_splits(m, n, k, num_cus, &sps);
  int32_t* part = nullptr;
  if (splits > 1) {
    if (wsp == nullptr) return hipErrorInvalidValue;
    part = reinterpret_cast<int32_t*>(wsp);
  }
  Q8Args g;
  g.c = c; g.qa = ops[0]; g.qb = ops[1]; g.ea = ea; g.eb = eb;
  g.m = m; g.n = n; g.k = k;
  g.pitch_words = pitch / 4;
  g.a_bytes = m * pitch;
  g.b_bytes = n * pitch;
  const int64_t tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  g.tiles_m = (int)tm;
  g.tiles_n = (int)tn;
  g.part = part;
  g.sps = sps;
  hipLaunchKernelGGL(q8_gemm_kernel, dim3((unsigned)(tm * tn), (unsigned)splits), dim3(NTHREADS), 0, stream, g);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  hipLaunchKernelGGL(q8_reduce_kernel, dim3((unsigned)((m * n + 255) / 256)), dim3(256), 0, stream, c, part, ea, eb,
                     m, n, (int)splits);
  return hipGetLastError();
}


hipError_t run_q15_quantize(int8_t* hi, int8_t* lo, int32_t* exps, const float* x, int64_t rows, int64_t cols,
                            hipStream_t stream) {
  if (rows <= 0 || cols <= 0) return hipSuccess;
  hipLaunchKernelGGL(q15_quantize_kernel, dim3((unsigned)rows), dim3(Q8_THREADS), 0, stream, hi, lo, exps, x, cols);
  return hipGetLastError();
}

hipError_t run_q15_dequantize(float* out, const int8_t* hi, const int8_t* lo, const int32_t* exps, int64_t rows,
                              int64_t cols, hipStream_t stream) {
  const int64_t total = rows * cols;
  if (total <= 0) return hipSuccess;
  hipLaunchKernelGGL(q15_dequantize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, out, hi,
                     lo, exps, rows, cols);
  return hipGetLastError();
}

// The product reads whole 64-code slices: planes whose rows are not a multiple of 64 codes, or
// whose base is not 16-byte aligned, are repacked with zero codes to the next multiple.
static bool q15_in_place(const void* p, int64_t k) { return k % Q15_KS == 0 && ((uintptr_t)p % 16u) == 0; }
static int64_t q15_pitch(int64_t k) { return (k + Q15_KS - 1) / Q15_KS * Q15_KS; }

static bool q15_streams(const void* ah, const void* al, const void* bh, const void* bl, int64_t m, int64_t k);

int64_t q15_workspace_bytes(const void* ah, const void* al, const void* bh, const void* bl, int64_t m, int64_t n,
                            int64_t k, int num_cus) {
  if (q15_streams(ah, al, bh, bl, m, k)) return 0;  // the streaming kernel
  int64_t bytes = 0;
  if (!q15_in_place(ah, k) || !q15_in_place(al, k)) bytes += 2 * round256(m * q15_pitch(k));
  if (!q15_in_place(bh, k) || !q15_in_place(bl, k)) bytes += 2 * round256(n * q15_pitch(k));
  int64_t sps;
  const int64_t splits = q8_splits(m, n, k, num_cus, &sps, Q15_KS, 3);
  if (splits > 1) bytes += round256(splits * 3 * m * n * 4);
  return bytes;
}

// Few rows of A (m <= 4) under int15i64: the streaming kernel of the int8 product on both planes
// of A and B, the three Int32 sums of W-5 per cell (HH = ah.bh, MID = ah.bl + al.bh, LL = al.bl),
// each exact in any order below k = 65536 (|partial sums| stay under the contract's bound), then
// the cell's Int64 recombination and W-6 conversion.
template <int MR>
__global__ void __launch_bounds__(QV_THREADS) q15_gemv_kernel(float* c, const int8_t* ah, const int8_t* al,
                                                              const int32_t* ea, const int8_t* bh, const int8_t* bl,
                                                              const int32_t* eb, int64_t m, int64_t n, int64_t k) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * (QV_THREADS / 64) + (threadIdx.x >> 6);
  const int64_t j0 = wave * QV_ROWS;
  if (j0 >= n) return;  // whole waves only: nothing after this point synchronizes
  __amdgpu_buffer_rsrc_t rbh[QV_ROWS], rbl[QV_ROWS], rah[MR], ral[MR];
#pragma unroll
  for (int r = 0; r < QV_ROWS; ++r) {
    const int64_t j = j0 + r < n ? j0 + r : n - 1;  // rows past n: loaded, never stored
    rbh[r] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(bh + j * k), (short)0, (int)k, RSRC_WORD3);
    rbl[r] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(bl + j * k), (short)0, (int)k, RSRC_WORD3);
  }
#pragma unroll
  for (int i = 0; i < MR; ++i) {
    const int64_t ii = i < m ? i : m - 1;  // rows past m: computed, never stored
    rah[i] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(ah + ii * k), (short)0, (int)k, RSRC_WORD3);
    ral[i] = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(al + ii * k), (short)0, (int)k, RSRC_WORD3);
  }
  int32_t hh[MR][QV_ROWS], mid[MR][QV_ROWS], ll[MR][QV_ROWS];
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int r = 0; r < QV_ROWS; ++r) hh[i][r] = mid[i][r] = ll[i][r] = 0;
  for (int kc = 0; kc < (int)k; kc += 1024) {
    const int off = kc + 16 * lane;
    v4i wh[QV_ROWS], wl[QV_ROWS], xh[MR], xl[MR];
#pragma unroll
    for (int r = 0; r < QV_ROWS; ++r) {
      wh[r] = __builtin_amdgcn_raw_buffer_load_b128(rbh[r], off, 0, 0);
      wl[r] = __builtin_amdgcn_raw_buffer_load_b128(rbl[r], off, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < MR; ++i) {
      xh[i] = __builtin_amdgcn_raw_buffer_load_b128(rah[i], off, 0, 0);
      xl[i] = __builtin_amdgcn_raw_buffer_load_b128(ral[i], off, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < MR; ++i)
#pragma unroll
      for (int r = 0; r < QV_ROWS; ++r)
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          hh[i][r] = __builtin_amdgcn_sdot4(xh[i][d], wh[r][d], hh[i][r], false);
          mid[i][r] = __builtin_amdgcn_sdot4(xh[i][d], wl[r][d], mid[i][r], false);
          mid[i][r] = __builtin_amdgcn_sdot4(xl[i][d], wh[r][d], mid[i][r], false);
          ll[i][r] = __builtin_amdgcn_sdot4(xl[i][d], wl[r][d], ll[i][r], false);
        }
  }
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int r = 0; r < QV_ROWS; ++r) {
      int32_t a = hh[i][r], b = mid[i][r], d = ll[i][r];
#pragma unroll
      for (int sh = 32; sh >= 1; sh >>= 1) {
        a += __shfl_xor(a, sh, 64);
        b += __shfl_xor(b, sh, 64);
        d += __shfl_xor(d, sh, 64);
      }
      hh[i][r] = a;
      mid[i][r] = b;
      ll[i][r] = d;
    }
#pragma unroll
  for (int i = 0; i < MR; ++i)
#pragma unroll
    for (int r = 0; r < QV_ROWS; ++r)
      if (lane == i * QV_ROWS + r && i < m && j0 + r < n)
        c[i * n + j0 + r] = q15_cell(hh[i][r], mid[i][r], ll[i][r], (int64_t)ea[i] + eb[j0 + r]);
}

static bool q15_streams(const void* ah, const void* al, const void* bh, const void* bl, int64_t m, int64_t k) {
  return m <= QV_MAXM && q8_in_place(ah, k) && q8_in_place(al, k) && q8_in_place(bh, k) && q8_in_place(bl, k);
}

hipError_t run_q15_gemm(float* c, const int8_t* ah, const int8_t* al, const int32_t* ea, const int8_t* bh,
                        const int8_t* bl, const int32_t* eb, int64_t m, int64_t n, int64_t k, void* ws, int num_cus,
                        hipStream_t stream) {
  if (m <= 0 || n <= 0 || k <= 0 || k > INT15_MAX_K_DEV) return hipErrorInvalidValue;
  if (q15_streams(ah, al, bh, bl, m, k)) {
    const unsigned grid = (unsigned)((n + QV_ROWS * (QV_THREADS / 64) - 1) / (QV_ROWS * (QV_THREADS / 64)));
#define MLG_QV15(MR) hipLaunchKernelGGL(q15_gemv_kernel<MR>, dim3(grid), dim3(QV_THREADS), 0, stream, c, ah, al, ea, \
                                        bh, bl, eb, m, n, k)
    if (m == 1) MLG_QV15(1);
    else if (m == 2) MLG_QV15(2);
    else MLG_QV15(4);
#undef MLG_QV15
    return hipGetLastError();
  }
  const int64_t pitch = q15_pitch(k);
  if (32 * pitch + Q15_KS >= (int64_t(1) << 30)) return hipErrorInvalidValue;
  char* wsp = static_cast<char*>(ws);
  const void* pl[2][2] = {{ah, al}, {bh, bl}};
  const int64_t rows[2] = {m, n};
  for (int w = 0; w < 2; ++w) {
    if (q15_in_place(pl[w][0], k) && q15_in_place(pl[w][1], k)) continue;
    if (wsp == nullptr) return hipErrorInvalidValue;
    const int64_t total = rows[w] * pitch;
    for (int h = 0; h < 2; ++h) {
      hipLaunchKernelGGL(q8_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                         reinterpret_cast<int8_t*>(wsp), static_cast<const int8_t*>(pl[w][h]), rows[w], k, pitch);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      pl[w][h] = wsp;
      wsp += round256(total);
    }
  }
  int64_t sps;
  const int64_t splits = q8_splits(m, n, k, num_cus, &sps, Q15_KS, 3);
  int32_t* part = nullptr;
  if (splits > 1) {
    if (wsp == nullptr) return hipErrorInvalidValue;
    part = reinterpret_cast<int32_t*>(wsp);
  }
  Q15Args g;
  g.c = c; g.ah = pl[0][0]; g.al = pl[0][1]; g.bh = pl[1][0]; g.bl = pl[1][1]; g.ea = ea; g.eb = eb;
  g.m = m; g.n = n; g.k = k;
  g.pitch_words = pitch / 4;
  g.a_bytes = m * pitch;
  g.b_bytes = n * pitch;
  g.part = part;
  g.sps = sps;
  const int64_t tm = (m + BM - 1) / BM, tn = (n + BN - 1) / BN;
  g.tiles_m = (int)tm;
  g.tiles_n = (int)tn;
  hipLaunchKernelGGL(q15_gemm_kernel, dim3((unsigned)(tm * tn), (unsigned)splits), dim3(NTHREADS), 0, stream, g);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || splits == 1) return e;
  hipLaunchKernelGGL(q15_reduce_kernel, dim3((unsigned)((m * n + 255) / 256)), dim3(256), 0, stream, c, part, ea,
                     eb, m, n, (int)splits);
  return hipGetLastError();
}

}  // namespace mlg

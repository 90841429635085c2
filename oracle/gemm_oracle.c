/*
 * CPU oracle for the profile mojolearn.identical.gemm.fp32.v1 (TEST INFRASTRUCTURE).
 *
 * This file is the checker, never the product: only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load it.  The product path (mojolearn_amd) runs
 * hand-written gfx950 HIP kernels and has no CPU fallback.
 *
 * It restates, in plain C, the reference's normative CPU algorithm:
 *   - leaf rule                 gemm/contract.mojo:173-235
 *   - orientations _a_at/_b_at  gemm/host/gemm_oracle.mojo:122-137
 *   - leaf chain                gemm/host/gemm_oracle.mojo:146-206
 *   - balanced fold tree        gemm/host/gemm_oracle.mojo:218-272
 *   - gemm_oracle / _cell       gemm/host/gemm_oracle.mojo:275-371
 *   - gemm_oracle_serial        gemm/host/gemm_oracle.mojo:473-524
 *   - ftz (integer spelling)    checks/numerics.mojo:262-268
 *   - bf16 widen / narrow       checks/numerics.mojo:1548-1574
 *   - NaN canonicalization      core/nan_canon.mojo:55-130
 *   - bias add                  transformer/impl/llama/modeling_llama.mojo:3979-3989
 *   - card fill + FNV-1a64      bench/gemm_card_main.mojo:292-311, core/identity_trace.mojo:89-115
 *   - int8i32.v1 (L-3..L-7)     checks/numerics.mojo:1577-1677, gemm/host/gemm_lowbit_oracle.mojo:171-251
 *   - int15i64.v1 (W-1..W-7)    checks/numerics_int15.mojo:54-175, gemm/host/gemm_int15_oracle.mojo:116-270
 * and a fast threaded arm that computes the same bits (the role of the reference's
 * gemm/host/gemm_host_rows.mojo:467-556): operands flushed once, columns vectorised
 * with AVX2 FMA (one independent chain per column, so no reassociation inside a leaf),
 * the per-step flush done as a compare+select, leaves folded with the register-stack
 * form of the balanced tree (pushing partials in ascending order, merging with the
 * earlier slot on the left, draining lowest level first and joining on the left).
 *
 * Build flags (oracle/Makefile): -O3 -mavx2 -mfma -ffp-contract=off, no fast-math,
 * default MXCSR (no FTZ/DAZ).  fmaf() is therefore one IEEE fused multiply-add and
 * a*b is one IEEE multiply.
 *
 * Pinning (tests/test_oracle_*.py): the reference's own card hashes (device card and
 * host-capped oracle card), the verify-table gemm cells, the closed-form fixtures F1-F8
 * of gemm/checks/gemm_oracle_check.mojo, exact-rational brute force on tiny shapes,
 * and literal-tree == register-stack fold for P = 1..2100.
 *
 * orc_host_rows restates the reference's fast CPU column itself
 * (gemm/host/gemm_host_rows.mojo:163-225,246-556): flushed packed operands, panels of 32
 * columns, the per-step flush DEFERRED with a subnormal tracker and the panel recomputed with
 * a flush at every step when any raw result was subnormal, the fold in place, an unpacked
 * per-step-flush path for m <= 4.
 *
 * PLANTED MISTAKES.  A build with -DORC_SABOTAGE=<n> (oracle/Makefile target `sabotage`,
 * outputs under oracle/_sabotage/) plants one mistake of a plausible kind, so that a test can
 * be shown able to fail: a GPU parity case whose oracle answer moves under a variant is a case
 * that catches the same mistake in a kernel (tests/test_sabotage.py).  The default build
 * (ORC_SABOTAGE 0) plants nothing.  Under any variant the fast arms return orc_gemm's answer,
 * so the mistake reaches every caller (as the reference's GEMM_ORACLE_HOST_SABOTAGE does,
 * gemm/host/gemm_host_rows.mojo:473-487).
 *    1 fold pairs (q, q + width/2) instead of adjacent pairs (2q, 2q + 1)
 *    2 an odd level's last partial added to +0 instead of carried
 *    3 partials summed left to right (a serial fold)
 *    4 a step as a multiply and then an add (two roundings) instead of one fma
 *    5 a step whose exact value lies below 2^-126 flushed BEFORE rounding
 *    6 operands entering a step unflushed
 *    7 leaves of 32 steps (a tile kernel's slice) instead of the contract's leaf size
 *    8 every leaf's chain started from -0.0
 *    9 NaN words left with their payloads
 *   10 the bias add without flushing its operands
 *   11 the int8 column scale used unflushed
 *   12 the accumulator not flushed between steps
 *   13 orc_host_rows without the redo of its deferred flush (its own negative control,
 *      gemm/host/gemm_host_rows.mojo:84-87,200-201)
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define K_LEAF_MIN 128
#define MAX_LEAVES 1024
#define OP_NN 0
#define OP_NT 1
#define OP_TN 2

#ifndef ORC_SABOTAGE
#define ORC_SABOTAGE 0
#endif

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* checks/numerics.mojo:262-268: a subnormal becomes the zero of its own sign. */
static inline float ftz(float x) {
  uint32_t b = f2u(x);
  if ((b & 0x7F800000u) == 0u && (b & 0x007FFFFFu) != 0u) return u2f(b & 0x80000000u);
  return x;
}

float orc_ftz(float x) { return ftz(x); }
float orc_fma(float a, float b, float c) { return fmaf(a, b, c); }

/* gemm/contract.mojo:173-214 */
int64_t orc_leaf_size(int64_t k) {
  if (k <= 0) return 1;
#if ORC_SABOTAGE == 7
  if (k > 32) return 32;
#endif
  if (k <= K_LEAF_MIN) return k;
  int64_t p0 = (k + K_LEAF_MIN - 1) / K_LEAF_MIN;
  if (p0 <= MAX_LEAVES) return K_LEAF_MIN;
  return (k + MAX_LEAVES - 1) / MAX_LEAVES;
}

/* gemm/contract.mojo:217-226 */
int64_t orc_leaf_count(int64_t k, int64_t leaf) {
  if (k <= 0) return 0;
  if (leaf < 1) leaf = 1;
  return (k + leaf - 1) / leaf;
}

/* gemm/host/gemm_oracle.mojo:122-137 */
static inline float a_at(const float* a, int op, int64_t i, int64_t p, int64_t m, int64_t k) {
  return op == OP_TN ? a[p * m + i] : a[i * k + p];
}
static inline float b_at(const float* b, int op, int64_t p, int64_t j, int64_t n, int64_t k) {
  return op == OP_NT ? b[j * k + p] : b[p * n + j];
}

/* gemm/host/gemm_oracle.mojo:146-206 */
static inline float chain_step(float a, float b, float acc) {
#if ORC_SABOTAGE == 6
  const float fa = a, fb = b;
#else
  const float fa = ftz(a), fb = ftz(b);
#endif
#if ORC_SABOTAGE == 4
  const float prod = fa * fb; /* -ffp-contract=off: two roundings */
  return ftz(prod + acc);
#elif ORC_SABOTAGE == 5
  const double exact = (double)fa * (double)fb + (double)acc;
  if (exact != 0.0 && fabs(exact) < 0x1p-126) return exact < 0.0 ? -0.0f : 0.0f;
  return ftz(fmaf(fa, fb, acc));
#elif ORC_SABOTAGE == 12
  return fmaf(fa, fb, acc);
#else
  return ftz(fmaf(fa, fb, acc));
#endif
}

static float leaf_partial(const float* a, const float* b, int op, int64_t i, int64_t j, int64_t m,
                          int64_t n, int64_t k, int64_t p0, int64_t p1) {
#if ORC_SABOTAGE == 8
  float acc = -0.0f;
#else
  float acc = 0.0f;
#endif
  for (int64_t p = p0; p < p1; ++p) acc = chain_step(a_at(a, op, i, p, m, k), b_at(b, op, p, j, n, k), acc);
  return ftz(acc);
}

/* gemm/host/gemm_oracle.mojo:218-272: the literal level-by-level tree.  `buf` is
 * overwritten (it is the level being reduced in place: next[q] lands in cur[q]). */
float orc_fold_tree(float* buf, int64_t p) {
  if (p <= 0) return 0.0f;
#if ORC_SABOTAGE == 3
  float s = buf[0];
  for (int64_t t = 1; t < p; ++t) s = ftz(ftz(s) + ftz(buf[t]));
  return ftz(s);
#else
  int64_t width = p;
  while (width > 1) {
    int64_t pairs = width / 2;
#if ORC_SABOTAGE == 1
    for (int64_t q = 0; q < pairs; ++q) buf[q] = ftz(ftz(buf[q]) + ftz(buf[q + (width + 1) / 2]));
    if (width & 1) buf[pairs] = buf[pairs];
#else
    for (int64_t q = 0; q < pairs; ++q) buf[q] = ftz(ftz(buf[2 * q]) + ftz(buf[2 * q + 1]));
#if ORC_SABOTAGE == 2
    if (width & 1) buf[pairs] = ftz(ftz(buf[width - 1]) + 0.0f);
#else
    if (width & 1) buf[pairs] = buf[width - 1]; /* the carry: bit for bit */
#endif
#endif
    width = pairs + (width & 1);
  }
  return ftz(buf[0]);
#endif
}

/* The register-stack realisation of the same tree (what the device kernels and the
 * fast arm use); checked against orc_fold_tree for every P in tests. */
float orc_fold_stack(const float* parts, int64_t p) {
  if (p <= 0) return 0.0f;
  float slot[64];
  uint64_t occ = 0;
  for (int64_t t = 0; t < p; ++t) {
    float x = parts[t];
    int lvl = 0;
    while (occ & (1ull << lvl)) {
      x = ftz(ftz(slot[lvl]) + ftz(x));
      occ &= ~(1ull << lvl);
      ++lvl;
    }
    slot[lvl] = x;
    occ |= 1ull << lvl;
  }
  int have = 0;
  float r = 0.0f;
  for (int lvl = 0; lvl < 64; ++lvl) {
    if (!(occ & (1ull << lvl))) continue;
    r = have ? ftz(ftz(slot[lvl]) + ftz(r)) : slot[lvl];
    have = 1;
  }
  return ftz(r);
}

/* gemm/host/gemm_oracle.mojo:275-371 at an explicit leaf (0 = the contract's). */
void orc_gemm(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k, int op,
              int64_t leaf) {
  if (leaf <= 0) leaf = orc_leaf_size(k);
  int64_t pc = orc_leaf_count(k, leaf);
  float* parts = (float*)malloc(sizeof(float) * (size_t)(pc > 0 ? pc : 1));
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      if (pc == 0) { c[i * n + j] = 0.0f; continue; }
      if (pc == 1) { c[i * n + j] = ftz(leaf_partial(a, b, op, i, j, m, n, k, 0, k)); continue; }
      for (int64_t t = 0; t < pc; ++t) {
        int64_t e = (t + 1) * leaf;
        if (e > k) e = k;
        parts[t] = leaf_partial(a, b, op, i, j, m, n, k, t * leaf, e);
      }
      c[i * n + j] = orc_fold_tree(parts, pc);
    }
  free(parts);
}

/* gemm/host/gemm_oracle.mojo:473-524: one whole-k chain per cell (diagnostic). */
void orc_gemm_serial(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k,
                     int op) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) c[i * n + j] = ftz(leaf_partial(a, b, op, i, j, m, n, k, 0, k));
}

/* ---------------- fast arm: same bits, AVX2 + OpenMP ---------------- */

static inline __m256 vftz(__m256 x) {
  const __m256 sign = _mm256_castsi256_ps(_mm256_set1_epi32((int)0x80000000u));
  const __m256 tiny = _mm256_castsi256_ps(_mm256_set1_epi32(0x00800000));
  __m256 mag = _mm256_andnot_ps(sign, x);
  __m256 sub = _mm256_cmp_ps(mag, tiny, _CMP_LT_OQ); /* |x| < 2^-126 (zeros map to themselves) */
  return _mm256_blendv_ps(x, _mm256_and_ps(x, sign), sub);
}

#define FAST_VEC 4 /* 4 x 8 = 32 columns per panel */

/* One row i, one panel of 32 columns starting at j0 (full panel).  ae: row of A_eff
 * (flushed, length k), be: B_eff (flushed, k x ldb row-major). */
static void fast_panel(float* crow, const float* ae, const float* be, int64_t ldb, int64_t j0,
                       int64_t k, int64_t leaf, int64_t pc) {
  __m256 slot[48][FAST_VEC];
  uint64_t occ = 0;
  for (int64_t t = 0; t < pc; ++t) {
    int64_t p0 = t * leaf, p1 = p0 + leaf;
    if (p1 > k) p1 = k;
    __m256 acc[FAST_VEC];
    for (int v = 0; v < FAST_VEC; ++v) acc[v] = _mm256_setzero_ps();
    for (int64_t p = p0; p < p1; ++p) {
      __m256 av = _mm256_set1_ps(ae[p]);
      const float* bp = be + p * ldb + j0;
      for (int v = 0; v < FAST_VEC; ++v) acc[v] = vftz(_mm256_fmadd_ps(av, _mm256_loadu_ps(bp + 8 * v), acc[v]));
    }
    int lvl = 0;
    while (occ & (1ull << lvl)) {
      for (int v = 0; v < FAST_VEC; ++v) acc[v] = vftz(_mm256_add_ps(slot[lvl][v], acc[v]));
      occ &= ~(1ull << lvl);
      ++lvl;
    }
    for (int v = 0; v < FAST_VEC; ++v) slot[lvl][v] = acc[v];
    occ |= 1ull << lvl;
  }
  __m256 r[FAST_VEC];
  int have = 0;
  for (int lvl = 0; lvl < 48; ++lvl) {
    if (!(occ & (1ull << lvl))) continue;
    for (int v = 0; v < FAST_VEC; ++v) r[v] = have ? vftz(_mm256_add_ps(slot[lvl][v], r[v])) : slot[lvl][v];
    have = 1;
  }
  for (int v = 0; v < FAST_VEC; ++v) {
    if (!have) r[v] = _mm256_setzero_ps();
    _mm256_storeu_ps(crow + j0 + 8 * v, vftz(r[v]));
  }
}

/* Scalar tail column, same arithmetic. */
static float fast_cell(const float* ae, const float* be, int64_t ldb, int64_t j, int64_t k,
                       int64_t leaf, int64_t pc) {
  float slot[48];
  uint64_t occ = 0;
  for (int64_t t = 0; t < pc; ++t) {
    int64_t p0 = t * leaf, p1 = p0 + leaf;
    if (p1 > k) p1 = k;
    float acc = 0.0f;
    for (int64_t p = p0; p < p1; ++p) acc = ftz(fmaf(ae[p], be[p * ldb + j], acc));
    int lvl = 0;
    while (occ & (1ull << lvl)) {
      acc = ftz(slot[lvl] + acc);
      occ &= ~(1ull << lvl);
      ++lvl;
    }
    slot[lvl] = acc;
    occ |= 1ull << lvl;
  }
  float r = 0.0f;
  int have = 0;
  for (int lvl = 0; lvl < 48; ++lvl) {
    if (!(occ & (1ull << lvl))) continue;
    r = have ? ftz(slot[lvl] + r) : slot[lvl];
    have = 1;
  }
  return ftz(r);
}

/* A_eff (m x k, flushed) and B_eff (k x n, flushed) are materialised once; then rows
 * are spread over threads.  Output bits equal orc_gemm's. */
void orc_gemm_fast(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k,
                   int op, int64_t leaf, int nthreads) {
#if ORC_SABOTAGE != 0
  (void)nthreads;
  orc_gemm(c, a, b, m, n, k, op, leaf);
  return;
#endif
  if (leaf <= 0) leaf = orc_leaf_size(k);
  int64_t pc = orc_leaf_count(k, leaf);
  if (nthreads <= 0) nthreads = omp_get_max_threads();
  if (pc == 0) {
    for (int64_t i = 0; i < m * n; ++i) c[i] = 0.0f;
    return;
  }
  float* ae = (float*)malloc(sizeof(float) * (size_t)(m * k));
  float* be = (float*)malloc(sizeof(float) * (size_t)(k * n));
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t p = 0; p < k; ++p) ae[i * k + p] = ftz(a_at(a, op, i, p, m, k));
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int64_t p = 0; p < k; ++p)
    for (int64_t j = 0; j < n; ++j) be[p * n + j] = ftz(b_at(b, op, p, j, n, k));
  const int64_t panel = 8 * FAST_VEC;
  const int64_t npan = n / panel;
  /* work items: (row, panel) pairs, so skinny-m shapes still spread over threads */
  const int64_t items = m * (npan + 1);
#pragma omp parallel for num_threads(nthreads) schedule(dynamic, 4)
  for (int64_t it = 0; it < items; ++it) {
    int64_t i = it / (npan + 1), pj = it % (npan + 1);
    if (pj < npan) {
      fast_panel(c + i * n, ae + i * k, be, n, pj * panel, k, leaf, pc);
    } else {
      for (int64_t j = npan * panel; j < n; ++j) c[i * n + j] = fast_cell(ae + i * k, be, n, j, k, leaf, pc);
    }
  }
  free(ae);
  free(be);
}

/* ---------------- the reference's fast CPU column: gemm_host_rows ----------------
 * gemm/host/gemm_host_rows.mojo restated.  The arithmetic is orc_gemm's, cell for cell; what
 * changes is around it:
 *  - operands flushed once into packed copies: A_eff row-major [m][k]; B_eff as panels of
 *    GHR_G = 32 columns, each [k][32] contiguous, columns past n +0.0 (:232-288);
 *  - one panel's 32 cells of a row advance together as GHR_CHAINS = 4 AVX2 vectors of 8, one
 *    lane per cell, each lane one IEEE fma per step (:163-190);
 *  - the per-step flush DEFERRED: every raw result goes into the tracker
 *    min((bits - 1) & 0x7FFFFFFF), below 0x007FFFFF exactly when some raw result was
 *    subnormal (both zeros wrap high); then the panel is recomputed with a flush at every step
 *    (:120-131,185-198).  Operands are flushed, so only an accumulator can be subnormal, and
 *    where none was, ftz was the identity at every step;
 *  - the leaf partials folded in place level by level, an odd level's last row carried
 *    (:203-225);
 *  - m <= 4: no packing, B read in place, a flush at every step (:364-437);
 *  - tasks split the packing, then the cells by rows (m >= 2 tasks) or by panels (:509-551).
 * A NaN's payload may differ from orc_gemm's (x86 fma propagates the NaN of whichever operand
 * the compiler put first); after NaN canonicalization the words are orc_gemm's. */
#define GHR_FW 8
#define GHR_CHAINS 4
#define GHR_G (GHR_FW * GHR_CHAINS)
#define GHR_SMALL_M 4

static void ghr_pack_a(const float* a, int op, int64_t m, int64_t k, float* ap, int64_t lo, int64_t hi) {
  for (int64_t i = lo; i < hi; ++i)
    for (int64_t p = 0; p < k; ++p) ap[i * k + p] = ftz(a_at(a, op, i, p, m, k));
}

static void ghr_pack_b(const float* b, int op, int64_t n, int64_t k, float* bp, int64_t glo, int64_t ghi) {
  for (int64_t g = glo; g < ghi; ++g) {
    const int64_t j0 = g * GHR_G;
    const int64_t width = n - j0 < GHR_G ? n - j0 : GHR_G;
    float* panel = bp + g * k * GHR_G;
    for (int64_t p = 0; p < k; ++p)
      for (int64_t jj = 0; jj < GHR_G; ++jj)
        panel[p * GHR_G + jj] = jj < width ? ftz(b_at(b, op, p, j0 + jj, n, k)) : 0.0f;
  }
}

/* One panel's 32 cells over the leaf [pb, pe): dst[jj] = the leaf partial of column j0 + jj. */
static void ghr_panel_chain(const float* arow, const float* panel, int64_t pb, int64_t pe, float* dst,
                           int force_redo) {
  const __m256i one = _mm256_set1_epi32(1);
  const __m256i absm = _mm256_set1_epi32(0x7FFFFFFF);
  __m256 c[GHR_CHAINS];
  __m256i e[GHR_CHAINS];
  for (int q = 0; q < GHR_CHAINS; ++q) {
    c[q] = _mm256_setzero_ps();
    e[q] = _mm256_set1_epi32(-1);
  }
  for (int64_t p = pb; p < pe; ++p) {
    const __m256 sv = _mm256_set1_ps(arow[p]);
    for (int q = 0; q < GHR_CHAINS; ++q) {
      const __m256 raw = _mm256_fmadd_ps(sv, _mm256_loadu_ps(panel + p * GHR_G + q * GHR_FW), c[q]);
      e[q] = _mm256_min_epu32(e[q], _mm256_and_si256(_mm256_sub_epi32(_mm256_castps_si256(raw), one), absm));
      c[q] = raw;
    }
  }
  __m256i emin = _mm256_min_epu32(_mm256_min_epu32(e[0], e[1]), _mm256_min_epu32(e[2], e[3]));
  /* tracked values are below 2^31, so a signed compare orders them */
  const int sub = _mm256_movemask_epi8(_mm256_cmpgt_epi32(_mm256_set1_epi32(0x007FFFFF), emin)) != 0;
  int redo = force_redo || sub;
#if ORC_SABOTAGE == 13
  redo = 0;
#endif
  if (redo) {
    for (int q = 0; q < GHR_CHAINS; ++q) {
      __m256 acc = _mm256_setzero_ps();
      for (int64_t p = pb; p < pe; ++p)
        acc = vftz(_mm256_fmadd_ps(_mm256_set1_ps(arow[p]), _mm256_loadu_ps(panel + p * GHR_G + q * GHR_FW), acc));
      _mm256_storeu_ps(dst + q * GHR_FW, acc);
    }
    return;
  }
  for (int q = 0; q < GHR_CHAINS; ++q) _mm256_storeu_ps(dst + q * GHR_FW, c[q]);
}

/* The balanced tree over `pcount` rows of `width` partials at sp, in place, root in row 0. */
static void ghr_fold_in_place(float* sp, int64_t pcount, int64_t width) {
  int64_t w = pcount;
  while (w > 1) {
    const int64_t pairs = w / 2;
    for (int64_t q = 0; q < pairs; ++q) {
      float* dst = sp + q * width;
      const float* l = sp + 2 * q * width;
      const float* r = l + width;
      int64_t j = 0;
      for (; j + GHR_FW <= width; j += GHR_FW)
        _mm256_storeu_ps(dst + j, vftz(_mm256_add_ps(_mm256_loadu_ps(l + j), _mm256_loadu_ps(r + j))));
      for (; j < width; ++j) dst[j] = ftz(l[j] + r[j]);
    }
    if (w & 1) memmove(sp + pairs * width, sp + (w - 1) * width, sizeof(float) * (size_t)width); /* the carry */
    w = pairs + (w & 1);
  }
}

static void ghr_tile(const float* ap, const float* bp, float* c, int64_t n, int64_t k, int64_t lo, int64_t hi,
                     int64_t glo, int64_t ghi, int force_redo) {
  const int64_t leaf = orc_leaf_size(k), pcount = orc_leaf_count(k, leaf);
  float* scratch = (float*)malloc(sizeof(float) * (size_t)(pcount * GHR_G));
  for (int64_t g = glo; g < ghi; ++g) {
    const float* panel = bp + g * k * GHR_G;
    const int64_t j0 = g * GHR_G;
    const int64_t width = n - j0 < GHR_G ? n - j0 : GHR_G;
    for (int64_t i = lo; i < hi; ++i) {
      for (int64_t t = 0; t < pcount; ++t) {
        const int64_t pb = t * leaf, pe = pb + leaf < k ? pb + leaf : k;
        ghr_panel_chain(ap + i * k, panel, pb, pe, scratch + t * GHR_G, force_redo);
      }
      if (pcount > 1) ghr_fold_in_place(scratch, pcount, GHR_G);
      memcpy(c + i * n + j0, scratch, sizeof(float) * (size_t)width);
    }
  }
  free(scratch);
}

/* m <= 4: columns [jlo, jhi), B read in place, a flush at every step. */
static void ghr_small_m(const float* a, const float* b, float* c, int op, int64_t m, int64_t n, int64_t k,
                        int64_t jlo, int64_t jhi) {
  const int64_t leaf = orc_leaf_size(k), pcount = orc_leaf_count(k, leaf);
  const int64_t width = m * GHR_FW;
  float* scratch = (float*)malloc(sizeof(float) * (size_t)(pcount * width));
  for (int64_t j0 = jlo; j0 < jhi; j0 += GHR_FW) {
    const int full = j0 + GHR_FW <= jhi;
    for (int64_t t = 0; t < pcount; ++t) {
      const int64_t pb = t * leaf, pe = pb + leaf < k ? pb + leaf : k;
      float* dst = scratch + t * width;
      if (full) {
        __m256 acc[GHR_SMALL_M];
        for (int64_t i = 0; i < m; ++i) acc[i] = _mm256_setzero_ps();
        for (int64_t p = pb; p < pe; ++p) {
          float bv[GHR_FW];
          for (int r = 0; r < GHR_FW; ++r) bv[r] = ftz(b_at(b, op, p, j0 + r, n, k));
          const __m256 bw = _mm256_loadu_ps(bv);
          for (int64_t i = 0; i < m; ++i)
            acc[i] = vftz(_mm256_fmadd_ps(_mm256_set1_ps(ftz(a_at(a, op, i, p, m, k))), bw, acc[i]));
        }
        for (int64_t i = 0; i < m; ++i) _mm256_storeu_ps(dst + i * GHR_FW, acc[i]);
      } else {
        for (int64_t i = 0; i < m; ++i)
          for (int64_t jj = 0; jj < GHR_FW; ++jj) {
            float acc = 0.0f;
            if (j0 + jj < jhi)
              for (int64_t p = pb; p < pe; ++p)
                acc = ftz(fmaf(ftz(a_at(a, op, i, p, m, k)), ftz(b_at(b, op, p, j0 + jj, n, k)), acc));
            dst[i * GHR_FW + jj] = acc;
          }
      }
    }
    if (pcount > 1) ghr_fold_in_place(scratch, pcount, width);
    const int64_t cnt = jhi - j0 < GHR_FW ? jhi - j0 : GHR_FW;
    for (int64_t i = 0; i < m; ++i) memcpy(c + i * n + j0, scratch + i * GHR_FW, sizeof(float) * (size_t)cnt);
  }
  free(scratch);
}

/* gemm/host/gemm_host_rows.mojo:492-556 gemm_host_rows_into: C = op(A) . op(B), the bits of
 * orc_gemm, on `nthreads` threads (0 = all).  `force_redo` takes the flushed recomputation on
 * every panel (the reference's check of its redo path). */
void orc_host_rows(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k, int op,
                   int nthreads, int force_redo) {
#if ORC_SABOTAGE != 0 && ORC_SABOTAGE != 13
  (void)nthreads;
  (void)force_redo;
  orc_gemm(c, a, b, m, n, k, op, 0);
  return;
#endif
  if (m <= 0 || n <= 0) return;
  if (nthreads <= 0) nthreads = omp_get_max_threads();
  if (k <= 0) {
    for (int64_t i = 0; i < m * n; ++i) c[i] = 0.0f;
    return;
  }
  if (m <= GHR_SMALL_M) {
    const int64_t blocks = (n + GHR_FW - 1) / GHR_FW;
    const int64_t chunk = (blocks + nthreads - 1) / nthreads;
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int t = 0; t < nthreads; ++t) {
      const int64_t lo = t * chunk * GHR_FW, hi = (t + 1) * chunk * GHR_FW;
      if (lo < n) ghr_small_m(a, b, c, op, m, n, k, lo, hi < n ? hi : n);
    }
    return;
  }
  const int64_t npan = (n + GHR_G - 1) / GHR_G;
  float* ap = (float*)malloc(sizeof(float) * (size_t)(m * k));
  float* bp = (float*)malloc(sizeof(float) * (size_t)(npan * k * GHR_G));
  const int64_t rchunk = (m + nthreads - 1) / nthreads, pchunk = (npan + nthreads - 1) / nthreads;
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int t = 0; t < nthreads; ++t) {
    const int64_t r0 = t * rchunk, r1 = (t + 1) * rchunk < m ? (t + 1) * rchunk : m;
    const int64_t g0 = t * pchunk, g1 = (t + 1) * pchunk < npan ? (t + 1) * pchunk : npan;
    if (r0 < r1) ghr_pack_a(a, op, m, k, ap, r0, r1);
    if (g0 < g1) ghr_pack_b(b, op, n, k, bp, g0, g1);
  }
  const int by_rows = m >= 2 * (int64_t)nthreads;
#pragma omp parallel for num_threads(nthreads) schedule(static)
  for (int t = 0; t < nthreads; ++t) {
    if (by_rows) {
      const int64_t r0 = t * rchunk, r1 = (t + 1) * rchunk < m ? (t + 1) * rchunk : m;
      if (r0 < r1) ghr_tile(ap, bp, c, n, k, r0, r1, 0, npan, force_redo);
    } else {
      const int64_t g0 = t * pchunk, g1 = (t + 1) * pchunk < npan ? (t + 1) * pchunk : npan;
      if (g0 < g1) ghr_tile(ap, bp, c, n, k, 0, m, g0, g1, force_redo);
    }
  }
  free(ap);
  free(bp);
}

/* ---------------- seams around the product ---------------- */

/* transformer/impl/llama/modeling_llama.mojo:3979-3989: y = ftz(ftz(y) + ftz(b[col])). */
void orc_bias(float* y, const float* bias, int64_t m, int64_t n) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
#if ORC_SABOTAGE == 10
      y[i * n + j] = ftz(y[i * n + j] + bias[j]);
#else
      y[i * n + j] = ftz(ftz(y[i * n + j]) + ftz(bias[j]));
#endif
    }
}

/* core/nan_canon.mojo:55-110: every NaN word becomes 0x7FC00000, nothing else moves. */
void orc_nan_canon(float* x, int64_t count) {
  uint32_t* w = (uint32_t*)x;
#if ORC_SABOTAGE == 9
  (void)w;
  (void)count;
  return;
#endif
  for (int64_t i = 0; i < count; ++i)
    if ((w[i] & 0x7FFFFFFFu) > 0x7F800000u) w[i] = 0x7FC00000u;
}

/* checks/numerics.mojo:1548-1551 (L-1): bits << 16, exact. */
void orc_bf16_widen(float* out, const uint16_t* in, int64_t count) {
  for (int64_t i = 0; i < count; ++i) out[i] = u2f((uint32_t)in[i] << 16);
}

/* checks/numerics.mojo:1554-1574 (L-2): ftz, then RNE on the low 16 bits; a NaN stays a
 * quiet NaN with its sign and top payload bits; overflow rounds into the infinity. */
void orc_bf16_narrow(uint16_t* out, const float* in, int64_t count) {
  for (int64_t i = 0; i < count; ++i) {
    uint32_t bb = f2u(ftz(in[i]));
    if ((bb & 0x7F800000u) == 0x7F800000u && (bb & 0x007FFFFFu) != 0u) {
      out[i] = (uint16_t)((bb >> 16) | 0x0040u);
      continue;
    }
    uint32_t lsb = (bb >> 16) & 1u;
    out[i] = (uint16_t)((bb + 0x7FFFu + lsb) >> 16);
  }
}

/* The per-output-channel int8 weight of the decode workload: W_eff = ftz(f32(code) * ftz(scale[j])),
 * one RNE multiply (the checks/numerics.mojo:1665-1671 spelling with the power of two replaced
 * by an fp32 scale, flushed like every other operand seam).  `codes` is laid out as the B operand of `op` (k x n for NN/TN, n x k
 * for NT); the output is the dequantised matrix in the same layout. */
void orc_int8_dequant(float* out, const int8_t* codes, const float* scales, int64_t n, int64_t k,
                      int op) {
  for (int64_t p = 0; p < k; ++p)
    for (int64_t j = 0; j < n; ++j) {
      int64_t idx = op == OP_NT ? j * k + p : p * n + j;
#if ORC_SABOTAGE == 11
      out[idx] = ftz((float)codes[idx] * scales[j]);
#else
      out[idx] = ftz((float)codes[idx] * ftz(scales[j]));
#endif
    }
}

/* core/identity_trace.mojo:89-115: FNV-1a64 over bytes in order. */
/* ---- profile mojolearn.identical.gemm.int8i32.v1 (gemm/IDENTICAL_LOWBIT_CONTRACT.md L-3..L-7) ----
 * Both operands are int8 codes with one power-of-two exponent per row; OP_NT only. */

/* checks/numerics.mojo:1589-1598 pow2_f32: 2^e from the exponent field; above 127 the
 * infinity, below -126 +0.0 (no subnormal scales). */
static inline float pow2_f32(int64_t e) {
  if (e > 127) return u2f(0x7F800000u);
  if (e < -126) return 0.0f;
  return u2f((uint32_t)(e + 127) << 23);
}

/* checks/numerics.mojo:1577-1586 f32_round_half_even: the magic-constant rounding. */
static inline float round_half_even_f32(float x) {
  const float magic = 12582912.0f;
  if (x >= 0.0f) return (x + magic) - magic;
  return (x - magic) + magic;
}

/* checks/numerics.mojo:1609-1630 i32_to_f32_pinned (L-5): a 20-bit high part and a 12-bit
 * low part converted exactly, the high part scaled by 2^12 exactly, one IEEE addition. */
float orc_q8_i32_to_f32(int32_t v) {
  const int neg = v < 0;
  int64_t w = v;
  if (neg) w = -w;
  const uint32_t mag = (uint32_t)w;
  const float hi = (float)(mag >> 12);
  const float lo = (float)(mag & 0xFFFu);
  const float r = hi * 4096.0f + lo;
  return neg ? -r : r;
}

/* checks/numerics.mojo:1638-1647 int8_row_exponent (L-3): floor(log2 absmax) - 6 read off the
 * exponent field (checks/numerics.mojo:1601-1606); a zero row takes 0. */
int orc_q8_row_exponent(float absmax) {
  const float a = ftz(absmax);
  if (a == 0.0f || a != a) return 0;
  return (int)((f2u(a) >> 23) & 0xFFu) - 127 - 6;
}

/* checks/numerics.mojo:1650-1668 quantize_int8_value (L-4). */
static inline int8_t q8_value(float x, int e) {
  if (x != x) return 0;
  const float s = ftz(ftz(x) * pow2_f32(-(int64_t)e));
  float r = round_half_even_f32(s);
  /* A zero times an infinite 2^-e (a row whose absmax is below 2^-121) is NaN; the
   * reference's Int8(Int(NaN)) keeps the low byte of the integer-indefinite word, 0. */
  if (r != r) return 0;
  if (r > 127.0f) r = 127.0f;
  if (r < -127.0f) r = -127.0f;
  return (int8_t)(int)r;
}

/* gemm/host/gemm_lowbit_oracle.mojo:171-198 row_absmax + quantize_rows_int8: per row the
 * largest flushed magnitude (a NaN never wins the comparison), its exponent, the codes. */
void orc_q8_quantize_rows(int8_t* codes, int32_t* exps, const float* x, int64_t rows, int64_t cols) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float best = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      float v = ftz(x[r * cols + c]);
      if (v < 0.0f) v = -v;
      if (v > best) best = v;
    }
    const int e = orc_q8_row_exponent(best);
    exps[r] = e;
    for (int64_t c = 0; c < cols; ++c) codes[r * cols + c] = q8_value(x[r * cols + c], e);
  }
}

/* checks/numerics.mojo:1671-1677 dequant_int8_pinned (L-6) on an Int32 and an exponent sum. */
static inline float q8_dequant(int32_t acc, int64_t e_sum) {
  return ftz(orc_q8_i32_to_f32(acc) * pow2_f32(e_sum));
}

/* gemm/host/gemm_lowbit_oracle.mojo:201-214 dequantize_rows_int8: code * 2^e per row. */
void orc_q8_dequantize_rows(float* out, const int8_t* codes, const int32_t* exps, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) out[r * cols + c] = q8_dequant(codes[r * cols + c], exps[r]);
}

/* gemm/host/gemm_lowbit_oracle.mojo:217-251 int8_dot_cell + gemm_int8_oracle (L-7): OP_NT,
 * C[i,j] = ftz(f32(sum_p qa[i,p] qb[j,p]) * 2^(ea[i] + eb[j])), the sum exact in Int32 for
 * k <= 131072. */
void orc_q8_gemm(float* c, const int8_t* qa, const int32_t* ea, const int8_t* qb, const int32_t* eb, int64_t m,
                 int64_t n, int64_t k) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      int32_t acc = 0;
      for (int64_t p = 0; p < k; ++p) acc += (int32_t)qa[i * k + p] * (int32_t)qb[j * k + p];
      c[i * n + j] = q8_dequant(acc, (int64_t)ea[i] + (int64_t)eb[j]);
    }
}

/* ---- profile mojolearn.identical.gemm.int15i64.v1 (gemm/IDENTICAL_LOWBIT_CONTRACT.md section 6,
 * W-1..W-7): fifteen-bit codes kept as two int8 planes, hi = floor(c / 128) and lo = c mod 128, an
 * exact Int64 sum, one pinned conversion, one power-of-two scale; OP_NT only, k <= 65536. */

/* checks/numerics_int15.mojo:54-63 int15_row_exponent (W-1): floor(log2 absmax) - 13. */
int orc_q15_row_exponent(float absmax) {
  const float a = ftz(absmax);
  if (a == 0.0f || a != a) return 0;
  return (int)((f2u(a) >> 23) & 0xFFu) - 127 - 13;
}

/* checks/numerics_int15.mojo:66-93 quantize_int15_value (W-2): a NaN codes to 0 before the
 * scaling and after it (a zero times an infinite 2^-e). */
static inline int16_t q15_value(float x, int e) {
  if (x != x) return 0;
  const float s = ftz(ftz(x) * pow2_f32(-(int64_t)e));
  if (s != s) return 0;
  float r = round_half_even_f32(s);
  if (r > 16383.0f) r = 16383.0f;
  if (r < -16383.0f) r = -16383.0f;
  return (int16_t)(int)r;
}

/* checks/numerics_int15.mojo:96-109 (W-3): the low seven bits, and the arithmetic shift. */
static inline int8_t q15_lo(int16_t c) { return (int8_t)((int32_t)c & 127); }
static inline int8_t q15_hi(int16_t c) { return (int8_t)((int32_t)c >> 7); }

/* checks/numerics_int15.mojo:123-163 i64_to_f32_pinned (W-6): below 2^48 two exact 24-bit
 * conversions, the high one scaled by 2^24, one IEEE addition; from 2^48 the low sixteen bits
 * fold into a sticky bit and the result is scaled by 2^16. */
float orc_q15_i64_to_f32(int64_t v) {
  const int neg = v < 0;
  uint64_t mag = (uint64_t)v;
  if (neg) mag = (uint64_t)0 - mag;
  int reduced = 0;
  if (mag >= ((uint64_t)1 << 48)) {
    const uint64_t lost = mag & 0xFFFFu;
    mag >>= 16;
    if (lost) mag |= 1u;
    reduced = 1;
  }
  const float hi = (float)(int32_t)(mag >> 24);
  const float lo = (float)(int32_t)(mag & 0xFFFFFFu);
  float r = hi * 16777216.0f + lo;
  if (reduced) r = r * 65536.0f;
  return neg ? -r : r;
}

/* checks/numerics_int15.mojo:166-172 dequant_int15_pinned (W-7). */
static inline float q15_dequant(int64_t acc, int64_t e_sum) {
  return ftz(orc_q15_i64_to_f32(acc) * pow2_f32(e_sum));
}

/* gemm/host/gemm_int15_oracle.mojo:116-131 quantize_rows_int15 and :160-168 split_int15: per row
 * the int8i32 absmax, its W-1 exponent, the W-2 codes, written as the two planes. */
void orc_q15_quantize_rows(int8_t* hi, int8_t* lo, int32_t* exps, const float* x, int64_t rows, int64_t cols) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float best = 0.0f;
    for (int64_t c = 0; c < cols; ++c) {
      float v = ftz(x[r * cols + c]);
      if (v < 0.0f) v = -v;
      if (v > best) best = v;
    }
    const int e = orc_q15_row_exponent(best);
    exps[r] = e;
    for (int64_t c = 0; c < cols; ++c) {
      const int16_t q = q15_value(x[r * cols + c], e);
      hi[r * cols + c] = q15_hi(q);
      lo[r * cols + c] = q15_lo(q);
    }
  }
}

/* gemm/host/gemm_int15_oracle.mojo:147-157 dequantize_rows_int15 with :170-176 join_int15:
 * ftz(f32(hi * 128 + lo) * 2^e) through the W-6/W-7 seam. */
void orc_q15_dequantize_rows(float* out, const int8_t* hi, const int8_t* lo, const int32_t* exps, int64_t rows,
                             int64_t cols) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      const int64_t q = (int64_t)hi[r * cols + c] * 128 + (int64_t)lo[r * cols + c];
      out[r * cols + c] = q15_dequant(q, exps[r]);
    }
}

/* gemm/host/gemm_int15_oracle.mojo:179-189 int15_dot_cell and :232-270 gemm_int15_oracle, the
 * FLAT definition: codes joined from the planes, each product in Int32, the sum in Int64 (p
 * ascending), then W-6/W-7. */
void orc_q15_gemm(float* c, const int8_t* ah, const int8_t* al, const int32_t* ea, const int8_t* bh,
                  const int8_t* bl, const int32_t* eb, int64_t m, int64_t n, int64_t k) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      int64_t acc = 0;
      for (int64_t p = 0; p < k; ++p) {
        const int32_t qa = (int32_t)ah[i * k + p] * 128 + (int32_t)al[i * k + p];
        const int32_t qb = (int32_t)bh[j * k + p] * 128 + (int32_t)bl[j * k + p];
        acc += (int64_t)(qa * qb);
      }
      c[i * n + j] = q15_dequant(acc, (int64_t)ea[i] + (int64_t)eb[j]);
    }
}

/* gemm/f16_widen.mojo:12-37 f16_bits_to_f32_bits: float16 bits widened exactly, a subnormal
 * renormalized, NaN payloads kept. */
void orc_f16_widen(uint32_t* out, const uint16_t* in, int64_t count) {
  for (int64_t i = 0; i < count; ++i) {
    const uint32_t h = in[i];
    const uint32_t s = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x03FFu;
    if (e == 0u) {
      if (m == 0u) { out[i] = s; continue; }
      uint32_t shift = 0;
      while ((m & 0x0400u) == 0u) { m <<= 1; ++shift; }
      m &= 0x03FFu;
      out[i] = s | ((113u - shift) << 23) | (m << 13);
    } else if (e == 31u) {
      out[i] = s | 0x7F800000u | (m << 13);
    } else {
      out[i] = s | ((e + 112u) << 23) | (m << 13);
    }
  }
}

uint64_t orc_fnv1a64(const void* data, int64_t nbytes) {
  const uint8_t* p = (const uint8_t*)data;
  uint64_t h = 0xCBF29CE484222325ull;
  for (int64_t i = 0; i < nbytes; ++i) h = (h ^ (uint64_t)p[i]) * 0x100000001B3ull;
  return h;
}

/* bench/gemm_card_main.mojo:292-311: a splitmix64-style mix of (index, salt), then
 * <int in [-1048575, 1048575]> / 2^20, exact in binary32. */
static inline uint64_t card_mix(int64_t i, int64_t salt) {
  uint64_t z = (uint64_t)(i + 1) * 0x9E3779B97F4A7C15ull + (uint64_t)(salt + 1) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
void orc_card_fill(float* out, int64_t count, int64_t salt) {
  for (int64_t i = 0; i < count; ++i) {
    int64_t num = (int64_t)(card_mix(i, salt) % 2097151ull) - 1048575;
    out[i] = (float)num / 1048576.0f;
  }
}

int orc_max_threads(void) { return omp_get_max_threads(); }

/* ---- the sequence executor's GEMM word and its followers ------------------------------------
 * sequence/ops.mojo:518-531 op_gemm: C[i, j] (row stride ldc) = (accumulate ? ld(C[i, j]) : 0)
 * then, p ascending over the whole of k, acc = fma3(ld(A(i, p)), ld(B(p, j)), acc), stored
 * through st: acc = ftz(fma(ftz a, ftz b, acc)), one chain per cell seeded by the flushed old C
 * (or +0).  A(i, p) = a[i a_si + p a_sp], B(p, j) = b[p b_sp + j b_sj]
 * (sequence/ops.mojo:369-392 ld/st/mul/add/sub/fma3; gemm/neural_dispatch.mojo:245-274). */
void orc_seq_gemm(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k, int64_t a_si,
                  int64_t a_sp, int64_t b_sp, int64_t b_sj, int64_t ldc, int accumulate) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float acc = accumulate ? ftz(c[i * ldc + j]) : 0.0f;
      for (int64_t p = 0; p < k; ++p) acc = ftz(fmaf(ftz(a[i * a_si + p * a_sp]), ftz(b[p * b_sp + j * b_sj]), acc));
      c[i * ldc + j] = ftz(acc);
    }
}

/* checks/numerics.mojo:370-408 portable_expf: Cephes single-precision expf (cephes/single/expf.c)
 * with the reduction's multiply-add and the scaling written out as single roundings. */
float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.722835f) return u2f(0x7F800000u);
  if (x < -87.33655f) return 0.0f;
  const float zf = floorf(fmaf(x, 1.4426950408889634f, 0.5f));
  const int32_t kq = (int32_t)zf;
  float r = fmaf(zf, -0.693359375f, x);
  r = fmaf(zf, 2.12194440e-4f, r);
  float q = 1.9875691500e-4f;
  q = fmaf(q, r, 1.3981999507e-3f);
  q = fmaf(q, r, 8.3334519073e-3f);
  q = fmaf(q, r, 4.1665795894e-2f);
  q = fmaf(q, r, 1.6666665459e-1f);
  q = fmaf(q, r, 5.0000001201e-1f);
  const float r2 = r * r;
  float y = fmaf(q, r2, r) + 1.0f;
  const int32_t k1 = kq >> 1, k2 = kq - k1;
  y = y * u2f((uint32_t)(k1 + 127) << 23);
  y = y * u2f((uint32_t)(k2 + 127) << 23);
  if (y < 1.1754943508222875e-38f) return 0.0f;
  return y;
}

/* checks/numerics.mojo:1025-1037: flushed operands, one correctly rounded division, flushed result */
float orc_divf(float a, float b) { return ftz(ftz(a) / ftz(b)); }

/* checks/numerics.mojo:1079-1085 portable_sigmoidf: 1 / (1 + expf(-x)) */
float orc_sigmoidf(float x) {
  if (x != x) return x;
  return orc_divf(1.0f, orc_expf(-x) + 1.0f);
}

/* checks/numerics.mojo:1190-1222 portable_tanhf: Cephes single-precision tanhf with the input
 * flushed and the sign of zero kept; saturation above 0x42317218 */
float orc_tanhf(float x_in) {
  const float xx = ftz(x_in);
  if (xx != xx) return xx;
  if (xx == 0.0f) return xx;
  const float x = fabsf(xx);
  if (x > u2f(0x42317218u)) return xx < 0.0f ? -1.0f : 1.0f;
  if (x >= 0.625f) {
    const float e = orc_expf(x + x);
    const float q = orc_divf(2.0f, e + 1.0f);
    const float z = 1.0f - q;
    return xx < 0.0f ? -z : z;
  }
  const float zs = x * x;
  float p = -5.70498872745e-3f;
  p = fmaf(p, zs, 2.06390887954e-2f);
  p = fmaf(p, zs, -5.37397155531e-2f);
  p = fmaf(p, zs, 1.33314422036e-1f);
  p = fmaf(p, zs, -3.33332819422e-1f);
  const float pz = p * zs;
  return fmaf(pz, xx, xx);
}

/* sequence/act_values.mojo:60-85 act_value / act_bwd_value; codes: 0 identity, 1 logistic,
 * 2 tanh, 3 relu, 4 softmax (no branch: the word is left) */
float orc_act_value(float z, int code) {
  if (code == 1) return ftz(orc_sigmoidf(z));
  if (code == 2) return ftz(orc_tanhf(z));
  if (code == 3) return z > 0.0f ? z : 0.0f;
  return z;
}

float orc_act_bwd_value(float d, float z, int code) {
  if (code == 1) return ftz(ftz(ftz(d * z) * ftz(1.0f - z)));
  if (code == 2) return ftz(d * ftz(1.0f - ftz(z * z)));
  if (code == 3 && z == 0.0f) return 0.0f;
  return d;
}

/* The product's followers over its stored cells (gemm/checks/gemm_identical.mojo:8891-8912):
 * kind 3 PLUS_BIAS  ftz(ftz(cell) + ftz(p[j]))
 * kind 4 BIAS_ACT   ftz(act_value(ftz(ftz(cell) + ftz(p[j])), act))
 * kind 5 ACT_BWD    ftz(act_bwd_value(ftz(cell), ftz(p[i n + j]), act))   (p dense, row stride n)
 * c has row stride ldc. */
void orc_epilogue(float* c, int64_t ldc, int64_t m, int64_t n, int kind, const float* p, int act) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      const float cell = ftz(c[i * ldc + j]);
      float y = cell;
      if (kind == 3) y = ftz(cell + ftz(p[j]));
      else if (kind == 4) y = ftz(orc_act_value(ftz(cell + ftz(p[j])), act));
      else if (kind == 5) y = ftz(orc_act_bwd_value(cell, ftz(p[i * n + j]), act));
      c[i * ldc + j] = y;
    }
}

/* elementwise maps of the functions above, for the tests: which = 0 expf, 1 sigmoidf, 2 tanhf,
 * 3 divf(1, x) */
void orc_map(float* out, const float* in, int64_t count, int which) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    const float x = in[i];
    out[i] = which == 0 ? orc_expf(x) : which == 1 ? orc_sigmoidf(x) : which == 2 ? orc_tanhf(x) : orc_divf(1.0f, x);
  }
}

// Host dispatch of mojolearn.identical.gemm.fp32.v1 on gfx950: which kernel, workspace layout,
// launches; plus the bf16 conversions.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <string>

#include "act.h"
#include "contract.h"
#include "device_common.h"
#include "gemv.h"
#include "kernels.h"
#include "mfma.h"

namespace mlg {

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
static int64_t gemv_cols(int bt, int op, bool full = false) { return 64 * gv_cpl(bt, op == OP_NT, full); }
// Columns of a column group of the matrix-core kernels (OP_NN, 4 x 4 and 16 x 16 shapes).
static int64_t mf16_cols(int bt) { return 64 * mf_cpl(bt); }
// The narrowest column group any skinny kernel of this weight type and op uses: the completion
// counters a workspace carries cover it, whichever kernel the product's pointers then pick.
static int64_t counter_cols(int bt, int op) {
  return op == OP_NT ? gemv_cols(bt, op)
                     : std::min({gemv_cols(bt, op), gemv_cols(bt, op, true), mf16_cols(bt)});
}

// The skinny-M path takes OP_NN products with at most GV_MAXM float32 rows (dense operands,
// chains from +0).
static bool use_gemv(const GemmProblem& p) {
  if (p.seq || p.epi >= EPI_BIAS_ACT || p.a_type != T_F32 || p.m < 1 || p.m > GV_MAXM) return false;
  if (p.op == OP_NN) return true;
  // OP_NT: a lane's byte offset into a 64-row block of W is 32-bit
  return p.op == OP_NT && 64 * p.k * elem_bytes(p.b_type) + 512 < (int64_t(1) << 31);
}

// Stored shape of an operand of the MFMA path: [rows][cols] elements.
static void stored_shape(const GemmProblem& p, bool is_a, int64_t& rows, int64_t& cols) {
  if (is_a) {
    if (p.op == OP_TN) { rows = p.k; cols = p.m; } else { rows = p.m; cols = p.k; }
  } else {
    if (p.op == OP_NT) { rows = p.n; cols = p.k; } else { rows = p.k; cols = p.n; }
  }
}

// Element strides (row, column) of a stored operand: the caller's, or dense.
static void stored_strides(const GemmProblem& p, bool is_a, int64_t cols, int64_t& rs, int64_t& cs) {
  rs = cols;
  cs = 1;
  if (p.strided) {
    rs = is_a ? p.a_rs : p.b_rs;
    cs = is_a ? p.a_cs : p.b_cs;
  }
}

// Whether the MFMA path loads an operand where it lies: unit column stride, 16-byte aligned
// base and rows, and a row stride whose 32-row span stays below the loads' offset range.
static bool in_place(const GemmProblem& p, bool is_a) {
  int64_t rows, cols, rs, cs;
  stored_shape(p, is_a, rows, cols);
  stored_strides(p, is_a, cols, rs, cs);
  const int eb = elem_bytes(is_a ? p.a_type : p.b_type);
  const void* base = is_a ? p.a : p.b;
  return cs == 1 && rs > 0 && (rs * eb) % 16 == 0 && (base == nullptr || aligned(base, 16)) &&
         (32 * rs + KT) * eb < (int64_t(1) << 30);
}

// Floats of workspace the MFMA path needs to repack an operand it cannot load in place into
// dense rows of a multiple of 16 bytes (0 when it is loaded in place).
static int64_t repack_floats(const GemmProblem& p, bool is_a) {
  if (in_place(p, is_a)) return 0;
  int64_t rows, cols;
  stored_shape(p, is_a, rows, cols);
  const int eb = elem_bytes(is_a ? p.a_type : p.b_type);
  const int64_t ce = 16 / eb;
  const int64_t pitch = (cols + ce - 1) / ce * ce;
  return (rows * pitch * eb + 255) / 256 * 64;  // 256-byte granules
}

static int64_t round_floats(int64_t f) { return (f + 63) / 64 * 64; }

// A tile product whose tiles fill whole rounds of the CUs and leave a short last round (the LM
// head: 4 x 393 tiles on 256 CUs is 6 rounds and 36 tiles) runs as two column ranges: the
// columns of the whole rounds as they are (p1), and the remaining columns (p2) with their leaves
// split into aligned groups, so the last round is many short workgroups folded afterwards in the
// contract's order.  A cell's leaves and tree are the same in either range: the bits are the
// unsplit product's.  Only for operands loaded in place, one group per tile in the unsplit
// product, and a grouped tail of at most half a round's time.
static bool tail_split(const GemmProblem& p, int64_t P, int num_cus, GemmProblem& p1, GemmProblem& p2) {
  if (p.whole || p.seq || p.seed || P < 2 || num_cus <= 0) return false;
  const int64_t tm = (p.m + BM - 1) / BM, tn = (p.n + BN - 1) / BN, T = tm * tn;
  if (T <= num_cus || pick_group(P, T, num_cus) < P) return false;
  if (!in_place(p, true) || !in_place(p, false)) return false;
  const int64_t tn1 = T / num_cus * num_cus / tm;  // column tiles of the whole rounds
  if (tn1 < 1 || tn1 >= tn) return false;
  const int64_t r = tm * (tn - tn1);  // tail tiles
  const int64_t gsz = pick_group(P, r, num_cus);
  const int64_t ng = (P + gsz - 1) / gsz;
  if (ng < 2 || 2 * ((r * ng + num_cus - 1) / num_cus) > ng) return false;  // tail <= half a round
  const int64_t n1 = tn1 * BN;
  int64_t rows, cols, a_rs, a_cs, b_rs, b_cs;
  stored_shape(p, true, rows, cols);
  stored_strides(p, true, cols, a_rs, a_cs);
  stored_shape(p, false, rows, cols);
  stored_strides(p, false, cols, b_rs, b_cs);
  p1 = p;
  p1.whole = 1;
  p1.strided = 1;
  p1.a_rs = a_rs; p1.a_cs = a_cs; p1.b_rs = b_rs; p1.b_cs = b_cs;
  p1.ldc = p.ldc > 0 ? p.ldc : p.n;
  p2 = p1;
  p1.n = n1;
  p2.n = p.n - n1;
  if (p.c) p2.c = p.c + n1;  // (sizing queries pass no operands)
  // B's columns n1.. : later columns of each stored row (NN, TN) or later stored rows (NT)
  const int64_t boff = p.op == OP_NT ? n1 * b_rs : n1 * b_cs;
  if (p.b) p2.b = static_cast<const char*>(p.b) + boff * elem_bytes(p.b_type);
  else if (boff * elem_bytes(p.b_type) % 16 != 0) return false;
  if (p.scales) p2.scales = p.scales + n1;
  if (p.bias) p2.bias = p.bias + n1;
  return in_place(p1, false) && in_place(p2, false);
}

// Why a product cannot be launched ("" if it can): the fold stack's reach (StackF: the skinny
// kernels' cross-workgroup fold and fold_groups_kernel) and the grid's dimensions.
std::string launch_limit(const GemmProblem& p, int num_cus) {
  const int64_t L = p.leaf > 0 ? p.leaf : leaf_size(p.k);
  const int64_t P = leaf_count(p.k, L);
  if (P < 1 || p.m <= 0 || p.n <= 0) return "";
  if (use_gemv(p)) {
    const int64_t groups = gemv_groups(P);
    const int64_t ncg = (p.n + counter_cols(p.b_type, p.op) - 1) / counter_cols(p.b_type, p.op);
    if (groups > STACK_ROOTS)
      return "more leaf-group roots (" + std::to_string(groups) + ") than the fold stack covers (" +
             std::to_string(STACK_ROOTS) + "); use a larger leaf";
    if (ncg * groups > INT32_MAX) return "more workgroups than one launch holds; use a larger leaf";
    return "";
  }
  GemmProblem p1, p2;
  if (tail_split(p, P, num_cus, p1, p2)) {
    const std::string a = launch_limit(p1, num_cus);
    return a.empty() ? launch_limit(p2, num_cus) : a;
  }
  const int64_t tiles = ((p.m + BM - 1) / BM) * ((p.n + BN - 1) / BN);
  const int64_t gsz = P > 1 ? pick_group(P, tiles, num_cus) : 1;
  const int64_t ng = (P + gsz - 1) / gsz;
  if (ng > TILE_GROUPS)
    return "more leaf groups (" + std::to_string(ng) + ") than a grid column holds (" + std::to_string(TILE_GROUPS) +
           "); use a larger leaf";
  if (tiles > INT32_MAX) return "more tiles than one launch holds";
  return "";
}

int64_t gemm_counter_count(const GemmProblem& p) {
  const int64_t L = p.leaf > 0 ? p.leaf : leaf_size(p.k);
  const int64_t P = leaf_count(p.k, L);
  if (!use_gemv(p) || p.m <= 0 || p.n <= 0 || gemv_groups(P) <= 1) return 0;
  return (p.n + counter_cols(p.b_type, p.op) - 1) / counter_cols(p.b_type, p.op);
}

// Workspace: [completion counters][group roots][A repacked][B repacked], each part 256-byte
// aligned; the counters only for a skinny product folded across workgroups.
int64_t gemm_workspace_floats(const GemmProblem& p, int num_cus) {
  const int64_t L = p.leaf > 0 ? p.leaf : leaf_size(p.k);
  const int64_t P = leaf_count(p.k, L);
  if (P < 1 || p.m <= 0 || p.n <= 0) return 0;
  if (use_gemv(p))
    return gemv_groups(P) > 1 ? round_floats(gemm_counter_count(p)) + gemv_groups(P) * p.m * p.n : 0;
  GemmProblem p1, p2;
  if (tail_split(p, P, num_cus, p1, p2))
    return std::max(gemm_workspace_floats(p1, num_cus), gemm_workspace_floats(p2, num_cus));
  const int64_t tiles = ((p.m + BM - 1) / BM) * ((p.n + BN - 1) / BN);
  const int64_t gsz = P > 1 ? pick_group(P, tiles, num_cus) : 1;
  const int64_t ng = (P + gsz - 1) / gsz;
  return (ng > 1 ? round_floats(ng * p.m * p.n) : 0) + repack_floats(p, true) + repack_floats(p, false);
}

hipError_t run_gemm(const GemmProblem& p, float* ws, int num_cus, hipStream_t stream, unsigned* route) {
  if (p.m <= 0 || p.n <= 0) return hipSuccess;
  const int64_t L = p.leaf > 0 ? p.leaf : leaf_size(p.k);
  const int64_t P = leaf_count(p.k, L);
  const int64_t ldc = p.ldc > 0 ? p.ldc : p.n;
  // the store's follower: the activation ones, or the bias
  const int epi = p.epi >= EPI_BIAS_ACT ? p.epi : (p.bias ? EPI_PLUS_BIAS : EPI_NONE);
  const float* epi_p = p.epi >= EPI_BIAS_ACT ? p.epi_p : p.bias;
  if (P == 0) {
    if (route) { *route |= ROUTE_ZERO_K; return hipSuccess; }
    return launch_fold_groups(p.c, ldc, nullptr, p.m, p.n, 0, epi, epi_p, p.act, stream);
  }
  if (use_gemv(p)) {
    GemvArgs v;
    v.c = p.c; v.w = p.b; v.scales = p.scales; v.bias = p.bias;
    v.m = p.m; v.n = p.n; v.k = p.k; v.leaf = L; v.nleaves = P;
    v.ngroups = gemv_groups(P);
    v.ncg = (p.n + gemv_cols(p.b_type, p.op) - 1) / gemv_cols(p.b_type, p.op);
    // workspace: the column groups' completion counters, then the group roots
    v.counter = reinterpret_cast<unsigned int*>(ws);
    v.ws = ws ? ws + round_floats(gemm_counter_count(p)) : nullptr;
    const int eb = elem_bytes(p.b_type);
    int vec;
    if (p.op == OP_NT) {
      // 16-byte loads need a 16-byte-aligned base, rows and leaf starts
      vec = aligned(p.b, 16) && (p.k * eb) % 16 == 0 && (P == 1 || (L * eb) % 16 == 0) ? 4 : 3;
    } else {
      // word loads need 4-byte rows and base, and GV_CH rows within a 31-bit buffer offset
      vec = ((p.n * eb) % 4 == 0) && aligned(p.b, 4) && (int64_t)GV_CH * p.n * eb < (int64_t(1) << 31) ? 1 : 0;
      if (vec && L == GV_CH && p.k % GV_CH == 0) vec = 2;
    }
    const bool mfma = p.op == OP_NN && vec == 2 && p.m >= GV_MFMA4_MIN_M && aligned(p.a, 16) &&
                      16 * p.k * 4 < (int64_t(1) << 31);
    const bool four = p.m <= GV_MFMA4_MAX_M;
    if (mfma) v.ngroups = (P + (four ? MF4_LEAVES : MF_LEAVES) - 1) / (four ? MF4_LEAVES : MF_LEAVES);
    // whole leaves (vec 2): int8 on 16-bit lanes, and for the decode rows (m <= 2) eight leaves
    // a workgroup when that still leaves a workgroup for every CU
    int leaves = GV_LEAVES;
    if (p.op == OP_NN && !mfma && vec == 2) {
      v.ncg = (p.n + gemv_cols(p.b_type, p.op, true) - 1) / gemv_cols(p.b_type, p.op, true);
      const int64_t wide = (P + GV_WIDE_LEAVES - 1) / GV_WIDE_LEAVES;
      if (p.m <= 2 && v.ncg * wide >= num_cus) {
        leaves = GV_WIDE_LEAVES;
        v.ngroups = wide;
      }
    }
    if (route) {
      *route |= p.op == OP_NT ? ROUTE_GEMV_NT : (mfma ? (four ? ROUTE_MFMA4 : ROUTE_MFMA16) : ROUTE_GEMV_NN);
      if (v.ngroups > 1) *route |= ROUTE_GEMV_GROUPS;
      return hipSuccess;
    }
    if (gemv_groups(P) > 1 && ws == nullptr) return hipErrorInvalidValue;
    if (p.op == OP_NT)
      return launch_gemv_nt(v, static_cast<const float*>(p.a), p.b_type, p.m, vec - 3,
                            dim3((unsigned)(v.ncg * v.ngroups)), stream);
    if (mfma) {
      // the matrix-core kernels: fewer, wider groups (at most the workspace sized for
      // gemv_groups) and their own column groups (at least counter_cols wide)
      v.ncg = (p.n + mf16_cols(p.b_type) - 1) / mf16_cols(p.b_type);
      const dim3 mgrid((unsigned)(v.ncg * v.ngroups));
      if (four) return launch_gemv_mfma4_nn(v, static_cast<const float*>(p.a), p.b_type, p.m, mgrid, stream);
      return launch_gemv_mfma_nn(v, static_cast<const float*>(p.a), p.b_type, mgrid, stream);
    }
    return launch_gemv_nn(v, static_cast<const float*>(p.a), p.b_type, p.m, vec, leaves,
                          dim3((unsigned)(v.ncg * v.ngroups)), stream);
  }
  GemmProblem p1, p2;
  if (tail_split(p, P, num_cus, p1, p2)) {
    if (route) *route |= ROUTE_TAIL_SPLIT;
    hipError_t e = run_gemm(p1, ws, num_cus, stream, route);
    return e != hipSuccess ? e : run_gemm(p2, ws, num_cus, stream, route);
  }
  GemmArgs g;
  g.c = p.c; g.a = p.a; g.b = p.b; g.scales = p.scales; g.bias = p.bias; g.ws = ws;
  g.epi = epi; g.epi_p = epi_p; g.act = p.act;
  g.m = p.m; g.n = p.n; g.k = p.k; g.leaf = L; g.nleaves = P;
  g.ldc = ldc;
  g.seed = p.seed && P == 1 ? 1 : 0;
  if (p.seed && P != 1) return hipErrorInvalidValue;
  const int64_t tm = (p.m + BM - 1) / BM, tn = (p.n + BN - 1) / BN;
  g.tiles_m = (int)tm;
  g.tiles_n = (int)tn;
  const int64_t gsz = P > 1 ? pick_group(P, tm * tn, num_cus) : 1;
  g.group = gsz;
  g.ngroups = (P + gsz - 1) / gsz;
  const int64_t ra = repack_floats(p, true), rb = repack_floats(p, false);
  if (route) {
    *route |= ROUTE_TILE;
    if (gsz > 1) *route |= ROUTE_TILE_STACK;
    if (g.ngroups > 1) *route |= ROUTE_FOLD;
    if (ra > 0 || rb > 0) *route |= ROUTE_REPACK;
    return hipSuccess;
  }
  // workspace: [group roots][A repacked][B repacked], each part 256-byte aligned
  float* wsp = ws + (g.ngroups > 1 ? round_floats(g.ngroups * p.m * p.n) : 0);
  if ((g.ngroups > 1 || ra > 0 || rb > 0) && ws == nullptr) return hipErrorInvalidValue;
  for (int which = 0; which < 2; ++which) {
    const bool is_a = which == 0;
    int64_t rows, cols;
    stored_shape(p, is_a, rows, cols);
    const int eb = elem_bytes(is_a ? p.a_type : p.b_type);
    const int64_t ce = 16 / eb;
    int64_t rs, cs;
    stored_strides(p, is_a, cols, rs, cs);
    const void* src = is_a ? p.a : p.b;
    int64_t pitch = rs, bytes = ((rows - 1) * rs + cols) * eb;
    if ((is_a ? ra : rb) > 0) {
      pitch = (cols + ce - 1) / ce * ce;
      bytes = rows * pitch * eb;
      // one load instruction spans at most 32 stored rows (int8, index-major), and a slice
      // advances a k-major operand by KT rows: both below 2^30 bytes keep the loads' lane and
      // scalar offsets below 2^31
      if ((32 * pitch + KT) * eb >= (int64_t(1) << 30)) return hipErrorInvalidValue;
      hipError_t e = launch_repack((char*)wsp, (const char*)src, rows, cols, pitch, eb, rs, cs, stream);
      if (e != hipSuccess) return e;
      src = wsp;
      wsp += is_a ? ra : rb;
    }
    if (is_a) { g.a = src; g.a_pitch = pitch; g.a_bytes = bytes; }
    else { g.b = src; g.b_pitch = pitch; g.b_bytes = bytes; }
  }
  dim3 grid((unsigned)(tm * tn), (unsigned)g.ngroups);
  hipError_t e = launch_mfma(g, p.op, p.a_type, p.b_type, grid, stream);
  if (e != hipSuccess || g.ngroups == 1) return e;
  return launch_fold_groups(p.c, ldc, ws, p.m, p.n, g.ngroups, epi, epi_p, p.act, stream);
}

// ---------------------------------------------------------------------------
// Decode-packed int8 weights (gemv_packed.hip)

static int64_t pk_groups(int64_t n) { return (n + PK_GROUP_COLS - 1) / PK_GROUP_COLS; }

// The packed product on the matrix cores: 3 <= m <= 16, x on the 16-byte grid (its blocks are
// loaded straight into LDS in 16-byte chunks) and addressed in 31 bits.
static bool pk_mfma(int64_t m, int64_t k, const float* x) {
  return m >= PK_MFMA_MIN_M && m <= GV_MAXM && aligned(x, 16) && m * k * 4 <= INT32_MAX;
}

// Waves a workgroup of the packed product: the whole-column workgroups (32 leaves) when the
// launch still holds a workgroup for three of every four CUs, else 4-leaf groups.  The VALU
// kernel takes whole columns only for the decode rows (m <= 2: more rows would spill the x
// values a 16-wave workgroup keeps in scalar registers); the matrix-core one at every m.
static int pk_waves(int64_t m, int64_t n, int64_t k, bool mfma, int num_cus) {
  const int64_t P = k / GV_CH, whole = 2 * PK_WAVES_WHOLE;
  const bool fills = pk_groups(n) * ((P + whole - 1) / whole) * 4 >= 3 * (int64_t)num_cus;
  return (m <= 2 || mfma) && fills ? PK_WAVES_WHOLE : PK_WAVES_SPLIT;
}

static int64_t pk_ngroups(int64_t k, int waves) { return (k / GV_CH + 2 * waves - 1) / (2 * waves); }

int64_t int8w_packed_bytes(int64_t k, int64_t n) {
  if (k <= 0 || n <= 0 || k % GV_CH != 0 || k / GV_CH > MAX_LEAVES) return -1;
  return k * PK_GROUP_COLS * pk_groups(n);
}

hipError_t run_int8w_pack(void* dst, const int8_t* codes, int64_t k, int64_t n, hipStream_t stream) {
  if (int8w_packed_bytes(k, n) < 0 || !dst || !codes || !aligned(dst, 16)) return hipErrorInvalidValue;
  return launch_int8w_pack(dst, codes, k, n, stream);
}

// The workspace is sized for the narrowest workgroups (the most group roots), whichever width
// the device's CU count then picks.
int64_t gemv_packed_counter_count(int64_t m, int64_t n, int64_t k) {
  if (int8w_packed_bytes(k, n) < 0 || m < 1 || m > GV_MAXM || pk_ngroups(k, PK_WAVES_SPLIT) <= 1) return 0;
  return pk_groups(n);
}

int64_t gemv_packed_workspace_floats(int64_t m, int64_t n, int64_t k) {
  const int64_t cnt = gemv_packed_counter_count(m, n, k);
  return cnt > 0 ? round_floats(cnt) + pk_ngroups(k, PK_WAVES_SPLIT) * m * n : 0;
}

std::string gemv_packed_limit(int64_t m, int64_t n, int64_t k, const void* packed) {
  if (m < 1 || m > GV_MAXM) return "m must be 1 .. 16";
  if (int8w_packed_bytes(k, n) < 0) return "k must be a positive multiple of 128 with at most 1024 leaves, n >= 1";
  if (packed && !aligned(packed, 16)) return "the packed weights must be 16-byte aligned";
  // the loads' leaf stride (ncg KB) in a 32-bit offset, and the grid
  if (pk_groups(n) * 1024 + 1024 > INT32_MAX) return "n too large for the packed product";
  if (pk_groups(n) * pk_ngroups(k, PK_WAVES_SPLIT) > INT32_MAX) return "more workgroups than one launch holds";
  return "";
}

hipError_t run_gemv_packed(float* c, const float* x, const void* packed, const float* scales, const float* bias,
                           int64_t m, int64_t n, int64_t k, float* ws, int num_cus, hipStream_t stream) {
  if (!gemv_packed_limit(m, n, k, packed).empty() || !c || !x || !packed || !scales) return hipErrorInvalidValue;
  const bool mfma = pk_mfma(m, k, x);
  const int waves = pk_waves(m, n, k, mfma, num_cus);
  GemvArgs v;
  v.c = c; v.w = packed; v.scales = scales; v.bias = bias;
  v.m = m; v.n = n; v.k = k; v.leaf = GV_CH; v.nleaves = k / GV_CH; v.ncg = pk_groups(n);
  v.ngroups = pk_ngroups(k, waves);
  v.counter = reinterpret_cast<unsigned int*>(ws);
  v.ws = ws ? ws + round_floats(gemv_packed_counter_count(m, n, k)) : nullptr;
  if (v.ngroups > 1 && ws == nullptr) return hipErrorInvalidValue;
  const dim3 grid((unsigned)(v.ncg * v.ngroups));
  return mfma ? launch_gemv_packed_mfma(v, x, waves, grid, stream) : launch_gemv_packed(v, x, waves, grid, stream);
}

// Zero `count` 32-bit words (the completion counters of a skinny product) with a kernel: a
// memset node would not be safe in a captured graph.
__global__ void zero_words_kernel(unsigned int* p, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < count) p[i] = 0u;
}

hipError_t run_zero_words(unsigned int* p, int64_t count, hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(zero_words_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream, p, count);
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

// gemm/f16_widen.mojo:12-37 f16_bits_to_f32_bits: exact, integer operations only; a subnormal
// float16 renormalized into a normal float32, every NaN keeping its sign and payload.
__global__ void f16_widen_kernel(float* out, const uint16_t* in, int64_t count) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= count) return;
  const uint32_t h = in[i];
  const uint32_t s = (h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1Fu;
  uint32_t m = h & 0x03FFu;
  uint32_t w;
  if (e == 0u) {
    if (m == 0u) {
      w = s;
    } else {
      const uint32_t shift = (uint32_t)__builtin_clz(m) - 21u;  // shifts until bit 10 is set
      m = (m << shift) & 0x03FFu;
      w = s | ((113u - shift) << 23) | (m << 13);
    }
  } else if (e == 31u) {
    w = s | 0x7F800000u | (m << 13);
  } else {
    w = s | ((e + 112u) << 23) | (m << 13);
  }
  out[i] = __uint_as_float(w);
}

hipError_t run_f16_widen(float* out, const uint16_t* in, int64_t count, hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  hipLaunchKernelGGL(f16_widen_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, stream, out, in, count);
  return hipGetLastError();
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

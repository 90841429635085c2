/*
 * mlgemm.h -- C ABI of libmlgemm.so, the MI355X (gfx950) implementation of
 * mojolearn's identical-mode FP32 GEMM, profile mojolearn.identical.gemm.fp32.v1.
 *
 * Plain pointers and sizes only.  All functions are thread-safe; errors are reported
 * through the sink (linalg_native_v1) or mlg_last_error() (device entries).
 */
#ifndef MLGEMM_H
#define MLGEMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error sink of the native op table: (context, UTF-8 message pointer, byte length).
 * Replaces the reference's NativeDescriptorError, core/native_descriptor_abi.mojo:7-10. */
typedef void (*mlg_sink_t)(int64_t ctx, int64_t utf8_ptr, int64_t len);

/*
 * The op table entry, same signature, op numbering and error protocol as the reference's
 * `linalg_native_v1` (gemm/linalg_dispatch.mojo:78-89, ops :14-75).  All addresses are HOST
 * pointers owned by the caller, row-major and contiguous; the call uploads, computes,
 * downloads (NaN words canonicalized to 0x7FC00000) and drains before it returns.
 * Returns 0 and writes *(int64_t*)result, or calls sink(err_ctx, msg, len) once and
 * returns 1.  `floats`/`n_floats` must be 0 (as in the reference).
 *
 *   op  addrs                       ints                       result
 *   0   [c, a, b]                   [m, n, k, op]              m*n      gemm (gemm/linalg_native.mojo:170-197)
 *   1   [c, a, b_u16]               [m, n, k, op, a_bf16]      m*n      gemm_bf16 (gemm/linalg_native.mojo:199-256)
 *   8   [out_u16, x_f32]            [count]                    count    to_bf16 (L-2)
 *   9   [out_f32, bits_u16]         [count]                    count    from_bf16 (L-1)
 *   11  []                          []                         1        numeric mode (identical)
 *   12  []                          []                         1        fp32 profile version
 *   13  []                          []                         1        low-bit profile version
 *   14  []                          []                         1        int15 profile version
 *   Extensions of this build (no reference op; numbered after the reference's 0-14):
 *   15  [c, a, codes_i8, scales]    [m, n, k, op]              m*n      int8 weight x fp32 per-output-
 *                                                                       channel scale: B_eff[p,j] =
 *                                                                       ftz(f32(code) * ftz(scale[j]))
 *   16  [c, a, b, bias]             [m, n, k, op]              m*n      gemm then nn.Linear bias,
 *                                                                       Y = ftz(ftz(C) + ftz(bias[j]))
 *                                                                       (transformer/impl/llama/
 *                                                                       modeling_llama.mojo:3979-3989)
 *   2   [c, qa, ea, qb, eb]         [m, n, k]                  m*n      gemm_int8, profile int8i32.v1,
 *                                                                       OP_NT: codes int8 row-major, one
 *                                                                       int32 exponent per row; k <= 131072
 *                                                                       (gemm/linalg_native.mojo:258-321)
 *   3   [codes_i8, exps_i32, x]     [rows, cols]               rows*cols quantize_int8 (L-3, L-4; :323-357)
 *   4   [y_f32, codes_i8, exps_i32] [rows, cols]               rows*cols dequantize_int8 (L-6; :359-393)
 *   5   [c, ah, al, ea, bh, bl, eb] [m, n, k]                  m*n      gemm_int15, profile int15i64.v1,
 *                                                                       OP_NT: two int8 planes per operand
 *                                                                       (code = hi*128 + lo), one int32
 *                                                                       exponent per row; k <= 65536
 *                                                                       (gemm/linalg_native.mojo:395-442)
 *   6   [hi, lo, exps, x]           [rows, cols]               rows*cols quantize_int15 (W-1..W-3; :444-476)
 *   7   [y, hi, lo, exps]           [rows, cols]               rows*cols dequantize_int15 (W-6, W-7; :478-510)
 *  10   [f32_out, f16_bits]         [count]                    count    from_f16, exact (:564-576)
 */
int64_t linalg_native_v1(int64_t op, int64_t addrs, int64_t n_addrs, int64_t ints, int64_t n_ints,
                         int64_t floats, int64_t n_floats, int64_t result, int64_t err_ctx,
                         mlg_sink_t sink);

/* The ABI name the reference wraps in its PyCapsule ("mojolearn.linalg.v1",
 * gemm/linalg_dispatch.mojo:10). */
const char* mlg_abi_name(void);

/*
 * Device-pointer entries (the model for them: the reference's device-level
 * identical_gemm_into / identical_gemm_leaf_ptr_into, gemm/checks/gemm_identical.mojo:6062-6144,
 * gemm/neural_dispatch.mojo:245-320).  All buffers are DEVICE pointers (e.g. PyTorch-ROCm
 * data_ptr()), row-major and contiguous in the layout of `op` (0 NN, 1 NT, 2 TN).  The
 * work is enqueued on `stream` (a hipStream_t; NULL = the null stream) and the call
 * returns without waiting.  `bias` may be NULL.  `leaf` is the k-leaf size; 0 selects
 * the contract's (gemm/contract.mojo:173-214), k selects the one-chain sequence-executor
 * word (gemm/neural_dispatch.mojo:245-320).  Output NaN words are 0x7FC00000.
 * Return 0 on success; otherwise mlg_last_error() holds the message.
 */
int mlg_gemm_f32(float* c, const float* a, const float* b, const float* bias, int64_t m,
                 int64_t n, int64_t k, int32_t op, int64_t leaf, void* stream);

/* bf16-stored B (and optionally A): widened exactly (bits << 16) at the tile load
 * (bf16f32.v1, gemm/IDENTICAL_LOWBIT_CONTRACT.md L-1; reference device entry
 * identical_gemm_bf16w_into, gemm/checks/gemm_lowbit.mojo:369-395). */
int mlg_gemm_bf16w(float* c, const void* a, const uint16_t* b, const float* bias, int64_t m,
                   int64_t n, int64_t k, int32_t op, int32_t a_is_bf16, int64_t leaf, void* stream);

/* int8-stored B with one fp32 scale per output column j (this build's extension; the
 * reference's int8 rows use power-of-two exponents, checks/numerics.mojo:1665-1671):
 * B_eff[p,j] = ftz(f32(code[p,j]) * ftz(scales[j])), dequantized in the tile load. */
int mlg_gemm_int8w(float* c, const float* a, const int8_t* codes, const float* scales,
                   const float* bias, int64_t m, int64_t n, int64_t k, int32_t op, int64_t leaf,
                   void* stream);

/* The general device entry with a caller-supplied workspace: it allocates no device memory
 * and never synchronizes (so a caller may capture it in a HIP graph).
 * a_type: 0 float32, 1 bf16 bits; b_type: 0 float32, 1 bf16 bits, 2 int8 codes (with
 * `scales`, one per output column).  `workspace` must hold mlg_gemm_workspace_bytes_for()
 * bytes (0 bytes for most shapes; NULL is then accepted).  Its first mlg_gemm_counter_bytes()
 * bytes are completion counters: zero them before the workspace's first product; every
 * product leaves them zero, so a workspace that serves one product shape needs no clearing
 * between calls (a workspace that served another shape must be zeroed again).  Calls sharing
 * one workspace must be ordered (one stream).  Same semantics as mlg_gemm_f32/bf16w/int8w
 * otherwise.  (The reference's GemmWorkspace.run, gemm/checks/gemm_identical.mojo:10712-10888.) */
int mlg_gemm_ws(float* c, const void* a, const void* b, const float* scales, const float* bias,
                int64_t m, int64_t n, int64_t k, int32_t op, int32_t a_type, int32_t b_type,
                int64_t leaf, void* workspace, int64_t workspace_bytes, void* stream);

/* mlg_gemm_ws with no workspace argument, for callers that cannot allocate (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The workspace is the library's own scratch array, 32 MiB per GPU (a static device
 * array, held from the library's load on that GPU until the process ends); a product that needs
 * more (mlg_gemm_workspace_bytes_for) is refused with an error.  The call allocates and frees
 * nothing and never synchronizes; it clears the array's completion counters with a kernel on
 * `stream` first.  Every call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (two streams, two threads, two graphs replayed at once) race and must be ordered by the
 * caller. */
int mlg_gemm_noalloc(float* c, const void* a, const void* b, const float* scales, const float* bias, int64_t m,
                     int64_t n, int64_t k, int32_t op, int32_t a_type, int32_t b_type, int64_t leaf, void* stream);

/* Decode-packed int8 weights.  No counterpart in the reference: its int8 weights are row-major
 * codes converted to float32 before any product (python/mojolearn/lowbit.py:1-20); this is a
 * layout of this build's int8-weight decode path (mlg_gemm_int8w / mlg_gemm_ws with b_type 2,
 * op NN), for callers that keep a weight resident across many decode steps and can rearrange
 * it once.  codes[k][n] (k a positive multiple of 128 with at most 1024 leaves of 128, n >= 1)
 * becomes a copy of mlg_int8w_packed_bytes(k, n) = k * 64 * ceil(n / 64) bytes in which code
 * (p, j), biased to the unsigned byte code + 128, sits at ((s * P + t) * G + g) * 1024 + l * 16 + i,
 * with P = k / 128 leaves,
 * t = p / 128, s = (p % 128) / 16, i = p % 16, G = ceil(n / 64) groups, g = j / 64, l = j % 64
 * (columns past n are zero codes): sixteen rows of one column are one 16-byte word, a 64-column
 * group's block is one 1 KB chunk, and block s of every leaf is one contiguous slab.
 * mlg_int8w_pack writes the copy (dst 16-byte aligned) on `stream`; -1 / an error for a shape
 * the layout does not take. */
int64_t mlg_int8w_packed_bytes(int64_t k, int64_t n);
int mlg_int8w_pack(void* dst, const int8_t* codes, int64_t k, int64_t n, void* stream);

/* C[m][n] = X[m][k] . W_deq (+ bias) from a decode-packed W, 1 <= m <= 16: the same bits as
 * mlg_gemm_ws(c, x, codes, scales, bias, m, n, k, op 0, a_type 0, b_type 2, leaf 0, ...) on the
 * row-major codes (the contract's 128-step leaves, chains, tree, bias and store).  `workspace`
 * holds mlg_gemv_int8w_packed_workspace_bytes(m, n, k) bytes (0 when k <= 512; NULL then
 * accepted; at K = 4096 on a GPU that the launch fills, no byte of it is used); its first mlg_gemv_int8w_packed_counter_bytes(m, n, k) bytes
 * are completion counters, zeroed before its first product and left zero by every product (as
 * for mlg_gemm_ws).  Calls sharing a workspace must be ordered.  -1 from the size queries for a
 * shape the entry does not take. */
int64_t mlg_gemv_int8w_packed_workspace_bytes(int64_t m, int64_t n, int64_t k);
int64_t mlg_gemv_int8w_packed_counter_bytes(int64_t m, int64_t n, int64_t k);
int mlg_gemv_int8w_packed(float* c, const float* x, const void* packed, const float* scales, const float* bias,
                          int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes, void* stream);

/* Bytes of workspace mlg_gemm_ws needs for this product on the current device, for operands
 * a, b at these addresses (an operand the tile kernel cannot load in place -- base not 16-byte
 * aligned, rows not a multiple of 16 bytes -- is repacked into the workspace); -1 on error.
 * (identical_gemm_workspace_max_floats, gemm/checks/gemm_identical.mojo:10789-10844.) */
int64_t mlg_gemm_workspace_bytes_for(const void* a, const void* b, int64_t m, int64_t n, int64_t k, int32_t op,
                                     int32_t a_type, int32_t b_type, int64_t leaf);

/* The same for operands that are 16-byte aligned with rows of a multiple of 16 bytes. */
int64_t mlg_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int32_t op, int32_t a_type,
                                 int32_t b_type, int64_t leaf);

/* Bytes of completion counters at the start of that workspace (0 for most products). */
int64_t mlg_gemm_counter_bytes(int64_t m, int64_t n, int64_t k, int32_t op, int32_t a_type, int32_t b_type,
                               int64_t leaf);

/* Which kernels this product dispatches to, as bits (nothing launched, no operand read;
 * num_cus 0 = the current device's count, > 0 = that count, no device needed):
 *   1 gemm_mfma_kernel  2 fold_groups_kernel after it  4 gemv_nn_kernel  8 gemv_nt_kernel
 *   16 gemv_mfma4_nn_kernel  32 gemv_mfma_nn_kernel  64 whole rounds + grouped tail
 *   128 repack first  256 k = 0 (+0 stored)  512 a tile folds several leaves itself
 *   1024 a skinny product folded across workgroups.
 * -1 on error.  (The role of the reference's choose_gemm_plan, gemm_identical.mojo:4604-4801.) */
int64_t mlg_gemm_route(const void* a, const void* b, int64_t m, int64_t n, int64_t k, int32_t op, int32_t a_type,
                       int32_t b_type, int64_t leaf, int32_t num_cus);

/*
 * The caller-partition and sequence-executor words on strided operand views (device pointers,
 * enqueued on `stream`):  A_eff[i, p] = a[i a_si + p a_sp],  B_eff[p, j] = b[p b_sp + j b_sj].
 *
 * mlg_gemm_leaf_ptr: identical_gemm_leaf_ptr_into (gemm/neural_dispatch.mojo:245-307).  Leaf t
 * is [t leaf, min((t + 1) leaf, k)); each leaf one ascending chain from +0, the leaves folded
 * by the contract's tree; C dense (row stride n), not overlapping a or b.  (leaf, p_count)
 * must partition k: (p_count - 1) leaf < k <= p_count leaf.  m or n of 0 does nothing.
 */
int mlg_gemm_leaf_ptr(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k, int64_t leaf,
                      int64_t p_count, int64_t a_si, int64_t a_sp, int64_t b_sp, int64_t b_sj, void* stream);

/* identical_gemm_leaf_ptr_epi_into (gemm/neural_dispatch.mojo:316-397) with its follower
 * (gemm/checks/gemm_identical.mojo:8884-8912): epi 3 PLUS_BIAS ftz(ftz(cell) + ftz(epi_p[j]));
 * 4 BIAS_ACT ftz(act(ftz(ftz(cell) + ftz(epi_p[j])), epi_i)); 5 ACT_BWD
 * ftz(act_bwd(ftz(cell), ftz(epi_p[i n + j]), epi_i)).  Activation codes: 0 identity,
 * 1 logistic, 2 tanh, 3 relu, 4 softmax (left as is) (sequence/act_values.mojo:23-85).
 * The follower is fused into the product's store (one launch, as the reference fuses its
 * GEMM_EPI_* kinds, gemm/checks/gemm_identical.mojo:9626-9671).  epi_p must not overlap c. */
int mlg_gemm_leaf_ptr_epi(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k, int64_t leaf,
                          int64_t p_count, int64_t a_si, int64_t a_sp, int64_t b_sp, int64_t b_sj, int32_t epi,
                          const float* epi_p, int32_t epi_i, void* stream);

/* op_gemm (sequence/ops.mojo:518-531), the sequence executor's word: C[i ldc + j] =
 * one ascending chain over the whole of k, started from ftz(old C[i ldc + j]) when
 * `accumulate`, else +0.  k may be 0 (C becomes +0, or its flushed self). */
int mlg_seq_gemm(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k, int64_t a_si,
                 int64_t a_sp, int64_t b_sp, int64_t b_sj, int64_t ldc, int32_t accumulate, void* stream);

/* The followers alone over stored cells C[i ldc + j] (op_bias / op_act / op_act_bwd,
 * sequence/ops.mojo:565-569, sequence/act_values.mojo:30-57): epi 0 flushes, 3/4/5 as above. */
int mlg_follow(float* c, int64_t ldc, int64_t m, int64_t n, int32_t epi, const float* epi_p, int32_t epi_i,
               void* stream);

/* L-1 / L-2 conversions on device buffers (checks/numerics.mojo:1548-1574). */
int mlg_bf16_widen(float* out, const uint16_t* in, int64_t count, void* stream);
int mlg_bf16_narrow(uint16_t* out, const float* in, int64_t count, void* stream);

/* Profile mojolearn.identical.gemm.int8i32.v1 on device buffers (gemm/IDENTICAL_LOWBIT_CONTRACT.md
 * L-3..L-7; the reference's device entries identical_gemm_int8_into, quantize_rows_int8_device and
 * dequantize_rows_int8_device, gemm/linalg_native.mojo:258-393).
 * quantize: per row e = floor(log2 absmax) - 6 (0 for an all-zero row) and codes
 *   clamp(rne(ftz(x) * 2^-e), -127, 127), a NaN coding to 0.
 * dequantize: out = ftz(code * 2^e) per row.
 * gemm: OP_NT, C[i][j] = ftz(f32(sum_p qa[i][p] qb[j][p]) * 2^(ea[i] + eb[j])) with the sum exact in
 *   Int32 and converted by the pinned split (L-5); 1 <= k <= 131072.  mlg_gemm_int8i32 takes its
 *   workspace (a repack of operands whose k is not a multiple of 16 or whose base is not 16-byte
 *   aligned; Int32 partial sums when k is split to fill the CUs) from the stream-ordered pool;
 *   mlg_gemm_int8i32_ws takes it from the caller (mlg_gemm_int8i32_workspace_bytes bytes for
 *   these operand addresses on the current device, -1 on error) and allocates nothing. */
int mlg_int8_quantize(int8_t* codes, int32_t* exponents, const float* x, int64_t rows, int64_t cols,
                      void* stream);
int mlg_int8_dequantize(float* out, const int8_t* codes, const int32_t* exponents, int64_t rows,
                        int64_t cols, void* stream);
int mlg_gemm_int8i32(float* c, const int8_t* qa, const int32_t* ea, const int8_t* qb, const int32_t* eb,
                     int64_t m, int64_t n, int64_t k, void* stream);
int64_t mlg_gemm_int8i32_workspace_bytes(const int8_t* qa, const int8_t* qb, int64_t m, int64_t n, int64_t k);
int mlg_gemm_int8i32_ws(float* c, const int8_t* qa, const int32_t* ea, const int8_t* qb, const int32_t* eb,
                        int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes, void* stream);

/* IEEE float16 bits to float32, exact, NaN payloads kept (gemm/f16_widen.mojo:12-37). */
int mlg_f16_widen(float* out, const uint16_t* in, int64_t count, void* stream);

/* Profile mojolearn.identical.gemm.int15i64.v1 on device buffers (gemm/IDENTICAL_LOWBIT_CONTRACT.md
 * section 6, W-1..W-7; the reference's device entries for gemm_int15 / quantize_int15 /
 * dequantize_int15, gemm/linalg_native.mojo:395-510).  A code c in [-16383, 16383] is kept as two
 * int8 planes, hi = floor(c / 128) and lo = c mod 128.
 * quantize: per row e = floor(log2 absmax) - 13 (0 for an all-zero row), c = clamp(rne(ftz(x) *
 *   2^-e), -16383, 16383), a NaN coding to 0 before and after the scaling.
 * dequantize: out = ftz(f32(c) * 2^e) per row.
 * gemm: OP_NT, C[i][j] = ftz(f32(sum_p ca[i][p] cb[j][p]) * 2^(ea[i] + eb[j])), the sum exact in Int64
 *   (three Int32 plane sums, HH 2^14 + MID 2^7 + LL) and converted by W-6's pinned split;
 *   1 <= k <= 65536.  Workspace as for mlg_gemm_int8i32 (repacks of planes whose rows are not a
 *   multiple of 64 codes or 16-byte aligned; Int32 partial sums when k is split). */
int mlg_int15_quantize(int8_t* hi, int8_t* lo, int32_t* exponents, const float* x, int64_t rows, int64_t cols,
                       void* stream);
int mlg_int15_dequantize(float* out, const int8_t* hi, const int8_t* lo, const int32_t* exponents, int64_t rows,
                         int64_t cols, void* stream);
int mlg_gemm_int15i64(float* c, const int8_t* ah, const int8_t* al, const int32_t* ea, const int8_t* bh,
                      const int8_t* bl, const int32_t* eb, int64_t m, int64_t n, int64_t k, void* stream);
int64_t mlg_gemm_int15i64_workspace_bytes(const int8_t* ah, const int8_t* al, const int8_t* bh, const int8_t* bl,
                                          int64_t m, int64_t n, int64_t k);
int mlg_gemm_int15i64_ws(float* c, const int8_t* ah, const int8_t* al, const int32_t* ea, const int8_t* bh,
                         const int8_t* bl, const int32_t* eb, int64_t m, int64_t n, int64_t k, void* workspace,
                         int64_t workspace_bytes, void* stream);

/* The message of the calling thread's last failed mlg_* call ("" if none). */
const char* mlg_last_error(void);

/* Profile metadata: 1 = identical; fp32 profile version; low-bit profile version. */
int64_t mlg_numeric_mode(void);
int64_t mlg_profile_version(void);
int64_t mlg_lowbit_profile_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MLGEMM_H */

// Profile mojolearn.identical.gemm.int8i32.v1 (gemm/IDENTICAL_LOWBIT_CONTRACT.md L-3..L-7):
// launchers of the gfx950 kernels in gemm_q8.hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mlg {

constexpr int64_t INT8_MAX_K = 131072;  // contract L-7: 16129 * k < 2^31

// Per row: e = floor(log2 absmax) - 6 (0 for an all-zero row), codes clamp(rne(ftz(x) 2^-e), +-127).
hipError_t run_q8_quantize(int8_t* codes, int32_t* exps, const float* x, int64_t rows, int64_t cols,
                           hipStream_t stream);

// out[r][c] = ftz(code * 2^exps[r]) (NaN words canonical).
hipError_t run_q8_dequantize(float* out, const int8_t* codes, const int32_t* exps, int64_t rows, int64_t cols,
                             hipStream_t stream);

// Workspace bytes run_q8_gemm needs on a device of `num_cus` CUs: operand rows not a multiple
// of 16 bytes, or a base not 16-byte aligned, are repacked with zero codes; a product whose
// output tiles leave CUs idle splits k and keeps Int32 partial sums.
int64_t q8_workspace_bytes(const void* qa, const void* qb, int64_t m, int64_t n, int64_t k, int num_cus);

// C = qa . qb^T (OP_NT): C[i][j] = ftz(f32(sum_p qa[i][p] qb[j][p]) * 2^(ea[i] + eb[j])), the sum
// exact in Int32 (k <= INT8_MAX_K), f32 by the pinned split conversion; NaN words canonical.
hipError_t run_q8_gemm(float* c, const int8_t* qa, const int32_t* ea, const int8_t* qb, const int32_t* eb,
                       int64_t m, int64_t n, int64_t k, void* ws, int num_cus, hipStream_t stream);

// Profile mojolearn.identical.gemm.int15i64.v1 (contract section 6): codes as two int8 planes,
// hi = floor(c / 128), lo = c mod 128.
constexpr int64_t INT15_MAX_K = 65536;  // W-4: the shared MID accumulator is exact to k = 66052

// Per row: e = floor(log2 absmax) - 13, codes clamp(rne(ftz(x) 2^-e), +-16383) as planes.
hipError_t run_q15_quantize(int8_t* hi, int8_t* lo, int32_t* exps, const float* x, int64_t rows, int64_t cols,
                            hipStream_t stream);
// out[r][c] = ftz(f32(hi * 128 + lo) * 2^exps[r]).
hipError_t run_q15_dequantize(float* out, const int8_t* hi, const int8_t* lo, const int32_t* exps, int64_t rows,
                              int64_t cols, hipStream_t stream);
int64_t q15_workspace_bytes(const void* ah, const void* al, const void* bh, const void* bl, int64_t m, int64_t n,
                            int64_t k, int num_cus);
// C = a . b^T (OP_NT): ftz(f32(sum_p qa[i][p] qb[j][p]) * 2^(ea[i] + eb[j])), the sum exact in
// Int64 (three Int32 plane sums recombined), W-6's conversion; 1 <= k <= INT15_MAX_K.
hipError_t run_q15_gemm(float* c, const int8_t* ah, const int8_t* al, const int32_t* ea, const int8_t* bh,
                        const int8_t* bl, const int32_t* eb, int64_t m, int64_t n, int64_t k, void* ws, int num_cus,
                        hipStream_t stream);

}  // namespace mlg

// Read-only streams over an int8 matrix W[rows][cols]: the memory floors the skinny products are
// measured against (no arithmetic, no output beyond a sink word that is written only if the
// folded bits equal an unlikely value, so no load can be dropped).
//
//  pattern 0: a grid-stride stream of 16-byte loads over the whole matrix in address order --
//             the fastest read of the bytes;
//  pattern 1: the reads of the decode kernel (gemv_nn_kernel, whole 128-row leaves): a wave per
//             128-row leaf and 256-byte column strip, one 32-bit word per lane per row, rows in
//             16-row blocks through a ring three blocks ahead, four leaves a workgroup -- the
//             contract's leaf chains force every leaf of a column to be streamed at once.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "device_common.h"
#include "kernels.h"

namespace mlg {

constexpr int SR_THREADS = 256;
constexpr int SR_LINEAR_WGS = 2048;  // 8 workgroups per CU
constexpr int SR_RB = 16, SR_AHEAD = 3, SR_LEAF = 128;
constexpr uint32_t SR_UNLIKELY = 0x5EED1234u;

static bool sr_aligned(const void* p, int bytes) { return ((uintptr_t)p % (uintptr_t)bytes) == 0; }

__global__ void __launch_bounds__(SR_THREADS) stream_read_linear_kernel(const u4* __restrict__ w, int64_t n16,
                                                                         uint32_t* sink) {
  uint32_t acc = 0;
  for (int64_t i = (int64_t)blockIdx.x * SR_THREADS + threadIdx.x; i < n16; i += (int64_t)gridDim.x * SR_THREADS) {
    const u4 v = __builtin_nontemporal_load(w + i);
    acc = (acc ^ v[0] ^ v[1] ^ v[2] ^ v[3]) * 3u;
  }
  if (acc == SR_UNLIKELY) sink[0] = acc;
}

// grid: (cols / 256) column strips x (rows / 512) groups of four leaves
__global__ void __launch_bounds__(SR_THREADS) stream_read_leaf_kernel(const char* __restrict__ w, int cols,
                                                                       int nstrips, uint32_t* sink) {
  constexpr int NBLK = SR_LEAF / SR_RB, RING = SR_AHEAD + 1;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int strip = blockIdx.x % nstrips, grp = blockIdx.x / nstrips;
  const int64_t leaf = (int64_t)grp * 4 + wave;
  const char* base = w + leaf * SR_LEAF * cols + strip * 256;
  auto block_rs = [&](int b) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base) + (int64_t)b * SR_RB * cols, (short)0,
                                             0x7FFFFFFF, RSRC_WORD3);
  };
  uint32_t ring[RING][SR_RB];
#pragma unroll
  for (int b = 0; b < SR_AHEAD; ++b) {
    const __amdgpu_buffer_rsrc_t rs = block_rs(b);
#pragma unroll
    for (int i = 0; i < SR_RB; ++i) ring[b][i] = __builtin_amdgcn_raw_buffer_load_b32(rs, lane * 4, i * cols, 0);
  }
  uint32_t acc = 0;
#pragma unroll
  for (int b = 0; b < NBLK; ++b) {
    if (b + SR_AHEAD < NBLK) {
      __builtin_amdgcn_sched_barrier(0);
      const __amdgpu_buffer_rsrc_t rs = block_rs(b + SR_AHEAD);
#pragma unroll
      for (int i = 0; i < SR_RB; ++i)
        ring[(b + SR_AHEAD) % RING][i] = __builtin_amdgcn_raw_buffer_load_b32(rs, lane * 4, i * cols, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < SR_RB; ++i) acc = (acc ^ ring[b % RING][i]) * 3u;
  }
  if (acc == SR_UNLIKELY) sink[0] = acc;
}

hipError_t run_stream_read(const void* w, int64_t rows, int64_t cols, int pattern, uint32_t* sink,
                           hipStream_t stream) {
  if (rows <= 0 || cols <= 0 || w == nullptr || sink == nullptr) return hipErrorInvalidValue;
  if (pattern == 0) {
    if ((rows * cols) % 16 != 0 || !sr_aligned(w, 16)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read_linear_kernel, dim3(SR_LINEAR_WGS), dim3(SR_THREADS), 0, stream,
                       static_cast<const u4*>(w), rows * cols / 16, sink);
    return hipGetLastError();
  }
  if (pattern == 1) {
    // whole groups of four 128-row leaves, whole 256-byte strips, and a 16-row block of rows
    // within the loads' 31-bit offsets
    if (rows % (4 * SR_LEAF) != 0 || cols % 256 != 0 || !sr_aligned(w, 4) || (int64_t)SR_RB * cols >= (1LL << 31) ||
        cols > INT32_MAX)
      return hipErrorInvalidValue;
    const int nstrips = (int)(cols / 256);
    const int64_t nwg = (int64_t)nstrips * (rows / (4 * SR_LEAF));
    if (nwg > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(stream_read_leaf_kernel, dim3((unsigned)nwg), dim3(SR_THREADS), 0, stream,
                       static_cast<const char*>(w), (int)cols, nstrips, sink);
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

}  // namespace mlg

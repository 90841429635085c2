// Read-only streams over an int8 matrix W[rows][cols]: the memory floors the skinny products are
// measured against (no arithmetic, no output beyond a sink word that is written only if the
// folded bits equal an unlikely value, so no load can be dropped).
//
//  pattern 0: a grid-stride stream of 16-byte loads over the whole matrix in address order --
//             the fastest read of the bytes;
//  pattern 1: the reads of the decode kernel (gemv_nn_kernel, whole 128-row leaves): a wave per
//             128-row leaf and 256-byte column strip, one 32-bit word per lane per row, rows in
//             16-row blocks through a ring three blocks ahead, four leaves a workgroup -- the
//             contract's leaf chains force every leaf of a column to be streamed at once;
//  pattern 2: the reads of the decode-packed product's whole-column workgroups
//             (gemv_packed.hip): W[rows][cols] taken as the packed bytes of a rows x cols
//             matrix, a workgroup of 16 waves per 64-column group, each wave two adjacent
//             leaves, one 16-byte load per lane per 16-row block of a leaf, two blocks ahead,
//             non-temporal -- block s of every leaf is one slab the waves read together.
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

// grid: one workgroup per 64-column group of one 32-leaf group (rows = 4096, cols a multiple of 64)
constexpr int SR_PK_WAVES = 16, SR_PK_AHEAD = 2, SR_PK_BLOCKS = SR_LEAF / 16;
__global__ void __launch_bounds__(64 * SR_PK_WAVES) stream_read_packed_kernel(const char* __restrict__ w, int nleaves,
                                                                               int ncg, uint32_t* sink) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t cg = blockIdx.x % ncg, grp = blockIdx.x / ncg;
  const int64_t t0 = grp * 2 * SR_PK_WAVES + 2 * wave;
  const int64_t slab = (int64_t)nleaves * ncg * 1024;
  const char* base = w + (t0 * ncg + cg) * 1024;
  auto block_rs = [&](int s) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base) + s * slab, (short)0, 0x7FFFFFFF, RSRC_WORD3);
  };
  const int lstride = ncg * 1024;
  u4 ring[SR_PK_BLOCKS][2];
  uint32_t acc = 0;
#pragma unroll
  for (int s = 0; s < SR_PK_AHEAD; ++s)
#pragma unroll
    for (int q = 0; q < 2; ++q) ring[s][q] = __builtin_amdgcn_raw_buffer_load_b128(block_rs(s), lane * 16, q * lstride, 2);
#pragma unroll
  for (int s = 0; s < SR_PK_BLOCKS; ++s) {
    if (s + SR_PK_AHEAD < SR_PK_BLOCKS) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < 2; ++q)
        ring[s + SR_PK_AHEAD][q] = __builtin_amdgcn_raw_buffer_load_b128(block_rs(s + SR_PK_AHEAD), lane * 16, q * lstride, 2);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) acc = (acc ^ ring[s][q][0] ^ ring[s][q][1] ^ ring[s][q][2] ^ ring[s][q][3]) * 3u;
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
  if (pattern == 2) {
    // whole 32-leaf groups of 64-column groups: every load of a workgroup lies in the buffer
    if (rows % (2 * SR_PK_WAVES * SR_LEAF) != 0 || cols % 64 != 0 || !sr_aligned(w, 16) || rows * cols >= (1LL << 31))
      return hipErrorInvalidValue;
    const int nleaves = (int)(rows / SR_LEAF), ncg = (int)(cols / 64);
    const int64_t nwg = (int64_t)ncg * (nleaves / (2 * SR_PK_WAVES));
    hipLaunchKernelGGL(stream_read_packed_kernel, dim3((unsigned)nwg), dim3(64 * SR_PK_WAVES), 0, stream,
                       static_cast<const char*>(w), nleaves, ncg, sink);
    return hipGetLastError();
  }
  return hipErrorInvalidValue;
}

}  // namespace mlg

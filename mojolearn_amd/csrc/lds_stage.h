// Operand slices staged HBM -> LDS with buffer loads (the MFMA GEMM kernels): slice layout,
// loader, LDS hand-off barrier and operand reads.
#pragma once
#include "device_common.h"
#include "mfma.h"

namespace mlg {

// One staged slice (BM indices x SK steps; SK = KT unless a kernel says otherwise) of an
// operand of element type T, as NCH = BM*SK*bytes/16 chunks of 16 bytes, chunk position p loaded by lane p % 64 of
// load instruction p / 64 (a load instruction fills 1 KB of LDS, lane L at L*16).
//  * index-major (the operand stores k contiguously: A in NN/NT, B in NT): index r owns
//    CR = SK*bytes/16 chunks; its chunk c sits at position r*CR + (c ^ swz(r)), so the
//    lanes of one read (consecutive r, same c) land in different banks.
//  * k-major (the operand stores indices contiguously: B in NN/TN, A in TN): step s owns
//    RC = BM*bytes/16 chunks holding the BM indices in order.
template <int T, bool IMAJ, int SK = KT>
struct Slice {
  static constexpr int EB = Elem<T>::bytes;
  static constexpr int CE = Elem<T>::per16;
  static constexpr int NCH = BM * SK * EB / 16;  // at KT: 1024 / 512 / 256
  static constexpr int NI = NCH / 64;            // load instructions per slice: 16 / 8 / 4
  static constexpr int CR = SK * EB / 16;        // 8 / 4 / 2
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

// The global side of one operand: this lane's share of every slice's load instructions, as
// buffer loads straight into LDS.  Load instruction q of a slice covers RPI consecutive
// stored rows; its scalar resource starts at the first of them (at the step where the
// resource was built) and ends at the operand's end, and the lane's byte offset within it
// is fixed for the whole k loop.  Slices are issued in ascending order, one slice apart, so
// a slice's loads differ from the previous slice's only by a scalar offset (SOFF_STEP bytes
// per step); the resources are rebuilt only when that offset passes 2^30 (never for an
// index-major operand of fewer than 2^28 steps).  A chunk past the operand's end reads as
// zeros (the resource's record bound, exact because lane offset + scalar offset stays below
// 2^31); a chunk past a row's end reads the next row's bytes.  Neither reaches a stored
// cell: indices past m or n are never stored, steps past k are never executed.  The host
// keeps RPI * pitch * bytes below 2^30.
template <int T, bool IMAJ, int SK = KT>
struct DirectLoader {
  using S = Slice<T, IMAJ, SK>;
  static constexpr int RPI = IMAJ ? 64 / S::CR : 64 / S::RC;  // stored rows per instruction
  uint32_t voff[S::PER_WAVE];
  __amdgpu_buffer_rsrc_t rs[S::PER_WAVE];
  uint32_t soff;        // bytes from the resources' step to the next slice's first step
  uint32_t slice_step;  // bytes one slice advances the scalar offset

  __device__ __forceinline__ void init(int64_t pitch, int wave, int lane) {
#pragma unroll
    for (int h = 0; h < S::PER_WAVE; ++h) {
      const int q = (wave + NWAVES * h) % S::NI;
      int di, dk;
      S::coords(q * 64 + lane, di, dk);
      if constexpr (IMAJ) voff[h] = (uint32_t)(((di - q * RPI) * pitch + dk) * S::EB);
      else voff[h] = (uint32_t)(((dk - q * RPI) * pitch + di) * S::EB);
    }
    slice_step = (uint32_t)(IMAJ ? SK * S::EB : SK * pitch * S::EB);
    soff = 0x7FFFFFFFu;  // the first issue builds the resources
  }

  // Resources for the slice that starts at step k0; the scalar offset restarts at 0.
  __device__ __forceinline__ void bind(const void* base, int64_t total_bytes, int64_t pitch, int64_t idx0,
                                       int64_t k0, int wave) {
#pragma unroll
    for (int h = 0; h < S::PER_WAVE; ++h) {
      const int q = (wave + NWAVES * h) % S::NI;
      const int64_t off = IMAJ ? ((idx0 + q * RPI) * pitch + k0) * S::EB : ((k0 + q * RPI) * pitch + idx0) * S::EB;
      const int64_t rem = total_bytes - off;
      const int nrec = rem <= 0 ? 0 : (rem > 0x7FFFFFFF ? 0x7FFFFFFF : (int)rem);
      const char* first = static_cast<const char*>(base) + (rem > 0 ? off : 0);
      rs[h] = __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(first), (short)0, nrec, RSRC_WORD3);
    }
    soff = 0;
  }

  // Issue this wave's PER_WAVE loads of the slice that starts at step k0 into `slice`: the
  // slice after the previously issued one, or the first (when a slice has fewer load
  // instructions than waves, the extra waves repeat an earlier wave's chunk -- the same
  // bytes to the same place -- so every wave issues the same count and can wait on it with
  // one vmcnt).  `wave` must be wave-uniform.
  __device__ __forceinline__ void issue(char* slice, const void* base, int64_t total_bytes, int64_t pitch,
                                        int64_t idx0, int64_t k0, int wave) {
    if (soff > (1u << 30)) bind(base, total_bytes, pitch, idx0, k0, wave);
#pragma unroll
    for (int h = 0; h < S::PER_WAVE; ++h) {
      const int q = (wave + NWAVES * h) % S::NI;
#if defined(__HIP_DEVICE_COMPILE__)
      // (the host pass compiles kernel bodies only for their launch stubs; with this builtin
      // in a kernel template it drops the stubs of every instantiation after the first)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs[h], (lds_vptr)(slice + q * 1024), 16, voff[h], soff, 0, 0);
#else
      (void)slice;
#endif
    }
    soff += slice_step;
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
template <int T, bool IMAJ, int SK = KT>
__device__ __forceinline__ f4 read4(const char* slice, int idx, int s, float scale) {
  using S = Slice<T, IMAJ, SK>;
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

}  // namespace mlg

// Staged host <-> device transport of the host-pointer surface (the role of
// gemm/host_transport.mojo:42-45,193-272: pinned stage, double-buffered chunks).
//
// A job moves a list of uploads (host -> device) and a list of downloads (device -> host) at
// the same time.  Each transfer is cut into STAGE_CHUNK-byte chunks; STAGE_WORKERS host threads
// (the caller is worker 0) take the chunks round-robin.  A worker owns STAGE_DEPTH pinned slots
// per direction and one stream per direction: an upload chunk is copied into a free slot and
// its DMA enqueued on the worker's upload stream; a download chunk's DMA into a slot is enqueued
// ahead, waited for, then copied out.  Separate streams keep the copy engines fed back to back
// (one stream leaves a gap after every command while the runtime retires it).  A job can also
// carry "touch" ranges: host memory about to be written by a later download (a fresh output
// array), whose pages the workers fault in between their upload chunks, so the download's
// copy-out does not pay for them.  Transfers shorter than STAGE_MIN go as one plain copy.
// No arithmetic: bytes are moved, never changed.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>
#include <condition_variable>
#include <mutex>
#include <string>
#include <vector>

namespace mlt {

constexpr size_t STAGE_CHUNK = size_t(2) << 20;  // bytes per pinned slot
constexpr int STAGE_WORKERS = 8;                 // host copy threads, the caller included
constexpr int STAGE_DEPTH = 2;                   // slots per worker and direction
constexpr size_t STAGE_MIN = size_t(1) << 20;    // shorter transfers go as one plain copy
constexpr size_t TOUCH_PIECE = size_t(2) << 20;  // bytes of a touch range per work item

// One transfer: `bytes` between host memory and device memory.  A download whose `after` is
// set starts once that event has completed (e.g. the product that writes its source).
struct Span {
  void* host;
  void* dev;
  size_t bytes;
  hipEvent_t after = nullptr;
};

class Stager {
 public:
  // Pinned slots (2 * STAGE_WORKERS * STAGE_DEPTH * STAGE_CHUNK bytes), streams and events on
  // the current device, and the worker threads.  Throws std::runtime_error on a HIP failure.
  Stager();
  Stager(const Stager&) = delete;
  Stager& operator=(const Stager&) = delete;

  // Move every upload and download; fault in the pages of every touch range (content kept).
  // Returns when each upload's host memory has been read (its DMAs are enqueued, possibly still
  // running) and each download is complete in host memory.
  void run(const std::vector<Span>& ups, const std::vector<Span>& downs, const std::vector<Span>& touch = {});

  // Make `s` wait for every upload enqueued so far.
  void order_after_uploads(hipStream_t s);

 private:
  struct Chunk {
    char* host;
    char* dev;
    size_t bytes;
    hipEvent_t after;
  };
  void work(int w);
  void fail(hipError_t e, const char* what);
  bool ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    fail(e, what);
    return false;
  }
  void loop(int w);

  static constexpr int SLOTS = STAGE_WORKERS * STAGE_DEPTH;
  char* up_slots_ = nullptr;  // [SLOTS][STAGE_CHUNK]
  char* dn_slots_ = nullptr;
  hipEvent_t up_ev_[SLOTS];
  hipEvent_t dn_ev_[SLOTS];
  bool up_armed_[SLOTS];  // a DMA from the slot may still be running
  hipStream_t up_stream_[STAGE_WORKERS];
  hipStream_t dn_stream_[STAGE_WORKERS];
  hipEvent_t order_ev_[STAGE_WORKERS];
  std::atomic<bool> touch_ok_{true};  // the kernel populates pages on request

  // the current job
  std::vector<Chunk> ups_, downs_;
  std::vector<Span> touch_;
  std::string error_;

  std::mutex mu_;
  std::condition_variable go_, done_;
  uint64_t generation_ = 0;
  int remaining_ = 0;
};

}  // namespace mlt

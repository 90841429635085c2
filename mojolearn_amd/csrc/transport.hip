// Staged host <-> device transport (host code only); the scheme is described in transport.h.
#include "transport.h"

#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

#include <stdexcept>
#include <thread>

namespace mlt {

namespace {

void check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string("mlgemm: ") + what + " failed: " + hipGetErrorString(e));
}

void cut(const std::vector<Span>& spans, std::vector<Span>& small, std::vector<Span>& big) {
  for (const Span& s : spans) {
    if (s.bytes == 0) continue;
    (s.bytes < STAGE_MIN ? small : big).push_back(s);
  }
}

// Fault in the pages of [p, p + bytes) writable, keeping their content.  False when the kernel
// does not know the request (then nothing was changed).
bool populate(void* p, size_t bytes) {
  static const uintptr_t page = (uintptr_t)sysconf(_SC_PAGESIZE);
  const uintptr_t lo = (uintptr_t)p & ~(page - 1);
  const uintptr_t hi = ((uintptr_t)p + bytes + page - 1) & ~(page - 1);
#ifdef MADV_POPULATE_WRITE
  return madvise((void*)lo, hi - lo, MADV_POPULATE_WRITE) == 0;
#else
  (void)lo;
  (void)hi;
  return false;
#endif
}

}  // namespace

Stager::Stager() {
  check(hipHostMalloc((void**)&up_slots_, SLOTS * STAGE_CHUNK, hipHostMallocDefault), "hipHostMalloc");
  check(hipHostMalloc((void**)&dn_slots_, SLOTS * STAGE_CHUNK, hipHostMallocDefault), "hipHostMalloc");
  for (int i = 0; i < SLOTS; ++i) {
    check(hipEventCreateWithFlags(&up_ev_[i], hipEventDisableTiming), "hipEventCreate");
    check(hipEventCreateWithFlags(&dn_ev_[i], hipEventDisableTiming), "hipEventCreate");
    up_armed_[i] = false;
  }
  for (int w = 0; w < STAGE_WORKERS; ++w) {
    check(hipStreamCreateWithFlags(&up_stream_[w], hipStreamNonBlocking), "hipStreamCreate");
    check(hipStreamCreateWithFlags(&dn_stream_[w], hipStreamNonBlocking), "hipStreamCreate");
    check(hipEventCreateWithFlags(&order_ev_[w], hipEventDisableTiming), "hipEventCreate");
  }
  // The workers live as long as the process (the Stager is never destroyed); they sleep on
  // the condition variable between jobs.
  for (int w = 1; w < STAGE_WORKERS; ++w) std::thread(&Stager::loop, this, w).detach();
}

void Stager::fail(hipError_t e, const char* what) {
  std::lock_guard<std::mutex> lock(mu_);
  if (error_.empty()) error_ = std::string("mlgemm: ") + what + " failed: " + hipGetErrorString(e);
}

void Stager::loop(int w) {
  uint64_t seen = 0;
  for (;;) {
    {
      std::unique_lock<std::mutex> lock(mu_);
      go_.wait(lock, [&] { return generation_ != seen; });
      seen = generation_;
    }
    work(w);
    std::lock_guard<std::mutex> lock(mu_);
    if (--remaining_ == 0) done_.notify_one();
  }
}

// Worker w takes upload chunks w, w + W, ..., touch pieces w, w + W, ... and download chunks
// w, w + W, ..., one of each per round, so every kind of work advances together.  Its slots
// are w * DEPTH + j % DEPTH; its streams up_stream_[w] and dn_stream_[w].
void Stager::work(int w) {
  constexpr int W = STAGE_WORKERS, D = STAGE_DEPTH;
  auto mine = [&](size_t total) { return total > (size_t)w ? (total - w + W - 1) / W : 0; };
  const size_t nu = mine(ups_.size()), nd = mine(downs_.size());
  size_t pieces = 0;
  for (const Span& s : touch_) pieces += (s.bytes + TOUCH_PIECE - 1) / TOUCH_PIECE;
  const size_t nt = mine(pieces);
  hipStream_t ds = dn_stream_[w];
  hipEvent_t waited = nullptr;
  auto dn_issue = [&](size_t j) {
    const Chunk& c = downs_[w + j * W];
    const int slot = w * D + (int)(j % D);
    if (c.after && c.after != waited) {
      if (!ok(hipStreamWaitEvent(ds, c.after, 0), "hipStreamWaitEvent")) return false;
      waited = c.after;
    }
    char* buf = dn_slots_ + (size_t)slot * STAGE_CHUNK;
    return ok(hipMemcpyAsync(buf, c.dev, c.bytes, hipMemcpyDeviceToHost, ds), "hipMemcpyAsync D2H") &&
           ok(hipEventRecord(dn_ev_[slot], ds), "hipEventRecord");
  };
  auto touch_piece = [&](size_t t) {
    size_t p = w + t * W;  // global piece index
    for (const Span& s : touch_) {
      const size_t n = (s.bytes + TOUCH_PIECE - 1) / TOUCH_PIECE;
      if (p < n) {
        const size_t off = p * TOUCH_PIECE;
        const size_t len = s.bytes - off < TOUCH_PIECE ? s.bytes - off : TOUCH_PIECE;
        if (touch_ok_ && !populate((char*)s.host + off, len)) touch_ok_ = false;
        return;
      }
      p -= n;
    }
  };
  for (size_t j = 0; j < nd && j < (size_t)D; ++j)
    if (!dn_issue(j)) return;
  size_t iu = 0, it = 0, id = 0;
  while (iu < nu || it < nt || id < nd) {
    if (iu < nu) {
      const Chunk& c = ups_[w + iu * W];
      const int slot = w * D + (int)(iu % D);
      char* buf = up_slots_ + (size_t)slot * STAGE_CHUNK;
      if (up_armed_[slot] && !ok(hipEventSynchronize(up_ev_[slot]), "hipEventSynchronize")) return;
      memcpy(buf, c.host, c.bytes);
      if (!ok(hipMemcpyAsync(c.dev, buf, c.bytes, hipMemcpyHostToDevice, up_stream_[w]), "hipMemcpyAsync H2D") ||
          !ok(hipEventRecord(up_ev_[slot], up_stream_[w]), "hipEventRecord"))
        return;
      up_armed_[slot] = true;
      ++iu;
    }
    if (it < nt) touch_piece(it++);
    if (id < nd) {
      const Chunk& c = downs_[w + id * W];
      const int slot = w * D + (int)(id % D);
      if (!ok(hipEventSynchronize(dn_ev_[slot]), "hipEventSynchronize")) return;
      memcpy(c.host, dn_slots_ + (size_t)slot * STAGE_CHUNK, c.bytes);
      if (id + D < nd && !dn_issue(id + D)) return;
      ++id;
    }
  }
}

void Stager::run(const std::vector<Span>& ups, const std::vector<Span>& downs, const std::vector<Span>& touch) {
  std::vector<Span> small_up, big_up, small_dn, big_dn;
  cut(ups, small_up, big_up);
  cut(downs, small_dn, big_dn);
  for (const Span& s : small_up)
    check(hipMemcpyAsync(s.dev, s.host, s.bytes, hipMemcpyHostToDevice, up_stream_[0]), "hipMemcpyAsync H2D");
  for (const Span& s : small_dn) {
    if (s.after) check(hipStreamWaitEvent(dn_stream_[0], s.after, 0), "hipStreamWaitEvent");
    check(hipMemcpyAsync(s.host, s.dev, s.bytes, hipMemcpyDeviceToHost, dn_stream_[0]), "hipMemcpyAsync D2H");
  }
  if (!big_up.empty() || !big_dn.empty() || !touch.empty()) {
    ups_.clear();
    downs_.clear();
    for (const Span& s : big_up)
      for (size_t off = 0; off < s.bytes; off += STAGE_CHUNK)
        ups_.push_back({(char*)s.host + off, (char*)s.dev + off,
                        s.bytes - off < STAGE_CHUNK ? s.bytes - off : STAGE_CHUNK, nullptr});
    for (const Span& s : big_dn)
      for (size_t off = 0; off < s.bytes; off += STAGE_CHUNK)
        downs_.push_back({(char*)s.host + off, (char*)s.dev + off,
                          s.bytes - off < STAGE_CHUNK ? s.bytes - off : STAGE_CHUNK, s.after});
    touch_ = touch;
    {
      std::lock_guard<std::mutex> lock(mu_);
      error_.clear();
      remaining_ = STAGE_WORKERS - 1;
      ++generation_;
    }
    go_.notify_all();
    work(0);
    std::unique_lock<std::mutex> lock(mu_);
    done_.wait(lock, [&] { return remaining_ == 0; });
    if (!error_.empty()) throw std::runtime_error(error_);
  }
  if (!small_dn.empty()) check(hipStreamSynchronize(dn_stream_[0]), "hipStreamSynchronize");
}

void Stager::order_after_uploads(hipStream_t s) {
  for (int w = 0; w < STAGE_WORKERS; ++w) {
    check(hipEventRecord(order_ev_[w], up_stream_[w]), "hipEventRecord");
    check(hipStreamWaitEvent(s, order_ev_[w], 0), "hipStreamWaitEvent");
  }
}

}  // namespace mlt

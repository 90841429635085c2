// C ABI of libmlgemm.so (declared in include/mlgemm.h).
//
// linalg_native_v1 restates the reference's op table and error protocol
// (gemm/linalg_dispatch.mojo:14-102, core/native_descriptor_call.mojo:8-13,38-55,95-100):
// host pointers in, host pointers out, synchronous, one sink call on failure.  The
// device-pointer entries enqueue on a caller's stream and return.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <atomic>
#include <functional>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/mlgemm.h"
#include "act.h"
#include "contract.h"
#include "kernels.h"
#include "q8.h"
#include "transport.h"

namespace {

constexpr int64_t PROFILE_VERSION = 1;         // gemm/contract.mojo:140-151 (fp32.v1)
constexpr int64_t LOWBIT_PROFILE_VERSION = 1;  // gemm/contract.mojo:397
constexpr int64_t INT15_PROFILE_VERSION = 1;   // gemm/contract.mojo:406
constexpr int64_t NUMERIC_MODE_IDENTICAL = 1;

thread_local std::string g_last_error;

struct Fail : std::runtime_error {
  using std::runtime_error::runtime_error;
};

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw Fail(std::string("mlgemm: ") + what + " failed: " + hipGetErrorString(e));
}

int num_cus_of_current_device() {
  static std::mutex mu;
  static std::vector<int> cache;
  int dev = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  std::lock_guard<std::mutex> lock(mu);
  if ((int)cache.size() <= dev) cache.resize(dev + 1, 0);
  if (cache[dev] == 0) {
    int cus = 0;
    hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
              "hipDeviceGetAttribute");
    cache[dev] = cus > 0 ? cus : 1;
  }
  return cache[dev];
}

void check_problem(const mlg::GemmProblem& p, int cus) {
  if (p.m < 0 || p.n < 0 || p.k < 0) throw Fail("mlgemm: m, n and k must be >= 0");
  if (p.op != mlg::OP_NN && p.op != mlg::OP_NT && p.op != mlg::OP_TN)
    throw Fail("mlgemm: op must be 0 (OP_NN), 1 (OP_NT) or 2 (OP_TN), got " + std::to_string(p.op));
  if (p.leaf < 0) throw Fail("mlgemm: leaf must be >= 0 (0 = the contract's leaf size)");
  // the reference refuses partitions beyond its kernels' fold stack the same way
  // (gemm/neural_dispatch.mojo:284-285)
  const std::string why = mlg::launch_limit(p, cus);
  if (!why.empty()) throw Fail("mlgemm: " + why);
}

// Enqueue one product on `stream`.  Workspace: the caller's (user_ws_bytes >= 0; its counters
// zero, as every product leaves them), or one allocated from the stream-ordered pool, its
// counters zeroed by a kernel, and released on the same stream.
void enqueue_gemm(const mlg::GemmProblem& p, hipStream_t stream, void* user_ws = nullptr,
                  int64_t user_ws_bytes = -1) {
  const int cus = num_cus_of_current_device();
  check_problem(p, cus);
  if (p.m == 0 || p.n == 0) return;
  if (!p.c || (p.k > 0 && (!p.a || !p.b))) throw Fail("mlgemm: null operand pointer");
  if (p.b_type == mlg::T_I8 && p.k > 0 && !p.scales) throw Fail("mlgemm: int8 weight needs scales");
  const int64_t wsf = mlg::gemm_workspace_floats(p, cus);
  float* ws = nullptr;
  const bool own_ws = user_ws_bytes < 0;
  if (!own_ws && wsf > 0) {
    if (!user_ws || user_ws_bytes < wsf * (int64_t)sizeof(float))
      throw Fail("mlgemm: workspace of " + std::to_string(user_ws_bytes) + " bytes is smaller than the " +
                 std::to_string(wsf * (int64_t)sizeof(float)) + " this product needs (mlg_gemm_workspace_bytes)");
    ws = (float*)user_ws;
  }
  hipError_t e = hipSuccess;
  if (own_ws && wsf > 0) {
    hip_check(hipMallocAsync((void**)&ws, (size_t)wsf * sizeof(float), stream), "hipMallocAsync");
    e = mlg::run_zero_words(reinterpret_cast<unsigned int*>(ws), mlg::gemm_counter_count(p), stream);
  }
  if (e == hipSuccess) e = mlg::run_gemm(p, ws, cus, stream);
  if (own_ws && ws) {
    hipError_t f = hipFreeAsync(ws, stream);
    if (e == hipSuccess) e = f;
  }
  hip_check(e, "gemm launch");
}

int guarded(const std::function<void()>& fn) {
  try {
    fn();
    g_last_error.clear();
    return 0;
  } catch (const std::exception& ex) {
    g_last_error = ex.what();
    return 1;
  }
}

// ---- host-pointer transport (the role of gemm/host_entry.mojo:79-197 and
// gemm/host_transport.mojo:107-272): pooled device buffers guarded by a busy flag, and the
// staged transport (transport.h) on an upload and a download stream beside the compute
// stream.  A concurrent second caller gets fresh buffers, one stream and plain copies.
struct DeviceBuf {
  void* ptr = nullptr;
  size_t cap = 0;
  void* get(size_t bytes) {
    if (bytes == 0) bytes = 1;
    if (bytes > cap) {
      if (ptr) hip_check(hipFree(ptr), "hipFree");
      ptr = nullptr;
      cap = 0;
      hip_check(hipMalloc(&ptr, bytes), "hipMalloc");
      cap = bytes;
    }
    return ptr;
  }
  void release() {
    if (ptr) (void)hipFree(ptr);
    ptr = nullptr;
    cap = 0;
  }
};

// Row bands of a host product: at most MAX_BANDS, each about BAND_BYTES of A.
constexpr int MAX_BANDS = 8;
constexpr size_t BAND_BYTES = size_t(16) << 20;

struct HostPool {
  DeviceBuf c, a, b, x, y, w, a2, b2;
  hipStream_t stream = nullptr;   // products
  mlt::Stager* stager = nullptr;  // pooled set only; never destroyed: its workers live with the process
  hipEvent_t evc[MAX_BANDS] = {};
};

std::atomic<int> g_pool_busy{0};
HostPool g_pool;
std::mutex g_pool_init;

void init_pooled_set(HostPool& P) {
  if (!P.stream) hip_check(hipStreamCreateWithFlags(&P.stream, hipStreamNonBlocking), "hipStreamCreate");
  for (hipEvent_t& e : P.evc)
    if (!e) hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
  if (!P.stager) {
    try {
      P.stager = new mlt::Stager();
    } catch (const std::exception& ex) {
      throw Fail(ex.what());
    }
  }
}

struct Lease {
  HostPool* pool;
  HostPool fresh;
  bool pooled;
  Lease() {
    int expect = 0;
    pooled = g_pool_busy.compare_exchange_strong(expect, 1);
    if (pooled) {
      try {
        std::lock_guard<std::mutex> lock(g_pool_init);
        init_pooled_set(g_pool);
      } catch (...) {
        g_pool_busy.store(0);
        throw;
      }
      pool = &g_pool;
    } else {
      hip_check(hipStreamCreateWithFlags(&fresh.stream, hipStreamNonBlocking), "hipStreamCreate");
      pool = &fresh;
    }
  }
  ~Lease() {
    if (pooled) {
      g_pool_busy.store(0);
    } else {
      fresh.c.release(); fresh.a.release(); fresh.b.release(); fresh.x.release(); fresh.y.release();
      fresh.w.release(); fresh.a2.release(); fresh.b2.release();
      if (fresh.stream) (void)hipStreamDestroy(fresh.stream);
    }
  }
};

void up(void* dst, const void* src, size_t bytes, hipStream_t s) {
  if (bytes) hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, s), "hipMemcpy H2D");
}
void down(void* dst, const void* src, size_t bytes, hipStream_t s) {
  if (bytes) hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, s), "hipMemcpy D2H");
}

mlt::Span span(int64_t host, void* dev, int64_t bytes, hipEvent_t after = nullptr) {
  return mlt::Span{(void*)host, dev, (size_t)bytes, after};
}

// Uploads that the next work on P.stream reads.
void put(HostPool& P, const std::vector<mlt::Span>& ups) {
  if (!P.stager) {
    for (const mlt::Span& s : ups) up(s.dev, s.host, s.bytes, P.stream);
    return;
  }
  P.stager->run(ups, {});
  P.stager->order_after_uploads(P.stream);
}

// Downloads of what the work enqueued on P.stream wrote; returns with them in host memory.
void get(HostPool& P, std::vector<mlt::Span> downs) {
  if (!P.stager) {
    for (const mlt::Span& s : downs) down(s.host, s.dev, s.bytes, P.stream);
  } else {
    hip_check(hipEventRecord(P.evc[0], P.stream), "hipEventRecord");
    for (mlt::Span& s : downs) s.after = P.evc[0];
    P.stager->run({}, downs);
  }
  hip_check(hipStreamSynchronize(P.stream), "hipStreamSynchronize");
}

std::string shape_text(int64_t m, int64_t n, int64_t k) {
  return "m=" + std::to_string(m) + " n=" + std::to_string(n) + " k=" + std::to_string(k);
}

// gemm/host_entry.mojo:115-126: degenerate shapes are refused at the host surface.
void refuse_host_shape(const char* who, int64_t m, int64_t n, int64_t k, int64_t op) {
  if (m <= 0 || n <= 0 || k <= 0)
    throw Fail(std::string(who) + ": m, n and k must all be positive, got " + shape_text(m, n, k) +
               " (contract section 8 specifies the degenerate shapes; this surface has no gate on"
               " them and refuses rather than guesses)");
  if (op != mlg::OP_NN && op != mlg::OP_NT && op != mlg::OP_TN)
    throw Fail(std::string(who) + ": op must be 0 (OP_NN), 1 (OP_NT) or 2 (OP_TN), got " +
               std::to_string(op));
}

// A host product in row bands of A (OP_NN and OP_NT keep A[m][k] row-major).  Job j of the
// staged transport uploads band j (job 0 also B, and scales or bias, and faults in the output's
// pages) and downloads band j - 2 of C, after its product; band j is multiplied on the compute
// stream once its upload is in.  The link carries both directions at once and the products hide
// behind the transfers.  Every cell is computed exactly as in one launch (the leaf partition
// depends on k only).  An output whose host memory overlaps A's takes one band, so that A is
// read whole before any of C is written.
int64_t host_gemm(const std::vector<int64_t>& ad, const std::vector<int64_t>& pr, int a_type,
                  int b_type, bool with_bias) {
  const int64_t m = pr[0], n = pr[1], k = pr[2], op = pr[3];
  const char* who = b_type == mlg::T_BF16 ? "gemm_bf16" : (b_type == mlg::T_I8 ? "gemm_int8w" : "identical_gemm_host");
  refuse_host_shape(who, m, n, k, op);
  Lease lease;
  HostPool& P = *lease.pool;
  const int64_t ea = a_type == mlg::T_F32 ? 4 : 2;
  const int64_t eb = b_type == mlg::T_F32 ? 4 : (b_type == mlg::T_BF16 ? 2 : 1);
  char* dc = (char*)P.c.get((size_t)(m * n) * 4);
  char* da = (char*)P.a.get((size_t)(m * k * ea));
  void* db = P.b.get((size_t)(n * k * eb));
  float* dx = nullptr;
  if (b_type == mlg::T_I8 || with_bias) dx = (float*)P.x.get((size_t)n * 4);
  mlg::GemmProblem p{};
  p.b = db;
  p.scales = b_type == mlg::T_I8 ? dx : nullptr;
  p.bias = with_bias ? dx : nullptr;
  p.n = n; p.k = k; p.op = (int)op; p.a_type = a_type; p.b_type = b_type; p.leaf = 0;

  // bands: whole multiples of 256 rows, about BAND_BYTES of A each
  int64_t rows = m;
  const uintptr_t c_lo = (uintptr_t)ad[0], c_hi = c_lo + (uintptr_t)(m * n * 4);
  const uintptr_t a_lo = (uintptr_t)ad[1], a_hi = a_lo + (uintptr_t)(m * k * ea);
  const bool c_overlaps_a = c_lo < a_hi && a_lo < c_hi;
  if (P.stager && op != mlg::OP_TN && !c_overlaps_a) {
    int64_t nb = (m * k * ea) / (int64_t)BAND_BYTES;
    nb = nb < 1 ? 1 : (nb > MAX_BANDS ? MAX_BANDS : nb);
    rows = ((m + nb - 1) / nb + 255) / 256 * 256;
    if (rows > m) rows = m;
  }
  const int64_t nb = (m + rows - 1) / rows;
  auto band_rows = [&](int64_t j) { return (j + 1) * rows <= m ? rows : m - j * rows; };
  auto set_band = [&](int64_t j) {
    if (op == mlg::OP_TN) {
      p.a = da;
      p.c = (float*)dc;
      p.m = m;
    } else {
      p.a = da + j * rows * k * ea;
      p.c = (float*)(dc + j * rows * n * 4);
      p.m = band_rows(j);
    }
  };
  if (!P.stager) {
    up(da, (const void*)ad[1], (size_t)(m * k * ea), P.stream);
    up(db, (const void*)ad[2], (size_t)(n * k * eb), P.stream);
    if (dx) up(dx, (const void*)ad[3], (size_t)n * 4, P.stream);
    set_band(0);
    enqueue_gemm(p, P.stream);
    down((void*)ad[0], dc, (size_t)(m * n) * 4, P.stream);
    hip_check(hipStreamSynchronize(P.stream), "hipStreamSynchronize");
    return m * n;
  }
  for (int64_t j = 0; j < nb + 2; ++j) {
    std::vector<mlt::Span> ups, downs, touch;
    if (j == 0) {
      ups.push_back(span(ad[2], db, n * k * eb));
      if (dx) ups.push_back(span(ad[3], dx, n * 4));
      touch.push_back(span(ad[0], nullptr, m * n * 4));
    }
    if (j < nb) {
      if (op == mlg::OP_TN) ups.push_back(span(ad[1], da, m * k * ea));
      else ups.push_back(span(ad[1] + j * rows * k * ea, da + j * rows * k * ea, band_rows(j) * k * ea));
    }
    if (j >= 2) {
      const int64_t t = j - 2;
      downs.push_back(op == mlg::OP_TN ? span(ad[0], dc, m * n * 4, P.evc[t])
                                       : span(ad[0] + t * rows * n * 4, dc + t * rows * n * 4, band_rows(t) * n * 4, P.evc[t]));
    }
    P.stager->run(ups, downs, touch);
    if (j < nb) {
      P.stager->order_after_uploads(P.stream);
      set_band(j);
      enqueue_gemm(p, P.stream);
      hip_check(hipEventRecord(P.evc[j], P.stream), "hipEventRecord");
    }
  }
  hip_check(hipStreamSynchronize(P.stream), "hipStreamSynchronize");
  return m * n;
}

// from_f16 (gemm/linalg_native.mojo:564-576): float16 bits to float32.
int64_t host_from_f16(const std::vector<int64_t>& ad, const std::vector<int64_t>& pr) {
  if (pr.size() != 1) throw Fail("from_f16: params must contain 1 value (count)");
  const int64_t count = pr[0];
  if (count <= 0) throw Fail("from_f16: count must be positive, got " + std::to_string(count));
  Lease lease;
  HostPool& P = *lease.pool;
  float* dout = (float*)P.c.get((size_t)count * 4);
  uint16_t* din = (uint16_t*)P.a.get((size_t)count * 2);
  put(P, {span(ad[1], din, count * 2)});
  hip_check(mlg::run_f16_widen(dout, din, count, P.stream), "from_f16 launch");
  get(P, {span(ad[0], dout, count * 4)});
  return count;
}

int64_t host_convert(const std::vector<int64_t>& ad, const std::vector<int64_t>& pr, bool narrow) {
  const char* who = narrow ? "to_bf16" : "from_bf16";
  if (pr.size() != 1) throw Fail(std::string(who) + ": params must contain 1 value (count), got " + std::to_string(pr.size()));
  const int64_t count = pr[0];
  if (count <= 0) throw Fail(std::string(who) + ": count must be positive, got " + std::to_string(count));
  Lease lease;
  HostPool& P = *lease.pool;
  void* dout = P.c.get((size_t)count * (narrow ? 2 : 4));
  void* din = P.a.get((size_t)count * (narrow ? 4 : 2));
  put(P, {span(ad[1], din, count * (narrow ? 4 : 2))});
  if (narrow) hip_check(mlg::run_bf16_narrow((uint16_t*)dout, (const float*)din, count, P.stream), "to_bf16 launch");
  else hip_check(mlg::run_bf16_widen((float*)dout, (const uint16_t*)din, count, P.stream), "from_bf16 launch");
  get(P, {span(ad[0], dout, count * (narrow ? 2 : 4))});
  return count;
}

// ---- profile int8i32.v1 on host pointers (gemm/linalg_native.mojo:258-393; refusals :114-121)
int64_t host_q8_gemm(const std::vector<int64_t>& ad, const std::vector<int64_t>& pr) {
  if (pr.size() != 3) throw Fail("gemm_int8: params must contain 3 values (m, n, k), got " + std::to_string(pr.size()));
  const int64_t m = pr[0], n = pr[1], k = pr[2];
  if (m <= 0 || n <= 0 || k <= 0)
    throw Fail("gemm_int8: m, n and k must all be positive, got m=" + std::to_string(m) + " n=" +
               std::to_string(n) + " k=" + std::to_string(k));
  if (k > mlg::INT8_MAX_K)
    throw Fail("gemm_int8: k must be at most " + std::to_string(mlg::INT8_MAX_K) + " (contract L-7), got " +
               std::to_string(k));
  Lease lease;
  HostPool& P = *lease.pool;
  float* dc = (float*)P.c.get((size_t)(m * n) * 4);
  int8_t* dqa = (int8_t*)P.a.get((size_t)(m * k));
  int8_t* dqb = (int8_t*)P.b.get((size_t)(n * k));
  int32_t* dea = (int32_t*)P.x.get((size_t)m * 4);
  int32_t* deb = (int32_t*)P.y.get((size_t)n * 4);
  put(P, {span(ad[1], dqa, m * k), span(ad[2], dea, m * 4), span(ad[3], dqb, n * k), span(ad[4], deb, n * 4)});
  const int cus = num_cus_of_current_device();
  const int64_t wsb = mlg::q8_workspace_bytes(dqa, dqb, m, n, k, cus);
  void* dws = wsb > 0 ? P.w.get((size_t)wsb) : nullptr;
  hip_check(mlg::run_q8_gemm(dc, dqa, dea, dqb, deb, m, n, k, dws, cus, P.stream),
            "gemm_int8 launch");
  get(P, {span(ad[0], dc, m * n * 4)});
  return m * n;
}

int64_t host_q8_convert(const std::vector<int64_t>& ad, const std::vector<int64_t>& pr, bool quantize) {
  const char* who = quantize ? "quantize_int8" : "dequantize_int8";
  if (pr.size() != 2) throw Fail(std::string(who) + ": params must contain 2 values (rows, cols), got " + std::to_string(pr.size()));
  const int64_t rows = pr[0], cols = pr[1];
  if (rows <= 0 || cols <= 0)
    throw Fail(std::string(who) + ": rows and cols must be positive, got " + std::to_string(rows) + " x " + std::to_string(cols));
  Lease lease;
  HostPool& P = *lease.pool;
  float* df = (float*)P.c.get((size_t)(rows * cols) * 4);
  int8_t* dq = (int8_t*)P.a.get((size_t)(rows * cols));
  int32_t* de = (int32_t*)P.x.get((size_t)rows * 4);
  if (quantize) {  // addrs [codes, exponents, x]
    put(P, {span(ad[2], df, rows * cols * 4)});
    hip_check(mlg::run_q8_quantize(dq, de, df, rows, cols, P.stream), "quantize_int8 launch");
    get(P, {span(ad[0], dq, rows * cols), span(ad[1], de, rows * 4)});
  } else {  // addrs [y, codes, exponents]
    put(P, {span(ad[1], dq, rows * cols), span(ad[2], de, rows * 4)});
    hip_check(mlg::run_q8_dequantize(df, dq, de, rows, cols, P.stream), "dequantize_int8 launch");
    get(P, {span(ad[0], df, rows * cols * 4)});
  }
  return rows * cols;
}

// ---- profile int15i64.v1 on host pointers (gemm/linalg_native.mojo:395-510; refusals :114-121)
int64_t host_q15_gemm(const std::vector<int64_t>& ad, const std::vector<int64_t>& pr) {
  if (pr.size() != 3) throw Fail("gemm_int15: params must contain 3 values (m, n, k), got " + std::to_string(pr.size()));
  const int64_t m = pr[0], n = pr[1], k = pr[2];
  if (m <= 0 || n <= 0 || k <= 0)
    throw Fail("gemm_int15: m, n and k must all be positive, got m=" + std::to_string(m) + " n=" +
               std::to_string(n) + " k=" + std::to_string(k));
  if (k > mlg::INT15_MAX_K)
    throw Fail("gemm_int15: k must be at most " + std::to_string(mlg::INT15_MAX_K) + " (contract W-4), got " +
               std::to_string(k));
  Lease lease;  // addrs: c, a hi, a lo, a exponents, b hi, b lo, b exponents
  HostPool& P = *lease.pool;
  float* dc = (float*)P.c.get((size_t)(m * n) * 4);
  int8_t* dah = (int8_t*)P.a.get((size_t)(m * k));
  int8_t* dal = (int8_t*)P.a2.get((size_t)(m * k));
  int8_t* dbh = (int8_t*)P.b.get((size_t)(n * k));
  int8_t* dbl = (int8_t*)P.b2.get((size_t)(n * k));
  int32_t* dea = (int32_t*)P.x.get((size_t)m * 4);
  int32_t* deb = (int32_t*)P.y.get((size_t)n * 4);
  put(P, {span(ad[1], dah, m * k), span(ad[2], dal, m * k), span(ad[3], dea, m * 4), span(ad[4], dbh, n * k),
          span(ad[5], dbl, n * k), span(ad[6], deb, n * 4)});
  const int cus = num_cus_of_current_device();
  const int64_t wsb = mlg::q15_workspace_bytes(dah, dal, dbh, dbl, m, n, k, cus);
  void* dws = wsb > 0 ? P.w.get((size_t)wsb) : nullptr;
  hip_check(mlg::run_q15_gemm(dc, dah, dal, dea, dbh, dbl, deb, m, n, k, dws, cus, P.stream), "gemm_int15 launch");
  get(P, {span(ad[0], dc, m * n * 4)});
  return m * n;
}

int64_t host_q15_convert(const std::vector<int64_t>& ad, const std::vector<int64_t>& pr, bool quantize) {
  const char* who = quantize ? "quantize_int15" : "dequantize_int15";
  if (pr.size() != 2) throw Fail(std::string(who) + ": params must contain 2 values (rows, cols), got " + std::to_string(pr.size()));
  const int64_t rows = pr[0], cols = pr[1];
  if (rows <= 0 || cols <= 0)
    throw Fail(std::string(who) + ": rows and cols must be positive, got " + std::to_string(rows) + " x " + std::to_string(cols));
  Lease lease;
  HostPool& P = *lease.pool;
  float* df = (float*)P.c.get((size_t)(rows * cols) * 4);
  int8_t* dh = (int8_t*)P.a.get((size_t)(rows * cols));
  int8_t* dl = (int8_t*)P.a2.get((size_t)(rows * cols));
  int32_t* de = (int32_t*)P.x.get((size_t)rows * 4);
  if (quantize) {  // addrs [hi, lo, exponents, x]
    put(P, {span(ad[3], df, rows * cols * 4)});
    hip_check(mlg::run_q15_quantize(dh, dl, de, df, rows, cols, P.stream), "quantize_int15 launch");
    get(P, {span(ad[0], dh, rows * cols), span(ad[1], dl, rows * cols), span(ad[2], de, rows * 4)});
  } else {  // addrs [y, hi, lo, exponents]
    put(P, {span(ad[1], dh, rows * cols), span(ad[2], dl, rows * cols), span(ad[3], de, rows * 4)});
    hip_check(mlg::run_q15_dequantize(df, dh, dl, de, rows, cols, P.stream), "dequantize_int15 launch");
    get(P, {span(ad[0], df, rows * cols * 4)});
  }
  return rows * cols;
}

std::vector<int64_t> words(int64_t addr, int64_t n) {
  if (n < 0 || (n > 0 && addr == 0)) throw Fail("linalg native ABI: invalid descriptor span");
  std::vector<int64_t> v((size_t)n);
  if (n) memcpy(v.data(), (const void*)addr, (size_t)n * sizeof(int64_t));
  return v;
}

int64_t native_operation(int64_t op, const std::vector<int64_t>& a, const std::vector<int64_t>& p) {
  switch (op) {
    case 0:
      if (a.size() != 3) throw Fail("linalg native ABI: invalid gemm address count");
      if (p.size() != 4) throw Fail("gemm: params must contain 4 values (m, n, k, op), got " + std::to_string(p.size()));
      return host_gemm(a, p, mlg::T_F32, mlg::T_F32, false);
    case 1: {
      if (a.size() != 3) throw Fail("linalg native ABI: invalid gemm_bf16 address count");
      if (p.size() != 5)
        throw Fail("gemm_bf16: params must contain 5 values (m, n, k, op, a_bf16), got " + std::to_string(p.size()));
      std::vector<int64_t> p4(p.begin(), p.begin() + 4);
      return host_gemm(a, p4, p[4] != 0 ? mlg::T_BF16 : mlg::T_F32, mlg::T_BF16, false);
    }
    case 8:
      if (a.size() != 2) throw Fail("linalg native ABI: invalid to_bf16 address count");
      return host_convert(a, p, true);
    case 9:
      if (a.size() != 2) throw Fail("linalg native ABI: invalid from_bf16 address count");
      return host_convert(a, p, false);
    case 11:
    case 12:
    case 13:
    case 14:
      if (!a.empty() || !p.empty()) throw Fail("linalg native ABI: metadata takes no descriptors");
      return op == 11 ? NUMERIC_MODE_IDENTICAL
                      : (op == 12 ? PROFILE_VERSION : (op == 13 ? LOWBIT_PROFILE_VERSION : INT15_PROFILE_VERSION));
    case 15:
      if (a.size() != 4) throw Fail("linalg native ABI: invalid gemm_int8w address count");
      if (p.size() != 4) throw Fail("gemm_int8w: params must contain 4 values (m, n, k, op), got " + std::to_string(p.size()));
      return host_gemm(a, p, mlg::T_F32, mlg::T_I8, false);
    case 16:
      if (a.size() != 4) throw Fail("linalg native ABI: invalid gemm_bias address count");
      if (p.size() != 4) throw Fail("gemm_bias: params must contain 4 values (m, n, k, op), got " + std::to_string(p.size()));
      return host_gemm(a, p, mlg::T_F32, mlg::T_F32, true);
    case 2:
      if (a.size() != 5) throw Fail("linalg native ABI: invalid gemm_int8 address count");
      return host_q8_gemm(a, p);
    case 3:
      if (a.size() != 3) throw Fail("linalg native ABI: invalid quantize_int8 address count");
      return host_q8_convert(a, p, true);
    case 4:
      if (a.size() != 3) throw Fail("linalg native ABI: invalid dequantize_int8 address count");
      return host_q8_convert(a, p, false);
    case 5:
      if (a.size() != 7) throw Fail("linalg native ABI: invalid gemm_int15 address count");
      return host_q15_gemm(a, p);
    case 6:
      if (a.size() != 4) throw Fail("linalg native ABI: invalid quantize_int15 address count");
      return host_q15_convert(a, p, true);
    case 7:
      if (a.size() != 4) throw Fail("linalg native ABI: invalid dequantize_int15 address count");
      return host_q15_convert(a, p, false);
    case 10:
      if (a.size() != 2) throw Fail("linalg native ABI: invalid from_f16 address count");
      return host_from_f16(a, p);
    default:
      throw Fail("linalg native ABI: unknown operation");
  }
}

}  // namespace

extern "C" {

int64_t linalg_native_v1(int64_t op, int64_t addrs, int64_t n_addrs, int64_t ints, int64_t n_ints,
                         int64_t floats, int64_t n_floats, int64_t result, int64_t err_ctx,
                         mlg_sink_t sink) {
  (void)floats;
  try {
    if (result == 0 || n_floats != 0) throw Fail("linalg native ABI: invalid result or scalar span");
    std::vector<int64_t> a = words(addrs, n_addrs);
    std::vector<int64_t> p = words(ints, n_ints);
    *(int64_t*)result = native_operation(op, a, p);
    return 0;
  } catch (const std::exception& ex) {
    if (sink) {
      const std::string msg = ex.what();
      sink(err_ctx, (int64_t)(uintptr_t)msg.data(), (int64_t)msg.size());
    }
    return 1;
  }
}

const char* mlg_abi_name(void) { return "mojolearn.linalg.v1"; }

int mlg_gemm_f32(float* c, const float* a, const float* b, const float* bias, int64_t m, int64_t n,
                 int64_t k, int32_t op, int64_t leaf, void* stream) {
  return guarded([&] {
    mlg::GemmProblem p{};
    p.c = c; p.a = a; p.b = b; p.bias = bias; p.m = m; p.n = n; p.k = k; p.op = op;
    p.a_type = mlg::T_F32; p.b_type = mlg::T_F32; p.leaf = leaf;
    enqueue_gemm(p, (hipStream_t)stream);
  });
}

int mlg_gemm_bf16w(float* c, const void* a, const uint16_t* b, const float* bias, int64_t m,
                   int64_t n, int64_t k, int32_t op, int32_t a_is_bf16, int64_t leaf, void* stream) {
  return guarded([&] {
    mlg::GemmProblem p{};
    p.c = c; p.a = a; p.b = b; p.bias = bias; p.m = m; p.n = n; p.k = k; p.op = op;
    p.a_type = a_is_bf16 ? mlg::T_BF16 : mlg::T_F32; p.b_type = mlg::T_BF16; p.leaf = leaf;
    enqueue_gemm(p, (hipStream_t)stream);
  });
}

int mlg_gemm_int8w(float* c, const float* a, const int8_t* codes, const float* scales,
                   const float* bias, int64_t m, int64_t n, int64_t k, int32_t op, int64_t leaf,
                   void* stream) {
  return guarded([&] {
    mlg::GemmProblem p{};
    p.c = c; p.a = a; p.b = codes; p.scales = scales; p.bias = bias; p.m = m; p.n = n; p.k = k;
    p.op = op; p.a_type = mlg::T_F32; p.b_type = mlg::T_I8; p.leaf = leaf;
    enqueue_gemm(p, (hipStream_t)stream);
  });
}

}  // extern "C"

namespace {

// The caller's operand views A(i, p) = a[i a_si + p a_sp], B(p, j) = b[p b_sp + j b_sj] as a
// stored layout of the tile kernel: A row-major unless a_si == 1 != a_sp (then k-major,
// OP_TN), B k-major unless b_sp == 1 != b_sj (then index-major, OP_NT); A and B both
// transposed has no kernel, so A is then read as row-major (the repack gathers it).
void view_layout(mlg::GemmProblem& p, int64_t a_si, int64_t a_sp, int64_t b_sp, int64_t b_sj) {
  bool a_t = a_si == 1 && a_sp != 1;
  const bool b_t = b_sp == 1 && b_sj != 1;
  if (a_t && b_t) a_t = false;
  p.op = a_t ? mlg::OP_TN : (b_t ? mlg::OP_NT : mlg::OP_NN);
  p.strided = 1;
  if (a_t) { p.a_rs = a_sp; p.a_cs = a_si; } else { p.a_rs = a_si; p.a_cs = a_sp; }
  if (b_t) { p.b_rs = b_sj; p.b_cs = b_sp; } else { p.b_rs = b_sp; p.b_cs = b_sj; }
  p.a_type = mlg::T_F32;
  p.b_type = mlg::T_F32;
  p.seq = 1;
}

void refuse_partition(const char* who, int64_t k, int64_t leaf, int64_t p_count) {
  if (k <= 0 || leaf <= 0 || p_count <= 0 || (p_count - 1) * leaf >= k || p_count * leaf < k)
    throw Fail(std::string(who) + ": (leaf, p_count) does not partition k");
}

}  // namespace

extern "C" {

int mlg_gemm_leaf_ptr(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k, int64_t leaf,
                      int64_t p_count, int64_t a_si, int64_t a_sp, int64_t b_sp, int64_t b_sj, void* stream) {
  return guarded([&] {
    if (m <= 0 || n <= 0) return;
    refuse_partition("identical_gemm_leaf_ptr_into", k, leaf, p_count);
    mlg::GemmProblem p{};
    view_layout(p, a_si, a_sp, b_sp, b_sj);
    p.c = c; p.a = a; p.b = b; p.m = m; p.n = n; p.k = k; p.leaf = leaf;
    enqueue_gemm(p, (hipStream_t)stream);
  });
}

int mlg_gemm_leaf_ptr_epi(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k, int64_t leaf,
                          int64_t p_count, int64_t a_si, int64_t a_sp, int64_t b_sp, int64_t b_sj, int32_t epi,
                          const float* epi_p, int32_t epi_i, void* stream) {
  return guarded([&] {
    if (epi != mlg::EPI_PLUS_BIAS && epi != mlg::EPI_BIAS_ACT && epi != mlg::EPI_ACT_BWD)
      throw Fail("identical_gemm_leaf_ptr_epi_into: a store epilogue kind that reads a second buffer, got " +
                 std::to_string(epi));
    if (m <= 0 || n <= 0) return;
    refuse_partition("identical_gemm_leaf_ptr_epi_into", k, leaf, p_count);
    if (!epi_p) throw Fail("identical_gemm_leaf_ptr_epi_into: the epilogue's second buffer is null");
    mlg::GemmProblem p{};
    view_layout(p, a_si, a_sp, b_sp, b_sj);
    p.c = c; p.a = a; p.b = b; p.m = m; p.n = n; p.k = k; p.leaf = leaf;
    // the follower fused into the product's store (one launch, or the fold's when the leaves
    // are split into groups)
    if (epi == mlg::EPI_PLUS_BIAS) {
      p.bias = epi_p;
    } else {
      p.epi = epi; p.epi_p = epi_p; p.act = epi_i;
    }
    enqueue_gemm(p, (hipStream_t)stream);
  });
}

int mlg_seq_gemm(float* c, const float* a, const float* b, int64_t m, int64_t n, int64_t k, int64_t a_si,
                 int64_t a_sp, int64_t b_sp, int64_t b_sj, int64_t ldc, int32_t accumulate, void* stream) {
  return guarded([&] {
    if (m < 0 || n < 0 || k < 0)
      throw Fail("op_gemm: m, n and k must be >= 0, got " + shape_text(m, n, k));
    if (m == 0 || n == 0) return;
    if (m > 1 && ldc < n) throw Fail("op_gemm: the row stride of C (" + std::to_string(ldc) + ") is below n");
    if (k == 0) {
      hip_check(mlg::run_follow(c, ldc, m, n, accumulate ? 0 : 1, mlg::EPI_NONE, nullptr, 0, (hipStream_t)stream),
                "follower launch");
      return;
    }
    mlg::GemmProblem p{};
    view_layout(p, a_si, a_sp, b_sp, b_sj);
    p.c = c; p.a = a; p.b = b; p.m = m; p.n = n; p.k = k; p.leaf = k;
    p.ldc = ldc; p.seed = accumulate ? 1 : 0;
    enqueue_gemm(p, (hipStream_t)stream);
  });
}

int mlg_follow(float* c, int64_t ldc, int64_t m, int64_t n, int32_t epi, const float* epi_p, int32_t epi_i,
               void* stream) {
  return guarded([&] {
    if (epi != mlg::EPI_NONE && epi != mlg::EPI_PLUS_BIAS && epi != mlg::EPI_BIAS_ACT && epi != mlg::EPI_ACT_BWD)
      throw Fail("mlg_follow: epilogue kind must be 0, 3, 4 or 5, got " + std::to_string(epi));
    if (m <= 0 || n <= 0) return;
    if (epi != mlg::EPI_NONE && !epi_p) throw Fail("mlg_follow: the epilogue's second buffer is null");
    hip_check(mlg::run_follow(c, ldc, m, n, 0, epi, epi_p, epi_i, (hipStream_t)stream), "follower launch");
  });
}

int64_t mlg_gemm_workspace_bytes(int64_t m, int64_t n, int64_t k, int32_t op, int32_t a_type,
                                 int32_t b_type, int64_t leaf) {
  return mlg_gemm_workspace_bytes_for(nullptr, nullptr, m, n, k, op, a_type, b_type, leaf);
}

int64_t mlg_gemm_workspace_bytes_for(const void* a, const void* b, int64_t m, int64_t n, int64_t k, int32_t op,
                                     int32_t a_type, int32_t b_type, int64_t leaf) {
  int64_t out = -1;
  guarded([&] {
    mlg::GemmProblem p{};
    p.a = a; p.b = b; p.m = m; p.n = n; p.k = k; p.op = op; p.a_type = a_type; p.b_type = b_type; p.leaf = leaf;
    const int cus = num_cus_of_current_device();
    check_problem(p, cus);
    out = mlg::gemm_workspace_floats(p, cus) * (int64_t)sizeof(float);
  });
  return out;
}

int64_t mlg_gemm_counter_bytes(int64_t m, int64_t n, int64_t k, int32_t op, int32_t a_type, int32_t b_type,
                               int64_t leaf) {
  mlg::GemmProblem p{};
  p.m = m; p.n = n; p.k = k; p.op = op; p.a_type = a_type; p.b_type = b_type; p.leaf = leaf;
  return mlg::gemm_counter_count(p) * (int64_t)sizeof(unsigned int);
}

int64_t mlg_gemm_route(const void* a, const void* b, int64_t m, int64_t n, int64_t k, int32_t op, int32_t a_type,
                       int32_t b_type, int64_t leaf, int32_t num_cus) {
  int64_t out = -1;
  guarded([&] {
    mlg::GemmProblem p{};
    p.a = a; p.b = b; p.m = m; p.n = n; p.k = k; p.op = op; p.a_type = a_type; p.b_type = b_type; p.leaf = leaf;
    const int cus = num_cus > 0 ? num_cus : num_cus_of_current_device();
    check_problem(p, cus);
    unsigned route = 0;
    hip_check(mlg::run_gemm(p, nullptr, cus, nullptr, &route), "gemm route");
    out = route;
  });
  return out;
}

// The memory floors of the skinny products, for bench.py (not part of the reference's
// interface, so not in include/mlgemm.h).
int64_t mlg_int8w_packed_bytes(int64_t k, int64_t n) { return mlg::int8w_packed_bytes(k, n); }

int mlg_int8w_pack(void* dst, const int8_t* codes, int64_t k, int64_t n, void* stream) {
  return guarded([&] {
    if (mlg::int8w_packed_bytes(k, n) < 0)
      throw Fail("mlg_int8w_pack: k must be a positive multiple of 128 with at most 1024 leaves, n >= 1; got k=" +
                 std::to_string(k) + ", n=" + std::to_string(n));
    if (!dst || !codes) throw Fail("mlg_int8w_pack: null buffer");
    if ((uintptr_t)dst % 16 != 0) throw Fail("mlg_int8w_pack: the packed buffer must be 16-byte aligned");
    hip_check(mlg::run_int8w_pack(dst, codes, k, n, static_cast<hipStream_t>(stream)), "int8w pack launch");
  });
}

int64_t mlg_gemv_int8w_packed_workspace_bytes(int64_t m, int64_t n, int64_t k) {
  if (!mlg::gemv_packed_limit(m, n, k, nullptr).empty()) return -1;
  return mlg::gemv_packed_workspace_floats(m, n, k) * (int64_t)sizeof(float);
}

int64_t mlg_gemv_int8w_packed_counter_bytes(int64_t m, int64_t n, int64_t k) {
  if (!mlg::gemv_packed_limit(m, n, k, nullptr).empty()) return -1;
  return mlg::gemv_packed_counter_count(m, n, k) * (int64_t)sizeof(unsigned int);
}

int mlg_gemv_int8w_packed(float* c, const float* x, const void* packed, const float* scales, const float* bias,
                          int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes, void* stream) {
  return guarded([&] {
    const std::string why = mlg::gemv_packed_limit(m, n, k, packed);
    if (!why.empty()) throw Fail("mlg_gemv_int8w_packed: " + why + "; got " + shape_text(m, n, k));
    if (!c || !x || !packed || !scales) throw Fail("mlg_gemv_int8w_packed: null buffer");
    const int64_t need = mlg::gemv_packed_workspace_floats(m, n, k) * (int64_t)sizeof(float);
    if (need > 0 && (!workspace || workspace_bytes < need))
      throw Fail("mlg_gemv_int8w_packed: workspace of " + std::to_string(workspace_bytes) + " bytes is smaller than the " +
                 std::to_string(need) + " this product needs");
    hip_check(mlg::run_gemv_packed(c, x, packed, scales, bias, m, n, k, static_cast<float*>(workspace),
                                   num_cus_of_current_device(), static_cast<hipStream_t>(stream)),
              "packed gemv launch");
  });
}

int mlg_stream_read(const void* w, int64_t rows, int64_t cols, int32_t pattern, uint32_t* sink, void* stream) {
  return guarded([&] {
    hip_check(mlg::run_stream_read(w, rows, cols, pattern, sink, static_cast<hipStream_t>(stream)),
              "stream_read launch (pattern 0: 16-byte aligned, 16-byte multiple; pattern 1: rows a "
              "multiple of 512, cols of 256; pattern 2: rows a multiple of 4096, cols of 64, below 2^31 bytes)");
  });
}

int mlg_gemm_ws(float* c, const void* a, const void* b, const float* scales, const float* bias,
                int64_t m, int64_t n, int64_t k, int32_t op, int32_t a_type, int32_t b_type,
                int64_t leaf, void* workspace, int64_t workspace_bytes, void* stream) {
  return guarded([&] {
    if (a_type != mlg::T_F32 && a_type != mlg::T_BF16) throw Fail("mlgemm: a_type must be 0 (f32) or 1 (bf16)");
    if (b_type < mlg::T_F32 || b_type > mlg::T_I8) throw Fail("mlgemm: b_type must be 0 (f32), 1 (bf16) or 2 (int8)");
    if (a_type == mlg::T_BF16 && b_type != mlg::T_BF16) throw Fail("mlgemm: a bf16 A needs a bf16 B");
    mlg::GemmProblem p{};
    p.c = c; p.a = a; p.b = b; p.scales = scales; p.bias = bias; p.m = m; p.n = n; p.k = k; p.op = op;
    p.a_type = a_type; p.b_type = b_type; p.leaf = leaf;
    enqueue_gemm(p, (hipStream_t)stream, workspace, workspace_bytes < 0 ? 0 : workspace_bytes);
  });
}

}  // extern "C"

namespace {

// The workspace of mlg_gemm_noalloc: one array per GPU, held from the code object's load until
// the process ends.  In host code `scratch` names a host-side stand-in, never device memory: the
// entry uses only the address hipGetSymbolAddress gives for the current device.
constexpr int64_t NOALLOC_SCRATCH_BYTES = int64_t(32) << 20;
static __device__ __align__(256) char scratch[NOALLOC_SCRATCH_BYTES];

// This device's address of `scratch`, looked up once per device with that device current.
void* scratch_on_current_device() {
  constexpr int MAX_DEVICES = 64;
  static std::mutex mu;
  static void* ptr[MAX_DEVICES] = {};
  int dev = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= MAX_DEVICES) throw Fail("mlg_gemm_noalloc: device ordinal out of range");
  std::lock_guard<std::mutex> lock(mu);
  if (!ptr[dev]) {
    void* p = nullptr;
    hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!p) throw Fail("mlg_gemm_noalloc: hipGetSymbolAddress gave no address for the scratch array");
    ptr[dev] = p;
  }
  return ptr[dev];
}

}  // namespace

extern "C" {

int mlg_gemm_noalloc(float* c, const void* a, const void* b, const float* scales, const float* bias, int64_t m,
                     int64_t n, int64_t k, int32_t op, int32_t a_type, int32_t b_type, int64_t leaf, void* stream) {
  return guarded([&] {
    if (a_type != mlg::T_F32 && a_type != mlg::T_BF16) throw Fail("mlgemm: a_type must be 0 (f32) or 1 (bf16)");
    if (b_type < mlg::T_F32 || b_type > mlg::T_I8) throw Fail("mlgemm: b_type must be 0 (f32), 1 (bf16) or 2 (int8)");
    if (a_type == mlg::T_BF16 && b_type != mlg::T_BF16) throw Fail("mlgemm: a bf16 A needs a bf16 B");
    mlg::GemmProblem p{};
    p.c = c; p.a = a; p.b = b; p.scales = scales; p.bias = bias; p.m = m; p.n = n; p.k = k; p.op = op;
    p.a_type = a_type; p.b_type = b_type; p.leaf = leaf;
    const int cus = num_cus_of_current_device();
    check_problem(p, cus);
    if (p.m == 0 || p.n == 0) return;
    const int64_t need = mlg::gemm_workspace_floats(p, cus) * (int64_t)sizeof(float);
    if (need > NOALLOC_SCRATCH_BYTES)
      throw Fail("mlg_gemm_noalloc: this product needs " + std::to_string(need) + " bytes of workspace, more than the " +
                 std::to_string(NOALLOC_SCRATCH_BYTES) + " of the library's scratch array; use mlg_gemm_ws");
    void* ws = need > 0 ? scratch_on_current_device() : nullptr;
    // the array keeps the last call's contents: its completion counters start at zero here
    // (a kernel, not a memset: the call may be captured in a graph)
    const int64_t ncnt = mlg::gemm_counter_count(p);
    if (ncnt > 0) hip_check(mlg::run_zero_words(static_cast<unsigned int*>(ws), ncnt, (hipStream_t)stream),
                            "counter clear launch");
    enqueue_gemm(p, (hipStream_t)stream, ws, need);
  });
}

int mlg_bf16_widen(float* out, const uint16_t* in, int64_t count, void* stream) {
  return guarded([&] { hip_check(mlg::run_bf16_widen(out, in, count, (hipStream_t)stream), "from_bf16 launch"); });
}

int mlg_bf16_narrow(uint16_t* out, const float* in, int64_t count, void* stream) {
  return guarded([&] { hip_check(mlg::run_bf16_narrow(out, in, count, (hipStream_t)stream), "to_bf16 launch"); });
}

int mlg_int8_quantize(int8_t* codes, int32_t* exponents, const float* x, int64_t rows, int64_t cols, void* stream) {
  return guarded([&] {
    if (rows < 0 || cols < 0) throw Fail("quantize_int8: rows and cols must be >= 0");
    if (rows > 0 && cols > 0 && (!codes || !exponents || !x)) throw Fail("quantize_int8: null pointer");
    hip_check(mlg::run_q8_quantize(codes, exponents, x, rows, cols, (hipStream_t)stream), "quantize_int8 launch");
  });
}

int mlg_int8_dequantize(float* out, const int8_t* codes, const int32_t* exponents, int64_t rows, int64_t cols,
                        void* stream) {
  return guarded([&] {
    if (rows < 0 || cols < 0) throw Fail("dequantize_int8: rows and cols must be >= 0");
    if (rows > 0 && cols > 0 && (!codes || !exponents || !out)) throw Fail("dequantize_int8: null pointer");
    hip_check(mlg::run_q8_dequantize(out, codes, exponents, rows, cols, (hipStream_t)stream), "dequantize_int8 launch");
  });
}

static void check_q8_args(float* c, const int8_t* qa, const int32_t* ea, const int8_t* qb, const int32_t* eb,
                          int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0)
    throw Fail("gemm_int8: m, n and k must all be positive, got m=" + std::to_string(m) + " n=" +
               std::to_string(n) + " k=" + std::to_string(k));
  if (k > mlg::INT8_MAX_K)
    throw Fail("gemm_int8: k must be at most " + std::to_string(mlg::INT8_MAX_K) + " (contract L-7), got " +
               std::to_string(k));
  if (!c || !ea || !eb || !qa || !qb) throw Fail("gemm_int8: null operand pointer");
}

int mlg_gemm_int8i32(float* c, const int8_t* qa, const int32_t* ea, const int8_t* qb, const int32_t* eb,
                     int64_t m, int64_t n, int64_t k, void* stream) {
  return guarded([&] {
    check_q8_args(c, qa, ea, qb, eb, m, n, k);
    hipStream_t s = (hipStream_t)stream;
    const int cus = num_cus_of_current_device();
    const int64_t wsb = mlg::q8_workspace_bytes(qa, qb, m, n, k, cus);
    void* ws = nullptr;
    if (wsb > 0) hip_check(hipMallocAsync(&ws, (size_t)wsb, s), "hipMallocAsync");
    hipError_t e = mlg::run_q8_gemm(c, qa, ea, qb, eb, m, n, k, ws, cus, s);
    if (ws) {
      hipError_t f = hipFreeAsync(ws, s);
      if (e == hipSuccess) e = f;
    }
    hip_check(e, "gemm_int8 launch");
  });
}

int64_t mlg_gemm_int8i32_workspace_bytes(const int8_t* qa, const int8_t* qb, int64_t m, int64_t n, int64_t k) {
  int64_t r = -1;
  const int rc = guarded([&] {
    if (m <= 0 || n <= 0 || k <= 0 || k > mlg::INT8_MAX_K) throw Fail("gemm_int8: invalid shape");
    r = mlg::q8_workspace_bytes(qa, qb, m, n, k, num_cus_of_current_device());
  });
  return rc == 0 ? r : -1;
}

int mlg_gemm_int8i32_ws(float* c, const int8_t* qa, const int32_t* ea, const int8_t* qb, const int32_t* eb,
                        int64_t m, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes, void* stream) {
  return guarded([&] {
    check_q8_args(c, qa, ea, qb, eb, m, n, k);
    const int cus = num_cus_of_current_device();
    const int64_t need = mlg::q8_workspace_bytes(qa, qb, m, n, k, cus);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
      throw Fail("gemm_int8: workspace of " + std::to_string(workspace_bytes) + " bytes, this product needs " +
                 std::to_string(need));
    hip_check(mlg::run_q8_gemm(c, qa, ea, qb, eb, m, n, k, need > 0 ? workspace : nullptr, cus,
                               (hipStream_t)stream),
              "gemm_int8 launch");
  });
}

int mlg_f16_widen(float* out, const uint16_t* in, int64_t count, void* stream) {
  return guarded([&] { hip_check(mlg::run_f16_widen(out, in, count, (hipStream_t)stream), "from_f16 launch"); });
}

int mlg_int15_quantize(int8_t* hi, int8_t* lo, int32_t* exponents, const float* x, int64_t rows, int64_t cols,
                       void* stream) {
  return guarded([&] {
    if (rows < 0 || cols < 0) throw Fail("quantize_int15: rows and cols must be >= 0");
    if (rows > 0 && cols > 0 && (!hi || !lo || !exponents || !x)) throw Fail("quantize_int15: null pointer");
    hip_check(mlg::run_q15_quantize(hi, lo, exponents, x, rows, cols, (hipStream_t)stream), "quantize_int15 launch");
  });
}

int mlg_int15_dequantize(float* out, const int8_t* hi, const int8_t* lo, const int32_t* exponents, int64_t rows,
                         int64_t cols, void* stream) {
  return guarded([&] {
    if (rows < 0 || cols < 0) throw Fail("dequantize_int15: rows and cols must be >= 0");
    if (rows > 0 && cols > 0 && (!out || !hi || !lo || !exponents)) throw Fail("dequantize_int15: null pointer");
    hip_check(mlg::run_q15_dequantize(out, hi, lo, exponents, rows, cols, (hipStream_t)stream),
              "dequantize_int15 launch");
  });
}

static void check_q15_args(float* c, const int8_t* ah, const int8_t* al, const int32_t* ea, const int8_t* bh,
                           const int8_t* bl, const int32_t* eb, int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0)
    throw Fail("gemm_int15: m, n and k must all be positive, got m=" + std::to_string(m) + " n=" +
               std::to_string(n) + " k=" + std::to_string(k));
  if (k > mlg::INT15_MAX_K)
    throw Fail("gemm_int15: k must be at most " + std::to_string(mlg::INT15_MAX_K) + " (contract W-4), got " +
               std::to_string(k));
  if (!c || !ah || !al || !ea || !bh || !bl || !eb) throw Fail("gemm_int15: null operand pointer");
}

int mlg_gemm_int15i64(float* c, const int8_t* ah, const int8_t* al, const int32_t* ea, const int8_t* bh,
                      const int8_t* bl, const int32_t* eb, int64_t m, int64_t n, int64_t k, void* stream) {
  return guarded([&] {
    check_q15_args(c, ah, al, ea, bh, bl, eb, m, n, k);
    hipStream_t s = (hipStream_t)stream;
    const int cus = num_cus_of_current_device();
    const int64_t wsb = mlg::q15_workspace_bytes(ah, al, bh, bl, m, n, k, cus);
    void* ws = nullptr;
    if (wsb > 0) hip_check(hipMallocAsync(&ws, (size_t)wsb, s), "hipMallocAsync");
    hipError_t e = mlg::run_q15_gemm(c, ah, al, ea, bh, bl, eb, m, n, k, ws, cus, s);
    if (ws) {
      hipError_t f = hipFreeAsync(ws, s);
      if (e == hipSuccess) e = f;
    }
    hip_check(e, "gemm_int15 launch");
  });
}

int64_t mlg_gemm_int15i64_workspace_bytes(const int8_t* ah, const int8_t* al, const int8_t* bh, const int8_t* bl,
                                          int64_t m, int64_t n, int64_t k) {
  int64_t r = -1;
  const int rc = guarded([&] {
    if (m <= 0 || n <= 0 || k <= 0 || k > mlg::INT15_MAX_K) throw Fail("gemm_int15: invalid shape");
    r = mlg::q15_workspace_bytes(ah, al, bh, bl, m, n, k, num_cus_of_current_device());
  });
  return rc == 0 ? r : -1;
}

int mlg_gemm_int15i64_ws(float* c, const int8_t* ah, const int8_t* al, const int32_t* ea, const int8_t* bh,
                         const int8_t* bl, const int32_t* eb, int64_t m, int64_t n, int64_t k, void* workspace,
                         int64_t workspace_bytes, void* stream) {
  return guarded([&] {
    check_q15_args(c, ah, al, ea, bh, bl, eb, m, n, k);
    const int cus = num_cus_of_current_device();
    const int64_t need = mlg::q15_workspace_bytes(ah, al, bh, bl, m, n, k, cus);
    if (need > 0 && (workspace == nullptr || workspace_bytes < need))
      throw Fail("gemm_int15: workspace of " + std::to_string(workspace_bytes) + " bytes, this product needs " +
                 std::to_string(need));
    hip_check(mlg::run_q15_gemm(c, ah, al, ea, bh, bl, eb, m, n, k, need > 0 ? workspace : nullptr, cus,
                                (hipStream_t)stream),
              "gemm_int15 launch");
  });
}

const char* mlg_last_error(void) { return g_last_error.c_str(); }

int64_t mlg_numeric_mode(void) { return NUMERIC_MODE_IDENTICAL; }
int64_t mlg_profile_version(void) { return PROFILE_VERSION; }
int64_t mlg_lowbit_profile_version(void) { return LOWBIT_PROFILE_VERSION; }

}  // extern "C"

// runtime.hpp -- host runtime of the MI355X lookup library: errors, thread
// pool, execution contexts and buffer staging.
//
// Reference counterparts (file:line in /root/reference):
//   errors -> C status      src/nve_c_api_internal.hpp:48-92, include/common.hpp
//   thread pool             include/thread_pool.hpp:50-151, src/thread_pool.cpp:97-160
//   execution context       include/execution_context.hpp:34-84, include/layer_utils.hpp:66-199
//   buffer staging          include/buffer_wrapper.hpp:34-123
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <condition_variable>
#include <deque>
#include <functional>
#include <future>
#include <map>
#include <memory>
#include <mutex>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/nve_c_api.h"

namespace nve_amd {

// ---------------------------------------------------------------------------
// errors: each carries the C status it maps to
// ---------------------------------------------------------------------------
class Error : public std::runtime_error {
 public:
  Error(nve_status_t status, const std::string& msg) : std::runtime_error(msg), status_(status) {}
  nve_status_t status() const { return status_; }

 private:
  nve_status_t status_;
};

template <typename... T>
std::string cat(const T&... parts) {
  std::ostringstream os;
  (os << ... << parts);
  return os.str();
}

#define NVE_CHECK_ARG(cond, ...)                                                        \
  do {                                                                                  \
    if (!(cond)) throw ::nve_amd::Error(NVE_ERROR_INVALID_ARGUMENT, ::nve_amd::cat(__VA_ARGS__)); \
  } while (0)
#define NVE_CHECK(cond, ...)                                                        \
  do {                                                                              \
    if (!(cond)) throw ::nve_amd::Error(NVE_ERROR_RUNTIME, ::nve_amd::cat(__VA_ARGS__)); \
  } while (0)
#define NVE_NOT_IMPLEMENTED(...) \
  throw ::nve_amd::Error(NVE_ERROR_NOT_IMPLEMENTED, ::nve_amd::cat(__VA_ARGS__))
// A failed call also resets the thread's last-error state, so that a later
// launch check (hipGetLastError after a kernel launch) does not report it again.
#define NVE_HIP(expr)                                                                        \
  do {                                                                                       \
    const hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess)                                                                    \
      (void)hipGetLastError(), throw ::nve_amd::Error(e_ == hipErrorOutOfMemory ? NVE_ERROR_OUT_OF_MEMORY : NVE_ERROR_CUDA, \
                             ::nve_amd::cat(#expr, ": ", hipGetErrorName(e_), " (",              \
                                            hipGetErrorString(e_), ")"));                    \
  } while (0)

// Makes `device` current for the scope (ScopedDevice, include/cuda_support.hpp).
class ScopedDevice {
 public:
  explicit ScopedDevice(int device);
  ~ScopedDevice();

 private:
  int prev_ = -1;
};

// Runs a table operation on `run` (a table's private stream) when it is set,
// else on `caller`: work queued on `caller` before the scope happens-before
// the operation, and work queued on `caller` after the scope waits for it
// (StreamCoordinator, layer_utils.hpp:88-118).  The ordering uses one reusable
// event per thread and device: a stream wait binds to the record made before it.
class StreamQueue {
 public:
  StreamQueue(hipStream_t caller, hipStream_t run);
  ~StreamQueue();
  StreamQueue(const StreamQueue&) = delete;
  StreamQueue& operator=(const StreamQueue&) = delete;
  const hipStream_t stream;

 private:
  const hipStream_t caller_;
};

// The lookup streams of the execution contexts that read one table (a
// ContextRegistry, layer_utils.hpp:66-82).  A modify that must not overwrite
// rows a queued lookup may still read orders itself after every lookup queued
// so far, on the device or on the host, instead of draining the whole device
// (ec_set_associative_device_modify.cuh:428-446): streams of other work, a
// model's compute streams for one, are left alone.  A stream is counted once
// per context that registered it.
class LookupStreams {
 public:
  void add(hipStream_t s);
  void remove(hipStream_t s);
  // Work queued on `s` after this call starts after every lookup queued so
  // far on the registered streams (one event record and stream wait each).
  void order_before(hipStream_t s);
  // Returns when every lookup queued so far on the registered streams is done.
  void drain();

 private:
  std::mutex mu_;
  std::map<hipStream_t, int> streams_;
};

// ---------------------------------------------------------------------------
// thread pool (SimpleThreadPool: default workers = max(cores - 2, 1))
// ---------------------------------------------------------------------------
class ThreadPool {
 public:
  explicit ThreadPool(int64_t num_workers);
  ~ThreadPool();
  std::future<void> submit(std::function<void()> task);
  int64_t num_workers() const { return (int64_t)workers_.size(); }

  static std::shared_ptr<ThreadPool> default_pool();
  static void configure_default(int64_t num_workers);

 private:
  void main_();
  std::vector<std::thread> workers_;
  std::deque<std::packaged_task<void()>> queue_;
  std::mutex mu_;
  std::condition_variable cv_;
  bool stop_ = false;
};

// Fields of the thread-pool JSON ({"implementation": "simple", "num_workers": N,
// ...}): the text must be valid JSON (a parse error is NVE_ERROR_RUNTIME); a
// field is read from a top-level object, dflt when absent.
int64_t json_int_field(const char* json, const char* field, int64_t dflt);
std::string json_string_field(const char* json, const char* field, const std::string& dflt);

// ---------------------------------------------------------------------------
// execution context: streams, named grow-only scratch buffers, a miss counter
// and the futures of work handed to the thread pool.
// ---------------------------------------------------------------------------
class ExecutionContext {
 public:
  ExecutionContext(int device, hipStream_t lookup, hipStream_t modify,
                   std::shared_ptr<ThreadPool> pool);
  virtual ~ExecutionContext();

  int device() const { return device_; }
  hipStream_t lookup_stream() const { return lookup_; }
  hipStream_t modify_stream() const { return modify_; }
  ThreadPool& pool() { return *pool_; }

  // Device (host = false) or pinned host (host = true) buffer of at least
  // `bytes`, kept under `name` and reused by later calls on this context.
  void* buffer(const std::string& name, size_t bytes, bool host = false);
  // Ordinary (pageable, 64-byte aligned) host memory under `name`: what a
  // context of the host layer uses, so that it never enters the HIP runtime.
  void* host_buffer(const std::string& name, size_t bytes);

  // Lookup counter of a host table (LinearHostTable counts resolved keys).
  int64_t& host_lookup_counter() { return host_counter_; }

  // Register this context's lookup stream with the table that `streams`
  // belongs to, until the context is destroyed.
  void watch(const std::shared_ptr<LookupStreams>& streams);

  // Device counter of cache misses (zeroed by reset_misses on lookup_stream).
  // Asking for it marks it as possibly counting; read_misses returns its total
  // (a kernel writes it into pinned host memory, then lookup_stream is
  // synchronized), take_misses does the same and zeroes the counter, and
  // prepare_misses zeroes it only when something may have counted since.
  unsigned long long* miss_counter();
  void reset_misses();
  int64_t read_misses();
  int64_t take_misses();
  void prepare_misses();

  void add_pending(std::future<void> f);
  void wait();

 private:
  struct Buf {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool host = false;
    bool plain = false;  // host_buffer: malloc'd, not pinned
  };
  int device_;
  hipStream_t lookup_, modify_;
  std::shared_ptr<ThreadPool> pool_;
  std::mutex bufs_mu_;  // the lookup thread and a pool task (auto-insert) share buffers
  std::map<std::string, Buf> bufs_;
  unsigned long long* misses_ = nullptr;
  unsigned long long* miss_total_ = nullptr;  // pinned host word the total is written to
  bool misses_clean_ = false;                  // the counter is zero on lookup_stream
  int64_t misses_total(int reset);
  int64_t host_counter_ = 0;
  std::mutex pending_mu_;
  std::vector<std::future<void>> pending_;
  std::vector<std::shared_ptr<LookupStreams>> watched_;
};

// ---------------------------------------------------------------------------
// staging of caller buffers that may live in host or device memory
// ---------------------------------------------------------------------------
enum class MemKind { Device, PinnedHost, PageableHost };
MemKind mem_kind(const void* p);

// Device-readable view of `bytes` at `p`: p itself when the GPU can read it,
// else a copy into the context buffer `name` (queued on `stream`).
const void* device_input(ExecutionContext& ctx, const char* name, const void* p, size_t bytes,
                         hipStream_t stream);

// Host-readable view of `bytes` at `p`: p itself unless it is device memory,
// else a synchronous copy (on `stream`) into the context's host buffer `name`.
const void* host_input(ExecutionContext& ctx, const char* name, const void* p, size_t bytes,
                       hipStream_t stream);

// Copies `bytes` (at most 64) of device memory to `host` and waits for
// `stream`.  The copy lands in a pinned per-thread slot first: a pageable
// destination costs a staged copy, tens of microseconds for a few bytes.
void read_small(void* host, const void* dev, size_t bytes, hipStream_t stream);
// Words of a device miss counter: the kernels stripe their atomics over 8
// words 16 apart, one per 128-byte line (kMissStripes, kMissStripeWords in
// the kernels); readers add up every word, the others staying 0.
constexpr int kMissCounterWords = 8 * 16;
int64_t read_miss_words(const unsigned long long* counter, hipStream_t stream);

template <typename T>
T read_back(const T* dev, hipStream_t stream) {
  T h;
  read_small(&h, dev, sizeof(T), stream);
  return h;
}

// fp16 <-> fp32 on the host (round to nearest even; NaN stays NaN).
float half_bits_to_float(uint16_t h);
uint16_t float_to_half_bits(float f);

// Device-writable target for `bytes` at `p`; when it differs from p, call
// finish_output afterwards to copy it back.
void* device_output(ExecutionContext& ctx, const char* name, void* p, size_t bytes);
void finish_output(void* user, const void* dev, size_t bytes, hipStream_t stream);

}  // namespace nve_amd

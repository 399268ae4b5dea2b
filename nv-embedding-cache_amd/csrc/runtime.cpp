// runtime.cpp -- see runtime.hpp.
#include "runtime.hpp"

#include "kernels/cache_launch.hpp"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>

namespace nve_amd {

void read_small(void* host, const void* dev, size_t bytes, hipStream_t stream) {
  NVE_CHECK(bytes <= 64, "read_small reads at most 64 bytes");
  // one pinned slot per thread, kept for the thread's life
  thread_local void* slot = nullptr;
  if (slot == nullptr) NVE_HIP(hipHostMalloc(&slot, 64, hipHostMallocDefault));
  NVE_HIP(launch_small_read(slot, dev, (int)bytes, stream));
  NVE_HIP(hipStreamSynchronize(stream));
  std::memcpy(host, slot, bytes);
}

ScopedDevice::ScopedDevice(int device) {
  if (device < 0) return;
  NVE_HIP(hipGetDevice(&prev_));
  if (prev_ != device) {
    NVE_HIP(hipSetDevice(device));
  } else {
    prev_ = -1;
  }
}

ScopedDevice::~ScopedDevice() {
  if (prev_ >= 0) (void)hipSetDevice(prev_);
}

// ---------------------------------------------------------------------------
namespace {
hipEvent_t order_event() {
  thread_local std::map<int, hipEvent_t> events;
  int dev = 0;
  NVE_HIP(hipGetDevice(&dev));
  hipEvent_t& e = events[dev];
  if (!e) NVE_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  return e;
}
}  // namespace

StreamQueue::StreamQueue(hipStream_t caller, hipStream_t run)
    : stream(run ? run : caller), caller_(caller) {
  if (stream != caller_) {
    hipEvent_t e = order_event();
    NVE_HIP(hipEventRecord(e, caller_));
    NVE_HIP(hipStreamWaitEvent(stream, e, 0));
  }
}

// ---------------------------------------------------------------------------
void LookupStreams::add(hipStream_t s) {
  std::lock_guard<std::mutex> lk(mu_);
  ++streams_[s];
}

void LookupStreams::remove(hipStream_t s) {
  std::lock_guard<std::mutex> lk(mu_);
  auto it = streams_.find(s);
  if (it != streams_.end() && --it->second == 0) streams_.erase(it);
}

void LookupStreams::order_before(hipStream_t s) {
  std::lock_guard<std::mutex> lk(mu_);
  hipEvent_t e = order_event();
  for (const auto& kv : streams_) {
    if (kv.first == s) continue;  // in stream order already
    NVE_HIP(hipEventRecord(e, kv.first));
    NVE_HIP(hipStreamWaitEvent(s, e, 0));
  }
}

void LookupStreams::drain() {
  std::lock_guard<std::mutex> lk(mu_);
  hipEvent_t e = order_event();
  for (const auto& kv : streams_) {
    NVE_HIP(hipEventRecord(e, kv.first));
    NVE_HIP(hipEventSynchronize(e));
  }
}

StreamQueue::~StreamQueue() {
  if (stream != caller_) {
    try {
      hipEvent_t e = order_event();  // created by the constructor on this thread and device
      if (hipEventRecord(e, stream) == hipSuccess) (void)hipStreamWaitEvent(caller_, e, 0);
    } catch (...) {
    }
  }
}

// ---------------------------------------------------------------------------
ThreadPool::ThreadPool(int64_t num_workers) {
  if (num_workers <= 0) {
    const int64_t cores = (int64_t)std::thread::hardware_concurrency();
    num_workers = cores - 2 > 1 ? cores - 2 : 1;  // thread_pool.cpp:112-116
  }
  for (int64_t i = 0; i < num_workers; ++i) workers_.emplace_back(&ThreadPool::main_, this);
}

ThreadPool::~ThreadPool() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_ = true;
  }
  cv_.notify_all();
  for (auto& t : workers_) t.join();
}

std::future<void> ThreadPool::submit(std::function<void()> task) {
  std::packaged_task<void()> pt(std::move(task));
  auto f = pt.get_future();
  {
    std::lock_guard<std::mutex> lk(mu_);
    queue_.emplace_back(std::move(pt));
  }
  cv_.notify_one();
  return f;
}

void ThreadPool::main_() {
  for (;;) {
    std::packaged_task<void()> t;
    {
      std::unique_lock<std::mutex> lk(mu_);
      cv_.wait(lk, [&] { return stop_ || !queue_.empty(); });
      if (queue_.empty()) return;
      t = std::move(queue_.front());
      queue_.pop_front();
    }
    t();
  }
}

namespace {
std::mutex g_pool_mu;
std::shared_ptr<ThreadPool> g_pool;
int64_t g_pool_workers = 0;
}  // namespace

std::shared_ptr<ThreadPool> ThreadPool::default_pool() {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  if (!g_pool) g_pool = std::make_shared<ThreadPool>(g_pool_workers);
  return g_pool;
}

void ThreadPool::configure_default(int64_t num_workers) {
  std::lock_guard<std::mutex> lk(g_pool_mu);
  NVE_CHECK(!g_pool, "The default thread pool is already in use");
  g_pool_workers = num_workers;
}

// ---------------------------------------------------------------------------
// JSON of the thread-pool configuration (thread_pool.cpp:57-109 parses it with
// nlohmann::json): the whole text must be one JSON value (RFC 8259), or the
// call fails as a parse error would; fields are read from a top-level object
// only (a field of another kind of value is absent).
// ---------------------------------------------------------------------------
namespace {

struct JsonReader {
  const std::string& s;
  size_t i = 0;

  [[noreturn]] void fail(const char* what) const {
    throw Error(NVE_ERROR_RUNTIME, cat("Malformed JSON: ", what, " at offset ", i));
  }
  void ws() {
    while (i < s.size() && (s[i] == ' ' || s[i] == '\t' || s[i] == '\n' || s[i] == '\r')) ++i;
  }
  bool digit() const { return i < s.size() && s[i] >= '0' && s[i] <= '9'; }
  std::string string() {  // at the opening quote; returns the decoded text (\u kept as is)
    ++i;
    std::string out;
    while (true) {
      if (i >= s.size()) fail("unterminated string");
      const char c = s[i++];
      if (c == '"') return out;
      if ((unsigned char)c < 0x20) fail("control character in a string");
      if (c != '\\') {
        out += c;
        continue;
      }
      if (i >= s.size()) fail("unterminated escape");
      const char e = s[i++];
      switch (e) {
        case '"': case '\\': case '/': out += e; break;
        case 'b': out += '\b'; break;
        case 'f': out += '\f'; break;
        case 'n': out += '\n'; break;
        case 'r': out += '\r'; break;
        case 't': out += '\t'; break;
        case 'u':
          for (int k = 0; k < 4; ++k, ++i)
            if (i >= s.size() || !std::isxdigit((unsigned char)s[i])) fail("bad \\u escape");
          out += "\\u" + s.substr(i - 4, 4);
          break;
        default: fail("bad escape");
      }
    }
  }
  void number() {
    if (s[i] == '-') ++i;
    if (!digit()) fail("bad number");
    if (s[i] == '0') ++i;
    else while (digit()) ++i;
    if (i < s.size() && s[i] == '.') {
      ++i;
      if (!digit()) fail("bad fraction");
      while (digit()) ++i;
    }
    if (i < s.size() && (s[i] == 'e' || s[i] == 'E')) {
      ++i;
      if (i < s.size() && (s[i] == '+' || s[i] == '-')) ++i;
      if (!digit()) fail("bad exponent");
      while (digit()) ++i;
    }
  }
  // one value; with `members`, a top-level object's fields as their raw texts
  void value(std::map<std::string, std::string>* members = nullptr) {
    ws();
    if (i >= s.size()) fail("unexpected end");
    const char c = s[i];
    if (c == '{') {
      ++i;
      ws();
      if (i < s.size() && s[i] == '}') {
        ++i;
        return;
      }
      while (true) {
        ws();
        if (i >= s.size() || s[i] != '"') fail("expected a member name");
        const std::string name = string();
        ws();
        if (i >= s.size() || s[i] != ':') fail("expected ':'");
        ++i;
        ws();
        const size_t at = i;
        value();
        if (members) (*members)[name] = s.substr(at, i - at);
        ws();
        if (i < s.size() && s[i] == ',') {
          ++i;
          continue;
        }
        if (i < s.size() && s[i] == '}') {
          ++i;
          return;
        }
        fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      ++i;
      ws();
      if (i < s.size() && s[i] == ']') {
        ++i;
        return;
      }
      while (true) {
        value();
        ws();
        if (i < s.size() && s[i] == ',') {
          ++i;
          continue;
        }
        if (i < s.size() && s[i] == ']') {
          ++i;
          return;
        }
        fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      string();
      return;
    }
    if (c == '-' || (c >= '0' && c <= '9')) {
      number();
      return;
    }
    for (const char* lit : {"true", "false", "null"}) {
      const size_t n = std::strlen(lit);
      if (s.compare(i, n, lit) == 0) {
        i += n;
        return;
      }
    }
    fail("unexpected character");
  }
};

// The members of the document's top-level object (none when it is another
// kind of value); throws on malformed JSON.
std::map<std::string, std::string> json_members(const char* json) {
  const std::string s(json ? json : "");
  JsonReader r{s};
  std::map<std::string, std::string> members;
  r.ws();
  const bool object = r.i < s.size() && s[r.i] == '{';
  r.value(object ? &members : nullptr);
  r.ws();
  if (r.i != s.size()) r.fail("trailing characters");
  return members;
}

}  // namespace

int64_t json_int_field(const char* json, const char* field, int64_t dflt) {
  const auto m = json_members(json);
  const auto it = m.find(field);
  if (it == m.end()) return dflt;
  const std::string& v = it->second;
  char* end = nullptr;
  const long long x = std::strtoll(v.c_str(), &end, 10);
  NVE_CHECK_ARG(!v.empty() && end == v.c_str() + v.size(), "JSON field '", field, "' must be an integer");
  return (int64_t)x;
}

std::string json_string_field(const char* json, const char* field, const std::string& dflt) {
  const auto m = json_members(json);
  const auto it = m.find(field);
  if (it == m.end()) return dflt;
  const std::string& v = it->second;
  NVE_CHECK_ARG(v.size() >= 2 && v.front() == '"', "JSON field '", field, "' must be a string");
  JsonReader r{v};
  return r.string();
}

// ---------------------------------------------------------------------------
ExecutionContext::ExecutionContext(int device, hipStream_t lookup, hipStream_t modify,
                                   std::shared_ptr<ThreadPool> pool)
    : device_(device), lookup_(lookup), modify_(modify), pool_(std::move(pool)) {
  if (!pool_) pool_ = ThreadPool::default_pool();
}

void ExecutionContext::watch(const std::shared_ptr<LookupStreams>& streams) {
  streams->add(lookup_);
  watched_.push_back(streams);
}

ExecutionContext::~ExecutionContext() {
  try {
    wait();
  } catch (...) {
  }
  for (auto& w : watched_) w->remove(lookup_);
  for (auto& kv : bufs_)
    if (kv.second.plain) std::free(kv.second.ptr);
  if (device_ < 0 && misses_ == nullptr) return;  // a host context holds no HIP memory
  ScopedDevice sd(device_);
  for (auto& kv : bufs_) {
    if (kv.second.plain) continue;
    if (kv.second.host)
      (void)hipHostFree(kv.second.ptr);
    else
      (void)hipFree(kv.second.ptr);
  }
  if (misses_) (void)hipFree(misses_);
  if (miss_total_) (void)hipHostFree(miss_total_);
}

void* ExecutionContext::host_buffer(const std::string& name, size_t bytes) {
  std::lock_guard<std::mutex> lk(bufs_mu_);
  Buf& b = bufs_[name];
  NVE_CHECK(b.ptr == nullptr || b.plain, "Context buffer '", name, "' is not a host buffer");
  if (b.ptr && b.bytes < bytes) {
    std::free(b.ptr);
    b.ptr = nullptr;
  }
  if (!b.ptr) {
    const size_t sz = (std::max<size_t>(bytes, 256) + 63) / 64 * 64;
    b.ptr = std::aligned_alloc(64, sz);
    if (!b.ptr) throw Error(NVE_ERROR_OUT_OF_MEMORY, cat("Out of host memory for ", sz, " bytes"));
    b.bytes = sz;
    b.host = true;
    b.plain = true;
  }
  return b.ptr;
}

void* ExecutionContext::buffer(const std::string& name, size_t bytes, bool host) {
  std::lock_guard<std::mutex> lk(bufs_mu_);
  Buf& b = bufs_[name];
  NVE_CHECK(!b.plain, "Context buffer '", name, "' is a plain host buffer");
  if (b.ptr && (b.bytes < bytes || b.host != host)) {
    // the stream may still use the old buffer
    NVE_HIP(hipStreamSynchronize(lookup_));
    NVE_HIP(hipStreamSynchronize(modify_));
    if (b.host)
      NVE_HIP(hipHostFree(b.ptr));
    else
      NVE_HIP(hipFree(b.ptr));
    b.ptr = nullptr;
  }
  if (!b.ptr) {
    const size_t sz = bytes > 256 ? bytes : 256;
    if (host)
      NVE_HIP(hipHostMalloc(&b.ptr, sz, hipHostMallocDefault));
    else
      NVE_HIP(hipMalloc(&b.ptr, sz));
    b.bytes = sz;
    b.host = host;
  }
  return b.ptr;
}

unsigned long long* ExecutionContext::miss_counter() {
  if (!misses_) {
    NVE_HIP(hipMalloc(&misses_, kMissCounterWords * sizeof(unsigned long long)));
    NVE_HIP(launch_fill_u64(reinterpret_cast<uint64_t*>(misses_), kMissCounterWords, 0, lookup_));
  }
  misses_clean_ = false;  // the caller may hand it to a counting kernel
  return misses_;
}

void ExecutionContext::reset_misses() {
  // a fill kernel rather than a memset node, so the lookup stays capturable
  NVE_HIP(launch_fill_u64(reinterpret_cast<uint64_t*>(miss_counter()), kMissCounterWords, 0, lookup_));
  misses_clean_ = true;
}

void ExecutionContext::prepare_misses() {
  if (!misses_clean_) reset_misses();
}

int64_t ExecutionContext::misses_total(int reset) {
  if (!misses_) miss_counter();
  if (!miss_total_) NVE_HIP(hipHostMalloc((void**)&miss_total_, 64, hipHostMallocDefault));
  NVE_HIP(launch_counter_total(misses_, kMissCounterWords, miss_total_, reset, lookup_));
  NVE_HIP(hipStreamSynchronize(lookup_));
  return (int64_t)*static_cast<volatile unsigned long long*>(miss_total_);
}

int64_t ExecutionContext::read_misses() { return misses_total(0); }

int64_t ExecutionContext::take_misses() {
  const int64_t t = misses_total(1);
  misses_clean_ = true;
  return t;
}

int64_t read_miss_words(const unsigned long long* counter, hipStream_t stream) {
  // the sum is written by a kernel into a pinned per-thread word
  thread_local unsigned long long* slot = nullptr;
  if (slot == nullptr) NVE_HIP(hipHostMalloc((void**)&slot, 64, hipHostMallocDefault));
  NVE_HIP(launch_counter_total(const_cast<unsigned long long*>(counter), kMissCounterWords, slot, 0, stream));
  NVE_HIP(hipStreamSynchronize(stream));
  return (int64_t)*static_cast<volatile unsigned long long*>(slot);
}

void ExecutionContext::add_pending(std::future<void> f) {
  std::lock_guard<std::mutex> lk(pending_mu_);
  pending_.push_back(std::move(f));
}

void ExecutionContext::wait() {
  std::vector<std::future<void>> fs;
  {
    std::lock_guard<std::mutex> lk(pending_mu_);
    fs.swap(pending_);
  }
  std::exception_ptr first;
  for (auto& f : fs) {
    try {
      f.get();
    } catch (...) {
      if (!first) first = std::current_exception();
    }
  }
  if (device_ >= 0) {  // a host context runs everything on the calling threads
    ScopedDevice sd(device_);
    NVE_HIP(hipStreamSynchronize(lookup_));
    NVE_HIP(hipStreamSynchronize(modify_));
  }
  if (first) std::rethrow_exception(first);
}

// ---------------------------------------------------------------------------
MemKind mem_kind(const void* p) {
  hipPointerAttribute_t attr;
  std::memset(&attr, 0, sizeof(attr));
  const hipError_t e = hipPointerGetAttributes(&attr, p);
  if (e != hipSuccess) {
    (void)hipGetLastError();  // clear: an unknown pointer is plain host memory
    return MemKind::PageableHost;
  }
  switch (attr.type) {
    case hipMemoryTypeDevice:
    case hipMemoryTypeManaged:
    case hipMemoryTypeUnified: return MemKind::Device;
    case hipMemoryTypeHost: return MemKind::PinnedHost;
    default: return MemKind::PageableHost;
  }
}

const void* device_input(ExecutionContext& ctx, const char* name, const void* p, size_t bytes,
                         hipStream_t stream) {
  if (p == nullptr || bytes == 0) return p;
  if (mem_kind(p) == MemKind::Device) return p;
  void* d = ctx.buffer(name, bytes, false);
  NVE_HIP(hipMemcpyAsync(d, p, bytes, hipMemcpyHostToDevice, stream));
  return d;
}

const void* host_input(ExecutionContext& ctx, const char* name, const void* p, size_t bytes,
                       hipStream_t stream) {
  if (p == nullptr || bytes == 0) return p;
  if (mem_kind(p) != MemKind::Device) return p;
  void* h = ctx.buffer(name, bytes, true);
  NVE_HIP(hipMemcpyAsync(h, p, bytes, hipMemcpyDeviceToHost, stream));
  NVE_HIP(hipStreamSynchronize(stream));
  return h;
}

float half_bits_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  if (e == 0) {
    const float f = std::ldexp((float)m, -24);  // zero or subnormal: m * 2^-24, exact
    return sign ? -f : f;
  }
  const uint32_t bits = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

uint16_t float_to_half_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);  // >= 65520 rounds to infinity
  if (ax < 0x38800000u) {
    // below 2^-14: a multiple of 2^-24 after rounding; scaling by 2^24 is exact
    float v;
    std::memcpy(&v, &ax, 4);
    return (uint16_t)(sign | (uint16_t)std::nearbyint(v * 16777216.0f));
  }
  uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // a carry bumps the exponent correctly
  return (uint16_t)(sign | h);
}

void* device_output(ExecutionContext& ctx, const char* name, void* p, size_t bytes) {
  if (p == nullptr || bytes == 0) return p;
  if (mem_kind(p) == MemKind::Device) return p;
  return ctx.buffer(name, bytes, false);
}

void finish_output(void* user, const void* dev, size_t bytes, hipStream_t stream) {
  if (user == dev || bytes == 0) return;
  NVE_HIP(hipMemcpyAsync(user, dev, bytes, hipMemcpyDeviceToHost, stream));
}

}  // namespace nve_amd

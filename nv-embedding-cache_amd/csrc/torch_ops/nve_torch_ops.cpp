// nve_torch_ops.cpp -- the nve_ops torch library, native: the two ops of the
// reference's torch binding (python/pynve/torch_bindings/torch_binding.cpp:85-92,
// implementations nve_torch_ops.cu:67-146 and nve_torch_ops_cpu.cpp:59-133)
// for HIP tensors (torch's CUDA dispatch key on ROCm) and host tensors (CPU key,
// host layers), calling libnve_amd.so's C ABI directly.
//
//   nve_ops::embedding_lookup(Tensor marker, Tensor keys, int embedding_size,
//                             int dtype) -> Tensor
//   nve_ops::embedding_lookup_with_pooling(Tensor marker, Tensor keys,
//       Tensor offsets, Tensor? weights, int pooling_type, int embedding_size,
//       int dtype) -> Tensor
//
// A layer is found through its marker tensor's data pointer in a registry that
// the Python layer fills when it builds the layer (the reference keeps the
// same map in nve_registry.cu:25-50).  Each registry entry owns one execution
// context per lookup stream, made on first use and destroyed when the entry is
// dropped or its layer's contexts are released.  Shape inference (the fake
// kernels) stays in Python, as in the reference.
#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <cstdint>
#include <cstdio>
#include <memory>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "nve_amd_ext.h"
#include "nve_c_api.h"

#define NVE_TORCH_API extern "C" __attribute__((visibility("default")))

namespace {

struct Entry {
  nve_layer_t layer = nullptr;
  int64_t row_bytes = 0;
  int32_t dtype = NVE_DTYPE_UNKNOWN;
  void* modify_stream = nullptr;
  int64_t logging_interval = -1;

  std::mutex mu;                                  // guards the two fields below
  std::unordered_map<void*, nve_context_t> ctxs;  // lookup stream (or thread) -> context
  int64_t lookups = 0;                            // hit-rate logging counter

  // A context is not thread-safe.  Lookups on a GPU stream share that stream's
  // context; lookups of CPU keys have no stream, so each calling thread gets a
  // context of its own, keyed by the address of a thread_local (the reference's
  // get_cpu_stream, nve_torch_ops_cpu.cpp:22,54), and made with no stream.
  nve_context_t context(void* stream) {
    static thread_local char thread_key;
    void* key = stream ? stream : static_cast<void*>(&thread_key);
    std::lock_guard<std::mutex> lk(mu);
    auto it = ctxs.find(key);
    if (it != ctxs.end()) return it->second;
    nve_context_t c = nullptr;
    check(nve_layer_create_execution_context(layer, &c, stream, modify_stream, nullptr, nullptr));
    ctxs.emplace(key, c);
    return c;
  }

  // Waits for and destroys every context (the binding's release step).
  void release() {
    std::lock_guard<std::mutex> lk(mu);
    for (auto& kv : ctxs) {
      nve_context_wait(kv.second);
      nve_context_destroy(kv.second);
    }
    ctxs.clear();
  }

  // Every logging_interval-th lookup writes its hit rates at the perf level
  // (binding_layers.hpp:370-387).
  void log_hit_rates(const float* hr) {
    if (logging_interval <= 0) return;
    int64_t n;
    {
      std::lock_guard<std::mutex> lk(mu);
      n = lookups++;
    }
    if (n % logging_interval != 0) return;
    char msg[96];
    std::snprintf(msg, sizeof msg, "Hit rates: %g, %g, %g", hr[0], hr[1], hr[2]);
    nve_amd_log_message(30, msg);
  }

  static void check(nve_status_t st) {
    if (st == NVE_SUCCESS) return;
    const char* m = nullptr;
    nve_get_last_error(&m);
    const std::string what = m ? m : "no message";
    TORCH_CHECK_VALUE(st != NVE_ERROR_INVALID_ARGUMENT, "nve_ops: invalid argument: ", what);
    TORCH_CHECK_NOT_IMPLEMENTED(st != NVE_ERROR_NOT_IMPLEMENTED, "nve_ops: ", what);
    TORCH_CHECK(false, "nve_ops: status ", (int)st, ": ", what);
  }
};

std::mutex g_mu;
std::unordered_map<const void*, std::shared_ptr<Entry>> g_entries;

std::shared_ptr<Entry> entry_of(const at::Tensor& marker) {
  const void* key = marker.data_ptr();
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_entries.find(key);
  TORCH_CHECK(it != g_entries.end(), "nve_ops: no binding registered for marker_ptr=", key,
              " (build the layer through pynve.torch before calling its ops)");
  return it->second;
}

void check_keys(const at::Tensor& t, const char* what) {
  TORCH_CHECK(t.scalar_type() == at::kLong, "nve_ops: ", what, " must hold int64 values, got ",
              t.scalar_type());
  TORCH_CHECK(t.is_contiguous(), "nve_ops: ", what, " must be a contiguous tensor");
}

at::ScalarType row_type(const Entry& e) {
  if (e.dtype == NVE_DTYPE_FLOAT32) return at::kFloat;
  if (e.dtype == NVE_DTYPE_FLOAT16) return at::kHalf;
  TORCH_CHECK(false, "nve_ops: the layer's rows are neither float32 nor float16 (type ", e.dtype, ")");
}

int64_t row_width(const Entry& e) { return e.row_bytes / (e.dtype == NVE_DTYPE_FLOAT32 ? 4 : 2); }

// The lookup stream: the current HIP stream of the keys' GPU; host layers run
// on the calling thread (no stream).
void* stream_of(const at::Tensor& keys) {
  if (!keys.is_cuda()) return nullptr;
  return c10::hip::getCurrentHIPStream(keys.get_device()).stream();
}

at::Tensor embedding_lookup(const at::Tensor& marker, const at::Tensor& keys, int64_t /*embedding_size*/,
                            int64_t /*dtype*/) {
  check_keys(keys, "keys");
  auto e = entry_of(marker);
  const int64_t n = keys.numel();
  at::Tensor out = at::empty({n, row_width(*e)}, keys.options().dtype(row_type(*e)));
  void* s = stream_of(keys);
  float hr[3] = {0.f, 0.f, 0.f};
  Entry::check(nve_layer_lookup(e->layer, e->context(s), n, keys.data_ptr(), out.data_ptr(), e->row_bytes,
                                nullptr, hr));
  e->log_hit_rates(hr);
  return out;
}

at::Tensor embedding_lookup_with_pooling(const at::Tensor& marker, const at::Tensor& keys,
                                         const at::Tensor& offsets, const std::optional<at::Tensor>& weights,
                                         int64_t pooling_type, int64_t /*embedding_size*/,
                                         int64_t /*dtype*/) {
  check_keys(keys, "keys");
  check_keys(offsets, "offsets");
  TORCH_CHECK(offsets.numel() >= 2, "nve_ops: offsets need num_bags + 1 >= 2 entries (the last one is ",
              "len(keys)), got ", offsets.numel());
  auto e = entry_of(marker);
  nve_data_type_t wt = NVE_DTYPE_UNKNOWN;
  const void* wp = nullptr;
  if (weights.has_value() && weights->defined()) {
    const at::Tensor& w = *weights;
    TORCH_CHECK(w.is_contiguous(), "nve_ops: weights must be a contiguous tensor");
    TORCH_CHECK(w.numel() == keys.numel(), "nve_ops: ", w.numel(), " weights for ", keys.numel(),
                " keys (one per key is required)");
    if (w.scalar_type() == at::kFloat)
      wt = NVE_DTYPE_FLOAT32;
    else if (w.scalar_type() == at::kHalf)
      wt = NVE_DTYPE_FLOAT16;
    else
      TORCH_CHECK(false, "nve_ops: weights must be float32 or float16, got ", w.scalar_type());
    wp = w.data_ptr();
  }
  const int64_t bags = offsets.numel() - 1;
  at::Tensor out = at::empty({bags, row_width(*e)}, keys.options().dtype(row_type(*e)));
  void* s = stream_of(keys);
  float hr[3] = {0.f, 0.f, 0.f};
  Entry::check(nve_layer_lookup_pooled(e->layer, e->context(s), keys.numel(), keys.data_ptr(), out.data_ptr(),
                                       e->row_bytes, nullptr, (nve_pooling_type_t)pooling_type,
                                       NVE_SPARSE_CSR, offsets.data_ptr(), offsets.numel(), 0, wp, wt,
                                       (nve_data_type_t)e->dtype, hr));
  e->log_hit_rates(hr);
  return out;
}

}  // namespace

TORCH_LIBRARY(nve_ops, m) {
  m.def("embedding_lookup(Tensor marker, Tensor keys, int embedding_size, int dtype) -> Tensor");
  m.def(
      "embedding_lookup_with_pooling(Tensor marker, Tensor keys, Tensor offsets, Tensor? weights, "
      "int pooling_type, int embedding_size, int dtype) -> Tensor");
}

// One implementation for both keys: the registered layer decides where the
// lookup runs (HIP kernels, or CPU threads for a host layer).
TORCH_LIBRARY_IMPL(nve_ops, CUDA, m) {
  m.impl("embedding_lookup", &embedding_lookup);
  m.impl("embedding_lookup_with_pooling", &embedding_lookup_with_pooling);
}

TORCH_LIBRARY_IMPL(nve_ops, CPU, m) {
  m.impl("embedding_lookup", &embedding_lookup);
  m.impl("embedding_lookup_with_pooling", &embedding_lookup_with_pooling);
}

// ---------------------------------------------------------------------------
// Registry, called by the Python layers (ctypes).  Return 0 on success.
// ---------------------------------------------------------------------------

// Maps marker -> layer.  row_bytes and dtype are the layer's row size and row
// type (float32 or float16), modify_stream the stream its contexts modify on
// (may be NULL), logging_interval the hit-rate logging period (<= 0: none).
// Registering a marker again replaces its entry.
NVE_TORCH_API int32_t nve_torch_ops_register(const void* marker, void* layer, int64_t row_bytes, int32_t dtype,
                                             void* modify_stream, int64_t logging_interval) {
  if (marker == nullptr || layer == nullptr || row_bytes <= 0) return 1;
  if (dtype != NVE_DTYPE_FLOAT32 && dtype != NVE_DTYPE_FLOAT16) return 1;
  auto e = std::make_shared<Entry>();
  e->layer = static_cast<nve_layer_t>(layer);
  e->row_bytes = row_bytes;
  e->dtype = dtype;
  e->modify_stream = modify_stream;
  e->logging_interval = logging_interval;
  std::shared_ptr<Entry> old;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto& slot = g_entries[marker];
    old = std::move(slot);
    slot = std::move(e);
  }
  if (old) old->release();
  return 0;
}

// Drops a marker's entry, waiting for and destroying its contexts.
NVE_TORCH_API int32_t nve_torch_ops_unregister(const void* marker) {
  std::shared_ptr<Entry> old;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_entries.find(marker);
    if (it == g_entries.end()) return 0;
    old = std::move(it->second);
    g_entries.erase(it);
  }
  old->release();
  return 0;
}

// Number of execution contexts (one per lookup stream used so far) of a
// marker's entry, in *out; returns 1 if the marker is not registered.
NVE_TORCH_API int32_t nve_torch_ops_num_contexts(const void* marker, int64_t* out) {
  std::shared_ptr<Entry> e;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_entries.find(marker);
    if (it == g_entries.end() || out == nullptr) return 1;
    e = it->second;
  }
  std::lock_guard<std::mutex> lk(e->mu);
  *out = (int64_t)e->ctxs.size();
  return 0;
}

// Waits for and destroys the contexts of every entry over `layer` (called
// before the layer is destroyed); the entries stay and make new contexts on
// their next lookup.
NVE_TORCH_API int32_t nve_torch_ops_release_layer(void* layer) {
  std::vector<std::shared_ptr<Entry>> hit;
  {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto& kv : g_entries)
      if (kv.second->layer == layer) hit.push_back(kv.second);
  }
  for (auto& e : hit) e->release();
  return 0;
}

/* nve_loader.hpp -- C++ loader of exported NVE models (AOTInductor packages).
 *
 * The C++ counterpart of the reference's python/pynve/torch_bindings/
 * nve_loader.hpp:130-253 (ResourceDirectory, LayerDirectory): a C++ inference
 * host that runs a model.pt2 package built by pynve.torch.nve_export.export_aot
 * recreates the package's embedding layers from the save directory
 * (metadata.json, weights/<key>.nve), gives each layer a marker tensor, points
 * the package's marker constant at it and registers the marker with the
 * nve_ops torch library, so the package's nve_ops calls reach the layer:
 *
 *     torch::inductor::AOTIModelPackageLoader loader(dir + "/model.pt2", "model", false, 1, dev);
 *     nve::LayerDirectory layers(dir, loader, dev);
 *     auto outputs = loader.run({keys});
 *
 * The layers are made through the C ABI (nve_c_api.h, libnve_amd.so) and
 * registered through libnve_torch_ops.so (which also registers the ops with
 * torch when it is loaded: link it, or dlopen it, before running the package).
 * Supported: GPULayer, LinearUVM and HostLayer entries of schema-1 and
 * schema-2 metadata, memory blocks of type Linear, Managed, Host and User
 * (shared by key, optionally across directories through a ResourceDirectory).
 * Hierarchical layers and NVL memory blocks are not part of this build.
 *
 * Header-only; needs torch's C++ headers and libraries, HIP and the two NVE
 * libraries.  Errors throw std::runtime_error.
 */
#pragma once

#include <hip/hip_runtime.h>
#include <torch/csrc/inductor/aoti_package/model_package_loader.h>
#include <ATen/ATen.h>

#include <cctype>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <memory>
#include <set>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "nve_amd_ext.h"
#include "nve_c_api.h"

/* The marker registry of libnve_torch_ops.so (marker data pointer -> layer). */
extern "C" int32_t nve_torch_ops_register(const void* marker, void* layer, int64_t row_bytes, int32_t dtype,
                                          void* modify_stream, int64_t logging_interval);
extern "C" int32_t nve_torch_ops_unregister(const void* marker);

namespace nve {

namespace loader_detail {

[[noreturn]] inline void fail(const std::string& what) { throw std::runtime_error("nve_loader: " + what); }

inline void check_status(nve_status_t st, const char* call) {
  if (st == NVE_SUCCESS) return;
  const char* m = nullptr;
  nve_get_last_error(&m);
  fail(std::string(call) + " failed: " + (m ? m : "no message"));
}

inline void check_hip(hipError_t e, const char* call) {
  if (e != hipSuccess) fail(std::string(call) + ": " + hipGetErrorString(e));
}

// ---------------------------------------------------------------------------
// A JSON value and a reader for the metadata file (objects, arrays, strings,
// numbers, true / false / null).  Integers keep all 64 bits (layer ids).
// ---------------------------------------------------------------------------
struct Json {
  enum Kind { Null, Bool, Int, Real, Str, Arr, Obj } kind = Null;
  bool b = false;
  int64_t i = 0;
  double d = 0.0;
  std::string s;
  std::vector<Json> a;
  std::vector<std::pair<std::string, Json>> o;

  const Json* find(const std::string& key) const {
    if (kind != Obj) return nullptr;
    for (const auto& kv : o)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
  const Json& at(const std::string& key) const {
    const Json* v = find(key);
    if (!v) fail("metadata entry has no '" + key + "'");
    return *v;
  }
  int64_t as_int() const {
    if (kind == Int) return i;
    if (kind == Real) return (int64_t)d;
    if (kind == Bool) return b ? 1 : 0;
    fail("expected a number in metadata");
  }
  const std::string& as_str() const {
    if (kind != Str) fail("expected a string in metadata");
    return s;
  }
  bool as_bool() const {
    if (kind == Bool) return b;
    if (kind == Int) return i != 0;
    fail("expected a boolean in metadata");
  }
  int64_t int_or(const std::string& key, int64_t dflt) const {
    const Json* v = find(key);
    return v && v->kind != Null ? v->as_int() : dflt;
  }
  std::string str_or(const std::string& key, const std::string& dflt) const {
    const Json* v = find(key);
    return v && v->kind == Str ? v->s : dflt;
  }
};

class JsonReader {
 public:
  explicit JsonReader(const std::string& text) : p_(text.data()), e_(text.data() + text.size()) {}

  Json document() {
    Json v = value();
    space();
    if (p_ != e_) fail("trailing characters after the metadata document");
    return v;
  }

 private:
  const char* p_;
  const char* e_;

  void space() {
    while (p_ < e_ && std::isspace((unsigned char)*p_)) ++p_;
  }
  char peek() {
    space();
    if (p_ >= e_) fail("metadata ends early");
    return *p_;
  }
  void expect(char c) {
    if (peek() != c) fail(std::string("metadata: expected '") + c + "'");
    ++p_;
  }
  bool word(const char* w) {
    const size_t n = std::strlen(w);
    if ((size_t)(e_ - p_) >= n && std::strncmp(p_, w, n) == 0) {
      p_ += n;
      return true;
    }
    return false;
  }

  Json value() {
    const char c = peek();
    Json v;
    if (c == '{') {
      ++p_;
      v.kind = Json::Obj;
      if (peek() == '}') {
        ++p_;
        return v;
      }
      for (;;) {
        std::string key = string();
        expect(':');
        v.o.emplace_back(std::move(key), value());
        if (peek() == ',') {
          ++p_;
          continue;
        }
        expect('}');
        return v;
      }
    }
    if (c == '[') {
      ++p_;
      v.kind = Json::Arr;
      if (peek() == ']') {
        ++p_;
        return v;
      }
      for (;;) {
        v.a.push_back(value());
        if (peek() == ',') {
          ++p_;
          continue;
        }
        expect(']');
        return v;
      }
    }
    if (c == '"') {
      v.kind = Json::Str;
      v.s = string();
      return v;
    }
    if (word("true")) {
      v.kind = Json::Bool;
      v.b = true;
      return v;
    }
    if (word("false")) {
      v.kind = Json::Bool;
      return v;
    }
    if (word("null")) return v;
    return number();
  }

  std::string string() {
    expect('"');
    std::string out;
    while (p_ < e_ && *p_ != '"') {
      char c = *p_++;
      if (c != '\\') {
        out.push_back(c);
        continue;
      }
      if (p_ >= e_) break;
      c = *p_++;
      switch (c) {
        case 'n': out.push_back('\n'); break;
        case 't': out.push_back('\t'); break;
        case 'r': out.push_back('\r'); break;
        case 'b': out.push_back('\b'); break;
        case 'f': out.push_back('\f'); break;
        case 'u': {
          if (e_ - p_ < 4) fail("metadata: short \\u escape");
          const unsigned cp = (unsigned)std::strtoul(std::string(p_, 4).c_str(), nullptr, 16);
          p_ += 4;
          if (cp < 0x80) {
            out.push_back((char)cp);
          } else if (cp < 0x800) {
            out.push_back((char)(0xC0 | (cp >> 6)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
          } else {
            out.push_back((char)(0xE0 | (cp >> 12)));
            out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
            out.push_back((char)(0x80 | (cp & 0x3F)));
          }
          break;
        }
        default: out.push_back(c);  // \" \\ \/
      }
    }
    if (p_ >= e_) fail("metadata: unterminated string");
    ++p_;
    return out;
  }

  Json number() {
    const char* b = p_;
    bool real = false;
    if (p_ < e_ && (*p_ == '-' || *p_ == '+')) ++p_;
    while (p_ < e_ && (std::isdigit((unsigned char)*p_) || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                       *p_ == '-' || *p_ == '+')) {
      if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') real = true;
      ++p_;
    }
    if (p_ == b) fail("metadata: unexpected character");
    const std::string t(b, p_);
    Json v;
    if (real) {
      v.kind = Json::Real;
      v.d = std::strtod(t.c_str(), nullptr);
    } else {
      v.kind = Json::Int;
      v.i = std::strtoll(t.c_str(), nullptr, 10);
    }
    return v;
  }
};

inline Json read_json_file(const std::string& path) {
  std::ifstream f(path, std::ios::binary);
  if (!f) fail("cannot open " + path);
  std::string text((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  return JsonReader(text).document();
}

// ---------------------------------------------------------------------------
// The .nve table file (the reference's serialization.hpp:110-140 format): a
// 12-byte header {u32 0x4E564500, u32 0, u32 2}, then entries of a 32-byte
// record {u64 key1, u64 name, u64 offset of the next record, u64 length}
// followed by `length` data bytes.  Little-endian.
// ---------------------------------------------------------------------------
struct NveEntry {
  bool found = false;
  uint64_t data_offset = 0;
};

inline NveEntry find_nve_entry(std::ifstream& f, uint64_t name, uint64_t bytes, const std::string& path) {
  uint32_t head[3] = {0, 0, 0};
  f.seekg(0);
  f.read(reinterpret_cast<char*>(head), sizeof head);
  if (f.gcount() != (std::streamsize)sizeof head || head[0] != 0x4E564500u || head[1] != 0 || head[2] != 2)
    fail(path + ": Incorrect file version");
  NveEntry e;
  uint64_t rec[4];
  for (;;) {
    f.read(reinterpret_cast<char*>(rec), sizeof rec);
    const std::streamsize got = f.gcount();
    if (got == 0) return e;  // the file ends: no entry of that name
    if (got != (std::streamsize)sizeof rec) fail(path + ": Problem reading table entry");
    if (rec[1] == name) {
      if (rec[3] != bytes) fail(path + ": Incorrect tensor size");
      e.found = true;
      e.data_offset = (uint64_t)f.tellg();
      return e;
    }
    f.clear();
    f.seekg((std::streamoff)rec[2]);
  }
}

}  // namespace loader_detail

// Rows of one embedding table: device memory (hipMalloc on `device`) or pinned
// host memory (hipHostMalloc), freed with the last layer that uses it.
struct TableStorage {
  void* ptr = nullptr;
  size_t bytes = 0;
  int device = -1;  // >= 0: device memory of that GPU
  TableStorage(size_t nbytes, int dev) : bytes(nbytes), device(dev) {
    const size_t sz = nbytes ? nbytes : 1;
    if (dev >= 0) {
      loader_detail::check_hip(hipSetDevice(dev), "hipSetDevice");
      loader_detail::check_hip(hipMalloc(&ptr, sz), "hipMalloc");
    } else {
      loader_detail::check_hip(hipHostMalloc(&ptr, sz, hipHostMallocDefault), "hipHostMalloc");
    }
  }
  ~TableStorage() {
    if (!ptr) return;
    if (device >= 0)
      (void)hipFree(ptr);
    else
      (void)hipHostFree(ptr);
  }
  TableStorage(const TableStorage&) = delete;
  TableStorage& operator=(const TableStorage&) = delete;
};

// Storage already built, by resource key, shared by the LayerDirectory objects
// given the same ResourceDirectory (exports of one model family that share
// tables); remap renames a key of a file to a key of the directory first.
// Not thread-safe.
class ResourceDirectory {
 public:
  std::shared_ptr<TableStorage> find(const std::string& key) const {
    auto it = storage_.find(remap(key));
    return it == storage_.end() ? nullptr : it->second;
  }
  void insert(const std::string& key, std::shared_ptr<TableStorage> s) { storage_[remap(key)] = std::move(s); }
  void add_remap(const std::string& from, const std::string& to) { remap_[from] = to; }
  std::string remap(const std::string& key) const {
    auto it = remap_.find(key);
    return it == remap_.end() ? key : it->second;
  }

 private:
  std::unordered_map<std::string, std::shared_ptr<TableStorage>> storage_;
  std::unordered_map<std::string, std::string> remap_;
};

// Name of a layer's marker constant in the exported graph.
inline std::string marker_fqn(const std::string& module_path) {
  return module_path.empty() ? std::string("marker_tensor") : module_path + ".marker_tensor";
}

struct LoadedLayer {
  int64_t layer_id = 0;
  std::string module_path;
  std::string layer_type;  // "GPULayer", "LinearUVM" or "HostLayer"
  nve_layer_t layer = nullptr;
  nve_table_t table = nullptr;          // the layer's GPU table or host table
  hipStream_t private_stream = nullptr;  // LinearUVM layers built for training
  std::shared_ptr<TableStorage> storage;
  int64_t row_bytes = 0;
  int32_t dtype = NVE_DTYPE_UNKNOWN;
  at::Tensor marker;  // owned here; the package holds a non-owning handle
};

// Builds and owns the layers of one save directory for one loaded package.
// Must outlive every run of the package; the destructor unregisters the
// markers and destroys the layers.
class LayerDirectory {
 public:
  LayerDirectory(const std::string& save_dir, torch::inductor::AOTIModelPackageLoader& loader, int device_index,
                 std::shared_ptr<ResourceDirectory> resources = nullptr, size_t gpu_cache_size_override = 0)
      : save_dir_(save_dir), device_(device_index),
        resources_(resources ? std::move(resources) : std::make_shared<ResourceDirectory>()) {
    using loader_detail::fail;
    const loader_detail::Json doc = loader_detail::read_json_file(save_dir + "/metadata.json");
    const auto fqns = loader.get_constant_fqns();
    const std::set<std::string> constants(fqns.begin(), fqns.end());
    const loader_detail::Json* entries = &doc;
    const loader_detail::Json* memblocks = nullptr;
    bool v2 = false;
    if (doc.kind == loader_detail::Json::Obj) {
      const int64_t version = doc.int_or("version", 1);
      if (version > 2)
        fail("metadata.json has schema version " + std::to_string(version) + "; this loader reads up to 2");
      v2 = true;
      entries = &doc.at("layers");
      if (const auto* res = doc.find("resources")) memblocks = res->find("memblocks");
    }
    if (entries->kind != loader_detail::Json::Arr) fail("metadata.json holds no layer list");
    try {
      std::set<std::string> weights_done;
      for (const auto& entry : entries->a) add_layer(entry, v2, memblocks, gpu_cache_size_override, constants,
                                                     weights_done, loader);
    } catch (...) {
      teardown();
      throw;
    }
  }

  ~LayerDirectory() { teardown(); }

  LayerDirectory(const LayerDirectory&) = delete;
  LayerDirectory& operator=(const LayerDirectory&) = delete;

  // Points every marker constant of the package at its layer's marker again
  // (after a constant-buffer swap replaced the package's handles with copies).
  void rebind_markers(torch::inductor::AOTIModelPackageLoader& loader) {
    for (auto& l : layers_) write_marker(loader, marker_fqn(l.module_path), l.marker);
  }

  size_t size() const { return layers_.size(); }
  const std::vector<LoadedLayer>& layers() const { return layers_; }
  const LoadedLayer& get_layer(int64_t layer_id) const {
    for (const auto& l : layers_)
      if (l.layer_id == layer_id) return l;
    loader_detail::fail("no layer with id " + std::to_string(layer_id));
  }

 private:
  std::string save_dir_;
  int device_;
  std::shared_ptr<ResourceDirectory> resources_;
  std::vector<LoadedLayer> layers_;

  static void write_marker(torch::inductor::AOTIModelPackageLoader& loader, const std::string& fqn,
                           const at::Tensor& marker) {
    // both constant buffers, as a non-owning (user-managed) handle: the package
    // then hands the op this very tensor, whose data pointer is registered
    std::unordered_map<std::string, at::Tensor> m{{fqn, marker}};
    loader.load_constants(m, /*use_inactive=*/false, /*check_full_update=*/false, /*user_managed=*/true);
    loader.load_constants(m, /*use_inactive=*/true, /*check_full_update=*/false, /*user_managed=*/true);
  }

  void teardown() {
    for (auto it = layers_.rbegin(); it != layers_.rend(); ++it) {
      if (it->marker.defined()) nve_torch_ops_unregister(it->marker.data_ptr());
      if (it->layer) nve_layer_destroy(it->layer);
      if (it->table) nve_table_destroy(it->table);
      if (it->private_stream) (void)hipStreamDestroy(it->private_stream);
    }
    layers_.clear();
  }

  std::shared_ptr<TableStorage> storage_for(const std::string& key, const loader_detail::Json* memblocks,
                                            const std::string& layer_type, int64_t rows, int64_t width,
                                            int64_t bytes, bool* fresh) {
    using loader_detail::fail;
    std::string mb_type = layer_type == "HostLayer" ? "Host" : "Managed";
    if (!key.empty()) {
      if (auto s = resources_->find(key)) {
        *fresh = false;
        return s;
      }
      const std::string eff = resources_->remap(key);
      const loader_detail::Json* d = memblocks ? memblocks->find(eff) : nullptr;
      if (!d) fail("storage_ref '" + eff + "' not found in resources.memblocks");
      if (d->at("row_elements").as_int() != width)
        fail("resource '" + eff + "' row_elements " + std::to_string(d->at("row_elements").as_int()) +
             " != layer embedding_size " + std::to_string(width));
      if (d->at("num_rows").as_int() != rows)
        fail("resource '" + eff + "' num_rows " + std::to_string(d->at("num_rows").as_int()) +
             " != layer num_embeddings " + std::to_string(rows));
      mb_type = d->str_or("type", "Managed");
    }
    if (mb_type.find("NVL") != std::string::npos || mb_type.find("MPI") != std::string::npos)
      fail("memory block type " + mb_type + " is not part of this build");
    // a GPU layer reads its rows from device memory (Linear / User blocks);
    // LinearUVM and host layers from pinned host memory
    const bool device = layer_type == "GPULayer";
    if (device && mb_type.find("Host") != std::string::npos)
      fail("a GPULayer cannot use a Host memory block");
    if (!device && mb_type.find("User") != std::string::npos)
      fail("'User' memory blocks load only for GPU layers");
    auto s = std::make_shared<TableStorage>((size_t)bytes, device ? (device_ >= 0 ? device_ : 0) : -1);
    if (!key.empty()) resources_->insert(key, s);
    *fresh = true;
    return s;
  }

  // Fills `s` from entry `name` of the .nve file (device memory through a
  // pinned staging buffer).  An absent entry leaves host rows alone and zeroes
  // device rows, as the Python loader does.
  static void load_weights(const std::string& path, uint64_t name, TableStorage& s) {
    using loader_detail::fail;
    std::ifstream f(path, std::ios::binary);
    if (!f) fail("cannot open " + path);
    const loader_detail::NveEntry e = loader_detail::find_nve_entry(f, name, s.bytes, path);
    if (s.device < 0) {
      if (!e.found) return;
      f.seekg((std::streamoff)e.data_offset);
      f.read(static_cast<char*>(s.ptr), (std::streamsize)s.bytes);
      if (f.gcount() != (std::streamsize)s.bytes) fail(path + ": Problem reading tensor");
      return;
    }
    loader_detail::check_hip(hipSetDevice(s.device), "hipSetDevice");
    if (!e.found) {
      loader_detail::check_hip(hipMemset(s.ptr, 0, s.bytes), "hipMemset");
      return;
    }
    constexpr size_t kStage = size_t(64) << 20;
    void* stage = nullptr;
    loader_detail::check_hip(hipHostMalloc(&stage, kStage, hipHostMallocDefault), "hipHostMalloc");
    f.seekg((std::streamoff)e.data_offset);
    size_t done = 0;
    while (done < s.bytes) {
      const size_t n = s.bytes - done < kStage ? s.bytes - done : kStage;
      f.read(static_cast<char*>(stage), (std::streamsize)n);
      if (f.gcount() != (std::streamsize)n) {
        (void)hipHostFree(stage);
        fail(path + ": Problem reading tensor");
      }
      const hipError_t err = hipMemcpy(static_cast<char*>(s.ptr) + done, stage, n, hipMemcpyHostToDevice);
      if (err != hipSuccess) {
        (void)hipHostFree(stage);
        loader_detail::check_hip(err, "hipMemcpy");
      }
      done += n;
    }
    (void)hipHostFree(stage);
  }

  void add_layer(const loader_detail::Json& entry, bool v2, const loader_detail::Json* memblocks,
                 size_t cache_override, const std::set<std::string>& constants, std::set<std::string>& weights_done,
                 torch::inductor::AOTIModelPackageLoader& loader) {
    using loader_detail::fail;
    // the entry joins the list first, so that a failure part way through is
    // torn down with the rest
    layers_.emplace_back();
    LoadedLayer& l = layers_.back();
    l.layer_id = entry.at("id").as_int();
    l.module_path = entry.at("module_path").as_str();
    l.layer_type = entry.at("layer_type").as_str();
    const int64_t rows = entry.at("num_embeddings").as_int();
    const int64_t width = entry.at("embedding_size").as_int();
    const std::string dt = entry.at("dtype").as_str();
    int64_t esize;
    if (dt.find("float32") != std::string::npos) {
      l.dtype = NVE_DTYPE_FLOAT32;
      esize = 4;
    } else if (dt.find("float16") != std::string::npos) {
      l.dtype = NVE_DTYPE_FLOAT16;
      esize = 2;
    } else {
      fail("layer '" + l.module_path + "': unsupported dtype " + dt);
    }
    l.row_bytes = width * esize;
    if (l.layer_type != "GPULayer" && l.layer_type != "LinearUVM" && l.layer_type != "HostLayer")
      fail("layer '" + l.module_path + "': layer_type " + l.layer_type + " is not part of this build");
    const std::string fqn = marker_fqn(l.module_path);
    if (!constants.count(fqn))
      fail("marker constant '" + fqn + "' is not an updatable constant of the package (export it with "
           "export_aot, which keeps runtime constant folding on)");
    const loader_detail::Json* cfg = entry.find("config");
    const loader_detail::Json none;
    if (!cfg) cfg = &none;

    // storage: by resource key (schema 2) or one block per layer (schema 1)
    std::string key = v2 ? entry.str_or("storage_ref", "") : "";
    if (v2 && key.empty()) fail("v2 metadata: layer '" + l.module_path + "' has no 'storage_ref'");
    bool fresh = false;
    l.storage = storage_for(key, memblocks, l.layer_type, rows, width, rows * width * esize, &fresh);
    std::string weight_key = key;
    if (weight_key.empty()) {
      weight_key = l.module_path;
      for (auto& c : weight_key)
        if (c == '.') c = '_';
    }
    if (fresh && !weights_done.count(weight_key)) {
      load_weights(save_dir_ + "/weights/" + weight_key + ".nve", (uint64_t)l.layer_id, *l.storage);
      weights_done.insert(weight_key);
    }

    const int64_t default_row = cfg->int_or("default_row_index", -1);
    const std::string name = l.module_path.empty() ? std::string("layer") : l.module_path;
    if (l.layer_type == "GPULayer") {
      nve_gpu_embedding_layer_config_t c = nve_gpu_embedding_layer_config_default();
      c.layer_name = name.c_str();
      c.device_id = device_ >= 0 ? device_ : 0;
      c.embedding_table = l.storage->ptr;
      c.num_embeddings = rows;
      c.embedding_width_in_bytes = l.row_bytes;
      c.value_dtype = (nve_data_type_t)l.dtype;
      c.default_row_index = default_row;
      loader_detail::check_status(nve_gpu_embedding_layer_create(&l.layer, NVE_KEY_INT64, &c, nullptr),
                                  "nve_gpu_embedding_layer_create");
    } else if (l.layer_type == "LinearUVM") {
      const int64_t cache = cache_override > 0 ? (int64_t)cache_override : entry.at("gpu_cache_size").as_int();
      if (cache <= 0) fail("layer '" + l.module_path + "': a LinearUVM layer needs gpu_cache_size > 0");
      nve_gpu_table_config_t t = nve_gpu_table_config_default();
      t.device_id = device_ >= 0 ? device_ : 0;
      t.cache_size = (uint64_t)cache;
      t.row_size_in_bytes = l.row_bytes;
      t.value_dtype = (nve_data_type_t)l.dtype;
      t.count_misses = 1;
      const int64_t mm = cfg->int_or("max_modify_size", 0);
      if (mm > 0) t.max_modify_size = mm;
      const int64_t mode = cfg->int_or("kernel_mode", 0);
      t.kernel_mode_type = (uint64_t)mode;
      if (mode == 2) {
        const int64_t v = cfg->int_or("kernel_mode_value_1", 0);
        t.kernel_mode_value = (uint64_t)(v > 0 ? v : 1024);
      } else if (mode == 3) {
        // PipelineGather parameters are read through a pointer when the table
        // is made: {task size, auxiliary streams}
        const int64_t v1 = cfg->int_or("kernel_mode_value_1", 0), v2p = cfg->int_or("kernel_mode_value_2", 0);
        pipeline_params_[0] = (uint64_t)(v1 > 0 ? v1 : 1024);
        pipeline_params_[1] = (uint64_t)(v2p > 0 ? v2p : 16);
        t.kernel_mode_value = (uint64_t)(uintptr_t)pipeline_params_;
      }
      t.uvm_table = l.storage->ptr;
      t.uvm_num_rows = rows;
      if (entry.find("optimize_for_training") && entry.at("optimize_for_training").as_bool()) {
        loader_detail::check_hip(hipSetDevice(t.device_id), "hipSetDevice");
        loader_detail::check_hip(hipStreamCreate(&l.private_stream), "hipStreamCreate");
        t.private_stream = l.private_stream;
      }
      loader_detail::check_status(nve_gpu_table_create(&l.table, NVE_KEY_INT64, &t, nullptr), "nve_gpu_table_create");
      nve_linear_uvm_layer_config_t c = nve_linear_uvm_layer_config_default();
      c.layer_name = name.c_str();
      c.default_row_index = default_row;
      loader_detail::check_status(nve_linear_uvm_layer_create(&l.layer, NVE_KEY_INT64, &c, l.table, nullptr),
                                  "nve_linear_uvm_layer_create");
    } else {  // HostLayer
      nve_host_table_config_t t = nve_host_table_config_default();
      t.key_size = 8;
      t.max_value_size = l.row_bytes;
      t.value_dtype = (nve_data_type_t)l.dtype;
      loader_detail::check_status(
          nve_amd_linear_host_table_create(&l.table, NVE_KEY_INT64, &t, l.storage->ptr, rows, 0),
          "nve_amd_linear_host_table_create");
      // keys of no row read the default row: the one saved, else zeros
      std::vector<uint8_t> def((size_t)l.row_bytes, 0);
      if (const loader_detail::Json* d = cfg->find("default_embedding")) {
        if (d->kind == loader_detail::Json::Arr && (int64_t)d->a.size() == l.row_bytes)
          for (size_t i = 0; i < def.size(); ++i) def[i] = (uint8_t)d->a[i].as_int();
      }
      nve_host_embedding_layer_config_t c = nve_host_embedding_layer_config_default();
      c.layer_name = name.c_str();
      c.default_embedding = def.data();
      c.default_embedding_size = l.row_bytes;
      loader_detail::check_status(nve_host_embedding_layer_create(&l.layer, NVE_KEY_INT64, &c, l.table, nullptr),
                                  "nve_host_embedding_layer_create");
    }

    auto opts = at::TensorOptions().dtype(at::kLong);
    opts = device_ >= 0 ? opts.device(at::kCUDA, device_) : opts.device(at::kCPU);
    at::Tensor marker = at::tensor(std::vector<int64_t>{l.layer_id}, opts);
    write_marker(loader, fqn, marker);
    if (nve_torch_ops_register(marker.data_ptr(), l.layer, l.row_bytes, l.dtype, nullptr,
                               cfg->int_or("logging_interval", -1)) != 0)
      fail("nve_torch_ops_register refused the marker of layer '" + l.module_path + "'");
    l.marker = std::move(marker);  // registered: unregistered by teardown
  }

  uint64_t pipeline_params_[2] = {1024, 16};
};

}  // namespace nve

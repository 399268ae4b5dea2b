// A C++ inference host for an exported NVE model: loads the AOTInductor
// package of a save directory (written by pynve.torch.nve_export.export_aot),
// rebuilds its layers with nve::LayerDirectory (include/nve_loader.hpp), runs
// it on the inputs stored beside it and compares every output with the stored
// eager outputs byte for byte.  Then replaces the first marker constant by a
// copy (a data pointer the ops do not know, as a constant-buffer rebuild
// leaves it): the run must fail; after LayerDirectory::rebind_markers it must
// give the same outputs again.
//
//   aoti_loader_check <save_dir> <io_dir> <device_index>
//
// io_dir/io.txt lists the tensors, one per line: "in <file> <dtype> <dims...>"
// or "out <file> <dtype> <dims...>" with dtype int64, float32 or float16; each
// file holds the tensor's bytes, row-major.  Prints "ok ..." and exits 0.
#include <ATen/ATen.h>
#include <torch/csrc/inductor/aoti_package/model_package_loader.h>

#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <sstream>
#include <string>
#include <vector>

#include "nve_loader.hpp"

namespace {

struct Spec {
  std::string file;
  at::ScalarType type;
  std::vector<int64_t> dims;
};

at::ScalarType type_of(const std::string& s) {
  if (s == "int64") return at::kLong;
  if (s == "float32") return at::kFloat;
  if (s == "float16") return at::kHalf;
  throw std::runtime_error("unknown dtype " + s);
}

at::Tensor read_tensor(const std::string& dir, const Spec& sp) {
  at::Tensor t = at::empty(sp.dims, at::TensorOptions().dtype(sp.type));
  std::ifstream f(dir + "/" + sp.file, std::ios::binary);
  f.read(static_cast<char*>(t.data_ptr()), (std::streamsize)t.nbytes());
  if (f.gcount() != (std::streamsize)t.nbytes()) throw std::runtime_error("short file " + sp.file);
  return t;
}

bool same_bytes(const at::Tensor& a, const at::Tensor& b) {
  const at::Tensor x = a.contiguous().cpu(), y = b.contiguous().cpu();
  return x.scalar_type() == y.scalar_type() && x.sizes() == y.sizes() &&
         std::memcmp(x.data_ptr(), y.data_ptr(), x.nbytes()) == 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 4) {
    std::fprintf(stderr, "usage: %s <save_dir> <io_dir> <device_index>\n", argv[0]);
    return 2;
  }
  const std::string save_dir = argv[1], io_dir = argv[2];
  const int dev = std::atoi(argv[3]);
  try {
    std::vector<Spec> ins, outs;
    std::ifstream io(io_dir + "/io.txt");
    std::string line;
    while (std::getline(io, line)) {
      std::istringstream ls(line);
      std::string kind, file, dt;
      if (!(ls >> kind >> file >> dt)) continue;
      Spec sp{file, type_of(dt), {}};
      int64_t d;
      while (ls >> d) sp.dims.push_back(d);
      (kind == "in" ? ins : outs).push_back(sp);
    }
    const c10::Device device = dev >= 0 ? c10::Device(c10::kCUDA, (c10::DeviceIndex)dev) : c10::Device(c10::kCPU);
    std::vector<at::Tensor> inputs;
    for (const auto& sp : ins) inputs.push_back(read_tensor(io_dir, sp).to(device));

    torch::inductor::AOTIModelPackageLoader loader(save_dir + "/model.pt2", "model", false, 1,
                                                   (c10::DeviceIndex)dev);
    nve::LayerDirectory layers(save_dir, loader, dev);
    std::vector<at::Tensor> got = loader.run(inputs);
    if (got.size() != outs.size()) {
      std::printf("FAIL: %zu outputs, %zu expected\n", got.size(), outs.size());
      return 1;
    }
    for (size_t i = 0; i < outs.size(); ++i) {
      if (!same_bytes(got[i], read_tensor(io_dir, outs[i]))) {
        std::printf("FAIL: output %zu differs from the eager output\n", i);
        return 1;
      }
    }
    // a copy of the first marker in place of the registered one (as a
    // constant-buffer rebuild leaves it), then the markers bound again
    const nve::LoadedLayer& l0 = layers.layers().front();
    std::unordered_map<std::string, at::Tensor> copy{{nve::marker_fqn(l0.module_path), l0.marker.clone()}};
    loader.load_constants(copy, false, false, true);
    loader.load_constants(copy, true, false, true);
    bool refused = false;  // the op finds no layer for the copy's pointer
    try {
      (void)loader.run(inputs);
    } catch (const std::exception&) {
      refused = true;
    }
    if (!refused) {
      std::printf("FAIL: a marker that is not registered still reached a layer\n");
      return 1;
    }
    layers.rebind_markers(loader);
    got = loader.run(inputs);
    for (size_t i = 0; i < outs.size(); ++i) {
      if (!same_bytes(got[i], read_tensor(io_dir, outs[i]))) {
        std::printf("FAIL: output %zu differs after rebind_markers\n", i);
        return 1;
      }
    }
    std::printf("ok %zu layers, %zu outputs bit-exact, refused with a foreign marker, again after rebind_markers\n", layers.size(), outs.size());
    return 0;
  } catch (const std::exception& e) {
    std::printf("FAIL: %s\n", e.what());
    return 1;
  }
}

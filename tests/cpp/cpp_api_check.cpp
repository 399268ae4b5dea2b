// cpp_api_check.cpp -- a C++ host written against the reference's layer and
// table classes (include/embedding_layer.hpp, gpu_table.hpp,
// linear_embedding_layer.hpp, host_embedding_layer.hpp), compiled against
// include/nve_amd.hpp and linked with libnve_amd.so.
//
//   cpp_api_check host   LinearHostTable + HostEmbeddingLayer (no GPU needed)
//   cpp_api_check gpu    GPUEmbeddingLayer, GpuTable + LinearUVMEmbeddingLayer
//
// Both modes also call the tables through the reference's buffer_ptr<T>
// (BufferWrapper) signatures: find with a hit mask, update_accumulate on the
// host table; insert, find, update and erase on a cache-only GPU table with
// keys staged on the device by BufferWrapper::access_buffer.
//
// Tables hold multiples of 1/64 in [-1, 1), so every sum of up to 256 of them
// is exact in fp32 and the pooled results are compared bit for bit with a
// plain loop.  Prints "<mode> ok" and exits 0, or names the first mismatch
// and exits 1.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "nve_amd.hpp"

namespace {

int fail(const char* what) {
  std::printf("FAIL: %s\n", what);
  return 1;
}

#define HIP_OK(expr)                                               \
  do {                                                             \
    if ((expr) != hipSuccess) return fail("HIP call failed: " #expr); \
  } while (0)

std::vector<float> dyadic_table(int64_t rows, int64_t dim, unsigned seed) {
  std::mt19937 gen(seed);
  std::uniform_int_distribution<int> d(-64, 63);
  std::vector<float> t((size_t)(rows * dim));
  for (auto& v : t) v = (float)d(gen) / 64.0f;
  return t;
}

// gather rows, and Fixed-hotness sums in key order
void reference(const std::vector<float>& t, int64_t dim, const std::vector<int64_t>& keys, int64_t hot,
               std::vector<float>* gathered, std::vector<float>* pooled) {
  const int64_t n = (int64_t)keys.size();
  gathered->assign((size_t)(n * dim), 0.0f);
  pooled->assign((size_t)(n / hot * dim), 0.0f);
  for (int64_t i = 0; i < n; ++i)
    for (int64_t e = 0; e < dim; ++e) {
      const float v = t[(size_t)(keys[(size_t)i] * dim + e)];
      (*gathered)[(size_t)(i * dim + e)] = v;
      (*pooled)[(size_t)(i / hot * dim + e)] += v;
    }
}

bool same(const std::vector<float>& a, const std::vector<float>& b) {
  return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
}

int run_host() {
  const int64_t rows = 5000, dim = 32, hot = 8, bags = 300;
  std::vector<float> table = dyadic_table(rows, dim, 7);
  nve::LinearHostTableConfig tc;
  tc.emb_table = table.data();
  tc.num_rows = rows;
  tc.max_value_size = dim * 4;
  tc.value_dtype = nve::DataType_t::Float32;
  auto host_table = std::make_shared<nve::LinearHostTable<int64_t>>(tc);
  nve::HostEmbeddingLayer<int64_t>::Config lc;
  lc.layer_name = "cpp";
  nve::HostEmbeddingLayer<int64_t> layer(lc, host_table);
  auto ctx = layer.create_execution_context(nullptr, nullptr, nullptr, nullptr);

  std::mt19937 gen(3);
  std::uniform_int_distribution<int64_t> kd(0, rows - 1);
  std::vector<int64_t> keys((size_t)(bags * hot));
  for (auto& k : keys) k = kd(gen);
  std::vector<float> want_g, want_p;
  reference(table, dim, keys, hot, &want_g, &want_p);

  std::vector<float> got_g(want_g.size()), got_p(want_p.size());
  layer.lookup(ctx, (int64_t)keys.size(), keys.data(), got_g.data(), dim * 4, nullptr, nullptr, nullptr);
  nve::EmbeddingLayerBase::PoolingParams pp;
  pp.pooling_type = nve::PoolingType_t::Sum;
  pp.sparse_type = nve::SparseType_t::Fixed;
  pp.fixed_hotness = hot;
  pp.output_type = nve::DataType_t::Float32;
  layer.lookup(ctx, (int64_t)keys.size(), keys.data(), got_p.data(), dim * 4, nullptr, &pp, nullptr);
  ctx->wait();
  if (!same(got_g, want_g)) return fail("host gather");
  if (!same(got_p, want_p)) return fail("host Sum");
  // the table API of the same table
  auto tctx = host_table->create_execution_context(nullptr, nullptr);
  std::vector<float> found(want_g.size());
  host_table->find(tctx, (int64_t)keys.size(), keys.data(), nullptr, dim * 4, found.data(), nullptr);
  if (!same(found, want_g)) return fail("host table find");
  {
    // the reference's buffer_ptr signatures (table.hpp:104-180)
    const int64_t n = (int64_t)keys.size();
    auto kb = std::make_shared<nve::BufferWrapper<const void>>(tctx, "keys", keys.data(), keys.size() * 8);
    std::vector<float> found2(want_g.size());
    std::vector<nve::bitmask64_t> mask((size_t)((n + 63) / 64), 0);
    auto vb = std::make_shared<nve::BufferWrapper<void>>(tctx, "values", found2.data(), found2.size() * 4);
    auto mb = std::make_shared<nve::BufferWrapper<nve::bitmask64_t>>(tctx, "hit_mask", mask.data(), mask.size() * 8);
    host_table->find(tctx, n, kb, mb, dim * 4, vb, nullptr);
    tctx->wait();
    if (!same(found2, want_g)) return fail("host table find through buffer_ptr");
    for (int64_t i = 0; i < n; ++i)
      if (!((mask[(size_t)(i / 64)] >> (i % 64)) & 1)) return fail("host table hit mask through buffer_ptr");
    // +1 on the first key's row, then read it back
    std::vector<float> ones((size_t)dim, 1.0f), row((size_t)dim);
    auto k0 = std::make_shared<nve::BufferWrapper<const void>>(tctx, "k0", keys.data(), 8);
    auto ub = std::make_shared<nve::BufferWrapper<const void>>(tctx, "updates", ones.data(), ones.size() * 4);
    auto rb = std::make_shared<nve::BufferWrapper<void>>(tctx, "row", row.data(), row.size() * 4);
    host_table->update_accumulate(tctx, 1, k0, dim * 4, dim * 4, ub, nve::DataType_t::Float32);
    host_table->find(tctx, 1, k0, nullptr, dim * 4, rb, nullptr);
    tctx->wait();
    for (int64_t e = 0; e < dim; ++e)
      if (row[(size_t)e] != want_g[(size_t)e] + 1.0f) return fail("host update_accumulate through buffer_ptr");
    if (kb->get_buffer(hipMemoryTypeDevice) != nullptr || kb->data() != keys.data())
      return fail("BufferWrapper made a copy nobody asked for");
    // updates of another type than the table's are refused (as the
    // reference's LinearHostTable accumulates into Float32 rows only)
    try {
      host_table->update_accumulate(tctx, 1, k0, dim * 4, dim * 4, ub, nve::DataType_t::Float16);
      return fail("Float16 updates into a Float32 host table accepted");
    } catch (const nve::Exception& e) {
      if (e.status() != NVE_ERROR_RUNTIME) return fail("wrong status for a mixed-type accumulate");
    }
  }
  // errors surface as nve::Exception with the C status
  try {
    layer.lookup(ctx, 4, nullptr, got_g.data(), dim * 4, nullptr, nullptr, nullptr);
    return fail("null keys accepted");
  } catch (const nve::Exception& e) {
    if (e.status() != NVE_ERROR_INVALID_ARGUMENT) return fail("wrong status for null keys");
  }
  std::printf("host ok\n");
  return 0;
}

// insert / find / update / erase of a cache-only GPU table (so that the hit
// mask means residency) through the reference's buffer_ptr signatures, the
// keys staged on the device by BufferWrapper::access_buffer
int table_through_buffer_ptr(hipStream_t s, const std::vector<int64_t>& keys, const std::vector<float>& want_g,
                             int64_t dim) {
  const int64_t n = 512, words = n / 64;
  nve::GPUTableConfig tc;
  tc.cache_size = 2 << 20;  // 1024 sets of 8 ways: 512 keys all fit
  tc.row_size_in_bytes = dim * 4;
  tc.value_dtype = nve::DataType_t::Float32;
  auto gt = std::make_shared<nve::GpuTable<int64_t>>(tc);
  auto tctx = gt->create_execution_context(s, s);
  auto host_keys = std::make_shared<nve::BufferWrapper<const void>>(tctx, "keys", keys.data(), n * 8);
  const void* dk = host_keys->access_buffer(hipMemoryTypeDevice, true, s);
  if (dk == nullptr || dk == keys.data() || host_keys->get_last_access() != hipMemoryTypeDevice)
    return fail("access_buffer did not stage the keys on the device");
  auto kb = std::make_shared<nve::BufferWrapper<const void>>(tctx, "dkeys", dk, n * 8);
  // and back: a host copy of the device keys, made once (a const buffer)
  const void* hk = kb->access_buffer(hipMemoryTypeHost, true, s);
  if (hk == nullptr || hk == dk || std::memcmp(hk, keys.data(), (size_t)n * 8) != 0 ||
      kb->get_buffer(hipMemoryTypeDevice) != dk || kb->access_buffer(hipMemoryTypeHost, true, s) != hk)
    return fail("access_buffer did not stage the device keys on the host");
  auto rows = std::make_shared<nve::BufferWrapper<const void>>(tctx, "rows", want_g.data(), (size_t)(n * dim) * 4);
  gt->insert(tctx, n, kb, dim * 4, dim * 4, rows);
  std::vector<float> vals((size_t)(n * dim));
  std::vector<nve::bitmask64_t> mask((size_t)words);
  auto vb = std::make_shared<nve::BufferWrapper<void>>(tctx, "values", vals.data(), vals.size() * 4);
  auto mb = std::make_shared<nve::BufferWrapper<nve::bitmask64_t>>(tctx, "hit_mask", mask.data(), mask.size() * 8);
  auto find = [&]() {
    std::fill(mask.begin(), mask.end(), 0);
    std::fill(vals.begin(), vals.end(), 0.0f);
    gt->find(tctx, n, kb, mb, dim * 4, vb, nullptr);
    tctx->wait();
    return hipStreamSynchronize(s) == hipSuccess;
  };
  auto hit = [&](int64_t i) { return (mask[(size_t)(i / 64)] >> (i % 64)) & 1; };
  auto row_is = [&](int64_t i, const float* want) {
    return std::memcmp(&vals[(size_t)(i * dim)], want, (size_t)dim * 4) == 0;
  };
  if (!find()) return fail("find through buffer_ptr");
  for (int64_t i = 0; i < n; ++i)
    if (!hit(i) || !row_is(i, &want_g[(size_t)(i * dim)])) return fail("GPU table insert + find through buffer_ptr");
  // new rows for keys[16..31], then keys[0..7] erased: the erased keys (and
  // later copies of them) miss, the updated ones return a new row
  std::vector<float> upd((size_t)(16 * dim));
  for (size_t j = 0; j < upd.size(); ++j) upd[j] = -(float)(j % 97) / 8.0f;
  auto uk = std::make_shared<nve::BufferWrapper<const void>>(tctx, "ukeys", keys.data() + 16, 16 * 8);
  auto ub = std::make_shared<nve::BufferWrapper<const void>>(tctx, "updates", upd.data(), upd.size() * 4);
  auto ek = std::make_shared<nve::BufferWrapper<const void>>(tctx, "ekeys", keys.data(), 8 * 8);
  gt->update(tctx, 16, uk, dim * 4, dim * 4, ub);
  gt->erase(tctx, 8, ek);
  if (!find()) return fail("find after update / erase");
  for (int64_t i = 0; i < n; ++i) {
    bool erased = false, updated = false, match = false;
    for (int64_t j = 0; j < 8; ++j) erased = erased || keys[(size_t)i] == keys[(size_t)j];
    for (int64_t j = 0; j < 16; ++j)  // a key given twice may keep either row
      if (keys[(size_t)i] == keys[(size_t)(16 + j)]) {
        updated = true;
        match = match || row_is(i, &upd[(size_t)(j * dim)]);
      }
    if (erased) {
      if (hit(i)) return fail("an erased key still hits");
    } else if (!hit(i)) {
      return fail("a resident key missed after update / erase");
    } else if (updated ? !match : !row_is(i, &want_g[(size_t)(i * dim)])) {
      return fail("GPU table update through buffer_ptr");
    }
  }
  return 0;
}

int run_gpu() {
  const int64_t rows = 20000, dim = 64, hot = 16, bags = 256;
  std::vector<float> table = dyadic_table(rows, dim, 11);
  void* d_table = nullptr;
  HIP_OK(hipMalloc(&d_table, table.size() * 4));
  HIP_OK(hipMemcpy(d_table, table.data(), table.size() * 4, hipMemcpyHostToDevice));
  std::mt19937 gen(5);
  std::uniform_int_distribution<int64_t> kd(0, rows - 1);
  std::vector<int64_t> keys((size_t)(bags * hot));
  for (auto& k : keys) k = kd(gen);
  std::vector<float> want_g, want_p;
  reference(table, dim, keys, hot, &want_g, &want_p);
  hipStream_t s = nullptr;
  HIP_OK(hipStreamCreate(&s));
  int rc = 0;
  {
    nve::GPUEmbeddingLayerConfig cfg;
    cfg.layer_name = "cpp_gpu";
    cfg.embedding_table = d_table;
    cfg.num_embeddings = rows;
    cfg.embedding_width_in_bytes = dim * 4;
    cfg.value_dtype = nve::DataType_t::Float32;
    nve::GPUEmbeddingLayer<int64_t> layer(cfg);
    auto ctx = layer.create_execution_context(s, s, nullptr, nullptr);
    std::vector<float> got_g(want_g.size()), got_p(want_p.size());
    layer.lookup(ctx, (int64_t)keys.size(), keys.data(), got_g.data(), dim * 4, nullptr, nullptr, nullptr);
    nve::EmbeddingLayerBase::PoolingParams pp;
    pp.pooling_type = nve::PoolingType_t::Sum;
    pp.fixed_hotness = hot;
    pp.output_type = nve::DataType_t::Float32;
    layer.lookup(ctx, (int64_t)keys.size(), keys.data(), got_p.data(), dim * 4, nullptr, &pp, nullptr);
    ctx->wait();
    HIP_OK(hipStreamSynchronize(s));
    if (!same(got_g, want_g)) rc = fail("GPU layer gather");
    if (!rc && !same(got_p, want_p)) rc = fail("GPU layer Sum");
  }
  if (!rc) {
    // a cache over a pinned backing table, read through a LinearUVM layer
    float* backing = nullptr;
    HIP_OK(hipHostMalloc((void**)&backing, table.size() * 4, hipHostMallocDefault));
    std::memcpy(backing, table.data(), table.size() * 4);
    nve::GPUTableConfig tc;
    tc.cache_size = 2 << 20;
    tc.row_size_in_bytes = dim * 4;
    tc.uvm_table = backing;
    tc.uvm_num_rows = rows;
    tc.value_dtype = nve::DataType_t::Float32;
    auto gt = std::make_shared<nve::GpuTable<int64_t>>(tc);
    {
      nve::LinearUVMEmbeddingLayer<int64_t>::Config lc;
      lc.layer_name = "cpp_uvm";
      lc.insert_heuristic = std::make_shared<nve::NeverInsertHeuristic>();
      nve::LinearUVMEmbeddingLayer<int64_t> layer(lc, gt);
      auto ctx = layer.create_execution_context(s, s, nullptr, nullptr);
      auto tctx = gt->create_execution_context(s, s);
      gt->insert_from_uvm(tctx, 512, keys.data());  // the batch's first 512 keys made resident
      std::vector<float> got_g(want_g.size());
      layer.lookup(ctx, (int64_t)keys.size(), keys.data(), got_g.data(), dim * 4, nullptr, nullptr, nullptr);
      ctx->wait();
      HIP_OK(hipStreamSynchronize(s));
      if (!same(got_g, want_g)) rc = fail("LinearUVM layer gather");
    }
    gt.reset();
    HIP_OK(hipHostFree(backing));
  }
  if (!rc) rc = table_through_buffer_ptr(s, keys, want_g, dim);
  HIP_OK(hipStreamDestroy(s));
  HIP_OK(hipFree(d_table));
  if (!rc) std::printf("gpu ok\n");
  return rc;
}

}  // namespace

int main(int argc, char** argv) {
  const char* mode = argc > 1 ? argv[1] : "host";
  try {
    if (std::strcmp(mode, "host") == 0) return run_host();
    if (std::strcmp(mode, "gpu") == 0) return run_gpu();
  } catch (const nve::Exception& e) {
    std::printf("FAIL: nve::Exception status %d: %s\n", (int)e.status(), e.what());
    return 1;
  }
  std::printf("usage: cpp_api_check host|gpu\n");
  return 2;
}

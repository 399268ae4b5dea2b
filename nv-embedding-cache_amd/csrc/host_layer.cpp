// host_layer.cpp -- see host_layer.hpp.
#include "host_layer.hpp"

#include <algorithm>
#include <cstring>

#include "host_kernels.hpp"
#include "trace.hpp"

namespace nve_amd {

namespace {

// Whether a GPU is present at all: without one every pointer is host memory
// and no HIP call is made for a host-layer buffer.
bool hip_device_present() {
  static const bool present = [] {
    int n = 0;
    const bool ok = hipGetDeviceCount(&n) == hipSuccess && n > 0;
    (void)hipGetLastError();
    return ok;
  }();
  return present;
}

bool is_device(const void* p) { return p && hip_device_present() && mem_kind(p) == MemKind::Device; }

// Host view of a caller buffer (BufferWrapper::access_buffer with copied
// content, buffer_wrapper.hpp:34-93): p itself unless it is device memory.
const void* host_view_in(ExecutionContext& ctx, const char* name, const void* p, size_t bytes) {
  if (!is_device(p) || bytes == 0) return p;
  void* h = ctx.host_buffer(name, bytes);
  NVE_HIP(hipMemcpyAsync(h, p, bytes, hipMemcpyDeviceToHost, ctx.lookup_stream()));
  NVE_HIP(hipStreamSynchronize(ctx.lookup_stream()));
  return h;
}

// Host-writable stand-in for an output buffer; write_back copies it to the
// caller's device buffer when they differ.
void* host_view_out(ExecutionContext& ctx, const char* name, void* p, size_t bytes) {
  if (!is_device(p) || bytes == 0) return p;
  return ctx.host_buffer(name, bytes);
}

void write_back(ExecutionContext& ctx, void* user, const void* host, size_t bytes) {
  if (user == host || bytes == 0) return;
  NVE_HIP(hipMemcpyAsync(user, host, bytes, hipMemcpyHostToDevice, ctx.lookup_stream()));
  NVE_HIP(hipStreamSynchronize(ctx.lookup_stream()));
}

int64_t load_offset(const void* offsets, int key_bytes, int64_t i) {
  return key_bytes == 4 ? (int64_t) static_cast<const int32_t*>(offsets)[i]
                        : static_cast<const int64_t*>(offsets)[i];
}

// values per stored row (layer_utils.cpp:368-380)
int64_t row_values(int dtype, int64_t row_bytes) {
  if (is_rowwise(dtype)) {
    NVE_CHECK(row_bytes > meta_bytes(dtype), "Quantized row size smaller than its scale/offset metadata");
    return row_bytes - meta_bytes(dtype);
  }
  NVE_CHECK(row_bytes % dtype_size(dtype) == 0, "Table row size not a multiple of the value element size");
  return row_bytes / dtype_size(dtype);
}

}  // namespace

// ---------------------------------------------------------------------------
// LinearHostTable
// ---------------------------------------------------------------------------
LinearHostTable::LinearHostTable(int key_bytes, const LinearHostTableConfig& cfg)
    : key_bytes_(key_bytes), cfg_(cfg) {
  // LinearHostTableConfig::check (linear_host_table.cpp:21-28)
  NVE_CHECK_ARG(key_bytes == 4 || key_bytes == 8, "Unsupported key size ", key_bytes);
  NVE_CHECK_ARG(cfg_.emb_table != nullptr, "The host table needs the rows' memory (emb_table)");
  NVE_CHECK_ARG(cfg_.num_rows > 0, "A host table needs at least one row");
  NVE_CHECK_ARG(cfg_.row_bytes > 0, "A host table needs a positive row size");
  NVE_CHECK_ARG(cfg_.max_threads > 0, "max_threads must be positive");
  NVE_CHECK_ARG(cfg_.value_dtype == kF32 || cfg_.value_dtype == kF16 || is_rowwise(cfg_.value_dtype),
                "Unsupported host table value type ", cfg_.value_dtype);
  if (is_rowwise(cfg_.value_dtype))
    NVE_CHECK_ARG(cfg_.row_bytes > meta_bytes(cfg_.value_dtype), "Row too small for its scale/offset");
  else
    NVE_CHECK_ARG(cfg_.row_bytes % dtype_size(cfg_.value_dtype) == 0,
                  "Row size is not a whole number of values");
}

int64_t LinearHostTable::threads(ExecutionContext& ctx) const {
  return std::max<int64_t>(1, std::min(ctx.pool().num_workers(), cfg_.max_threads));
}

int64_t LinearHostTable::find(ExecutionContext& ctx, int64_t n, const void* keys, uint64_t* hit_mask,
                              int64_t value_stride, void* values) {
  NVE_CHECK_ARG(n > 0, "Invalid number of keys");
  NVE_CHECK_ARG(keys != nullptr, "Invalid keys");
  NVE_CHECK_ARG(values != nullptr, "Invalid values");
  const int64_t hits = hostk::gather(ctx.pool(), threads(ctx), n, keys, key_bytes_, hit_mask,
                                     static_cast<uint8_t*>(values), value_stride,
                                     static_cast<const uint8_t*>(cfg_.emb_table), cfg_.row_bytes,
                                     (uint64_t)cfg_.num_rows);
  ctx.host_lookup_counter() += hits;
  return hits;
}

void LinearHostTable::find_any(ExecutionContext& ctx, int64_t n, const void* keys, uint64_t* hit_mask,
                               int64_t value_stride, void* values, int64_t* /*value_sizes*/) {
  NVE_CHECK_ARG(n > 0, "Invalid number of keys");
  NVE_CHECK_ARG(value_stride >= cfg_.row_bytes, "Value stride is smaller than a row");
  const size_t mask_bytes = (size_t)((n + 63) / 64) * 8;
  const void* hk = host_view_in(ctx, "find_keys", keys, (size_t)n * key_bytes_);
  uint64_t* hm = hit_mask;
  if (is_device(hit_mask)) {
    hm = static_cast<uint64_t*>(const_cast<void*>(host_view_in(ctx, "find_hits", hit_mask, mask_bytes)));
  }
  // rows already found keep their bytes, so device values are staged in full
  void* hv = values;
  const size_t vbytes = (size_t)n * value_stride;
  if (is_device(values)) hv = const_cast<void*>(host_view_in(ctx, "find_values", values, vbytes));
  find(ctx, n, hk, hm, value_stride, hv);
  write_back(ctx, values, hv, vbytes);
  write_back(ctx, hit_mask, hm, hit_mask ? mask_bytes : 0);
}

void LinearHostTable::update(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                             int64_t value_size, const void* values) {
  NVE_CHECK_ARG(n > 0, "Invalid number of keys");
  NVE_CHECK_ARG(keys != nullptr && values != nullptr, "Invalid keys or values");
  NVE_CHECK_ARG(value_size == cfg_.row_bytes, "Invalid value size");
  const void* hk = host_view_in(ctx, "update_keys", keys, (size_t)n * key_bytes_);
  const void* hv = host_view_in(ctx, "update_values", values, (size_t)n * value_stride);
  hostk::update_rows(ctx.pool(), threads(ctx), n, hk, key_bytes_, static_cast<const uint8_t*>(hv),
                     value_stride, static_cast<uint8_t*>(cfg_.emb_table), cfg_.row_bytes,
                     (uint64_t)cfg_.num_rows);
}

void LinearHostTable::update_accumulate(ExecutionContext& ctx, int64_t n, const void* keys,
                                        int64_t value_stride, int64_t value_size, const void* values,
                                        int value_type) {
  NVE_CHECK_ARG(n > 0, "Invalid number of keys");
  NVE_CHECK_ARG(keys != nullptr && values != nullptr, "Invalid keys or updates");
  NVE_CHECK_ARG(value_size == cfg_.row_bytes, "Invalid update size");
  NVE_CHECK(cfg_.value_dtype == kF32, "Accumulating into a host table needs fp32 rows");
  NVE_CHECK(value_type == kF32, "Unsupported update type ", value_type);
  const void* hk = host_view_in(ctx, "update_keys", keys, (size_t)n * key_bytes_);
  const void* hv = host_view_in(ctx, "update_values", values, (size_t)n * value_stride);
  hostk::accumulate_rows(ctx.pool(), threads(ctx), n, hk, key_bytes_, static_cast<const uint8_t*>(hv),
                         value_stride, static_cast<uint8_t*>(cfg_.emb_table), cfg_.row_bytes,
                         (uint64_t)cfg_.num_rows, kF32);
}

std::shared_ptr<ExecutionContext> LinearHostTable::create_execution_context(
    hipStream_t lookup, hipStream_t modify, std::shared_ptr<ThreadPool> pool) {
  return std::make_shared<ExecutionContext>(-1, lookup, modify, std::move(pool));
}

// ---------------------------------------------------------------------------
// HostEmbeddingLayer
// ---------------------------------------------------------------------------
HostEmbeddingLayer::HostEmbeddingLayer(int key_bytes, const HostEmbeddingLayerConfig& cfg,
                                       std::shared_ptr<LinearHostTable> table)
    : EmbeddingLayer(key_bytes, -1), cfg_(cfg), table_(std::move(table)) {
  NVE_CHECK_ARG(table_ != nullptr, "The host layer needs a host table");
  NVE_CHECK_ARG(table_->key_bytes() == key_bytes, "The host table's key type differs from the layer's");
  NVE_CHECK_ARG(cfg_.default_embedding.empty() ||
                    (int64_t)cfg_.default_embedding.size() == table_->config().row_bytes,
                "The default embedding must be exactly one row of the table (",
                table_->config().row_bytes, " bytes)");
}

std::shared_ptr<ExecutionContext> HostEmbeddingLayer::create_execution_context(
    hipStream_t lookup, hipStream_t modify, std::shared_ptr<ThreadPool> pool) {
  return table_->create_execution_context(lookup, modify, std::move(pool));
}

void HostEmbeddingLayer::lookup(ExecutionContext& ctx, int64_t num_keys, const void* keys, void* output,
                                int64_t output_stride, uint64_t* hitmask, const PoolingParams* pp,
                                float* hitrates) {
  NVE_CHECK_ARG(num_keys >= 0, "Invalid number of keys");
  NVE_CHECK_ARG(keys != nullptr || num_keys == 0, "Invalid keys");
  if (pp) validate_pool_params(*pp);
  const LinearHostTableConfig& tc = table_->config();
  const int64_t row = tc.row_bytes;

  if (num_keys == 0) {
    // an all-empty batch: CSR bags still get zero rows (host_embedding_layer.cpp:73-96)
    const int64_t out_rows = lookup_output_rows(0, pp);
    if (out_rows > 0) {
      NVE_CHECK_ARG(output != nullptr, "Invalid output");
      const size_t bytes = (size_t)out_rows * output_stride;
      void* h = host_view_out(ctx, "output", output, bytes);
      std::memset(h, 0, bytes);
      write_back(ctx, output, h, bytes);
    }
    if (hitrates) hitrates[0] = 1.0f;
    return;
  }
  NVE_CHECK_ARG(output != nullptr, "Invalid output");
  // same-type Concatenate is the raw gather (host_embedding_layer.cpp:110-124)
  if (pp && pp->pooling_type == NVE_POOL_CONCATENATE && pp->output_type == tc.value_dtype) pp = nullptr;
  if (!pp)
    NVE_CHECK_ARG(output_stride >= row, "Output stride ", output_stride, " is smaller than a row (", row,
                  " bytes)");

  const void* hkeys = host_view_in(ctx, "keys", keys, (size_t)num_keys * key_bytes_);
  const size_t out_bytes = (size_t)num_keys * output_stride;
  uint8_t* gathered;
  int64_t gather_stride;
  void* hout = nullptr;
  if (pp) {  // one raw row per key, reduced below
    gathered = static_cast<uint8_t*>(ctx.host_buffer("pool_gather", (size_t)num_keys * row));
    gather_stride = row;
  } else {
    hout = host_view_out(ctx, "output", output, out_bytes);
    gathered = static_cast<uint8_t*>(hout);
    gather_stride = output_stride;
  }

  // hit bits are needed by the caller or to fill missed keys with the default row
  const bool need_mask = hitmask != nullptr || !cfg_.default_embedding.empty();
  const size_t mask_bytes = (size_t)((num_keys + 63) / 64) * 8;
  uint64_t* hm = nullptr;
  if (need_mask) {
    hm = hitmask ? static_cast<uint64_t*>(host_view_out(ctx, "hitmask", hitmask, mask_bytes))
                 : static_cast<uint64_t*>(ctx.host_buffer("hitmask", mask_bytes));
    std::memset(hm, 0, mask_bytes);
  }

  ctx.host_lookup_counter() = 0;
  const int64_t hits = table_->find(ctx, num_keys, hkeys, hm, gather_stride, gathered);

  if (hits < num_keys && !cfg_.default_embedding.empty()) {
    const uint8_t* def = cfg_.default_embedding.data();
    const int64_t workers = std::max<int64_t>(1, ctx.pool().num_workers());
    const int64_t per = std::max<int64_t>(1, (num_keys + workers - 1) / workers);
    hostk::run_tasks(ctx.pool(), (num_keys + per - 1) / per, [&](int64_t t) {
      const int64_t e = std::min(num_keys, (t + 1) * per);
      for (int64_t k = t * per; k < e; ++k)
        if (!((hm[k >> 6] >> (k & 63)) & 1ull)) std::memcpy(gathered + k * gather_stride, def, (size_t)row);
    });
  }

  if (pp) {
    const int64_t out_rows = lookup_output_rows(num_keys, pp);
    pool_gathered(ctx, *pp, gathered, num_keys, static_cast<uint8_t*>(output), output_stride, out_rows);
  } else {
    write_back(ctx, output, hout, out_bytes);
  }
  if (hitmask) write_back(ctx, hitmask, hm, mask_bytes);
  if (hitrates) hitrates[0] = (float)hits / (float)num_keys;
}

void HostEmbeddingLayer::pool_gathered(ExecutionContext& ctx, const PoolingParams& pp,
                                       const uint8_t* gathered, int64_t num_keys, uint8_t* output,
                                       int64_t output_stride, int64_t out_rows) {
  const LinearHostTableConfig& tc = table_->config();
  const int vdt = tc.value_dtype;
  const int odt = pp.output_type;
  const bool concat = pp.pooling_type == NVE_POOL_CONCATENATE;
  NVE_CHECK_ARG(odt == kF32 || odt == kF16,
                "Host pooling writes fp32 or fp16 (the table's own type only for Concatenate)");
  const int64_t count = row_values(vdt, tc.row_bytes);
  const int oes = odt == kF16 ? 2 : 4;
  NVE_CHECK_ARG(output_stride >= count * oes, "Output stride ", output_stride, " holds fewer than ", count,
                " values of the output type");
  const int64_t workers = std::max<int64_t>(1, ctx.pool().num_workers());
  const size_t out_bytes = (size_t)out_rows * output_stride;
  uint8_t* hout = static_cast<uint8_t*>(host_view_out(ctx, "pool_output", output, out_bytes));

  if (concat) {  // one converted / dequantized row per key, no bag fields read
    hostk::convert(ctx.pool(), workers, vdt, count, odt, num_keys, gathered, tc.row_bytes, hout,
                   output_stride);
    write_back(ctx, output, hout, out_bytes);
    return;
  }

  hostk::PoolSpec sp;
  sp.dtype = vdt;
  sp.count = count;
  sp.pooling = pp.pooling_type;
  sp.sparse = pp.sparse_type;
  sp.out_type = odt;
  sp.offset_bytes = key_bytes_;
  int64_t num_bags;
  if (pp.sparse_type == NVE_SPARSE_FIXED) {
    NVE_CHECK_ARG(num_keys % pp.fixed_hotness == 0, "Number of keys does not divide by fixed hotness");
    num_bags = num_keys / pp.fixed_hotness;
    sp.fixed_hotness = pp.fixed_hotness;
  } else {
    // offsets have the key type; the CSR contract is checked before any row
    // is read (layer_utils.cpp:432-448)
    num_bags = pp.num_csr_offsets - 1;
    const void* off = host_view_in(ctx, "offsets", pp.csr_offsets, (size_t)pp.num_csr_offsets * key_bytes_);
    NVE_CHECK_ARG(load_offset(off, key_bytes_, 0) == 0, "CSR offsets must start at 0");
    for (int64_t b = 0; b < num_bags; ++b)
      NVE_CHECK_ARG(load_offset(off, key_bytes_, b) <= load_offset(off, key_bytes_, b + 1),
                    "CSR offsets must not decrease (offsets[", b + 1, "] < offsets[", b, "])");
    NVE_CHECK_ARG(load_offset(off, key_bytes_, num_bags) == num_keys,
                  "The last CSR offset must equal the number of keys (", num_keys, ")");
    sp.offsets = off;
  }
  NVE_CHECK(num_bags == out_rows, "Pooled row count mismatch");
  if (pp.weights) {
    NVE_CHECK_ARG(pp.weight_type == kF32 || pp.weight_type == kF16, "Pooling weights must be fp32 or fp16");
    sp.weights = host_view_in(ctx, "weights", pp.weights, (size_t)num_keys * dtype_size(pp.weight_type));
    sp.weight_type = pp.weight_type;
  }
  hostk::pool(ctx.pool(), workers, sp, num_bags, gathered, tc.row_bytes, hout, output_stride);
  write_back(ctx, output, hout, out_bytes);
}

void HostEmbeddingLayer::insert(ExecutionContext&, int64_t, const void*, int64_t, int64_t, const void*,
                                int64_t table_id) {
  NVE_CHECK(table_id < 1, "Invalid table_id");
  // a linear host table holds every row already (linear_host_table.hpp:110-114)
  NVE_LOG_INFO("Inserting into linear host table has no effect");
}

void HostEmbeddingLayer::update(ExecutionContext& ctx, int64_t n, const void* keys, int64_t value_stride,
                                int64_t value_size, const void* values, int64_t table_id) {
  NVE_CHECK(table_id < 1, "Invalid table_id");
  table_->update(ctx, n, keys, value_stride, value_size, values);
}

void HostEmbeddingLayer::accumulate(ExecutionContext& ctx, int64_t n, const void* keys,
                                    int64_t value_stride, int64_t value_size, const void* values,
                                    int value_type, int64_t table_id) {
  NVE_CHECK(table_id < 1, "Invalid table_id");
  table_->update_accumulate(ctx, n, keys, value_stride, value_size, values, value_type);
}

void HostEmbeddingLayer::clear(ExecutionContext&) {
  NVE_LOG_INFO("Clearing linear host table has no effect");  // linear_host_table.hpp:65-68
}

void HostEmbeddingLayer::erase(ExecutionContext&, int64_t n, const void* keys, int64_t table_id) {
  NVE_CHECK(table_id < 1, "Invalid table_id");
  if (n < 1) return;
  NVE_CHECK(keys != nullptr, "Invalid keys");
  NVE_LOG_INFO("Erasing from linear host table has no effect");  // linear_host_table.hpp:72-75
}

}  // namespace nve_amd

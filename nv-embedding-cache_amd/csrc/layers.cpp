// layers.cpp -- layer base, pooling-parameter validation, GPUEmbeddingLayer,
// LinearUVMEmbeddingLayer and the insert heuristics.
#include "layers.hpp"

#include <climits>
#include <cmath>

namespace nve_amd {

// ---------------------------------------------------------------------------
// pooling parameters (layer_utils.cpp:277-305, :307-328)
// ---------------------------------------------------------------------------
void validate_pool_params(const PoolingParams& pp) {
  NVE_CHECK_ARG(pp.output_type != kUnknown, "Unknown output type");
  if (pp.pooling_type == NVE_POOL_CONCATENATE) return;
  NVE_CHECK_ARG(pp.pooling_type >= NVE_POOL_SUM && pp.pooling_type <= NVE_POOL_WEIGHTED_MEAN,
                "Unsupported pooling type ", pp.pooling_type);
  if (is_weighted_pooling(pp.pooling_type))
    NVE_CHECK_ARG(pp.weights != nullptr, "Sparse weights are required for weighted pooling");
  switch (pp.sparse_type) {
    case NVE_SPARSE_FIXED:
      NVE_CHECK_ARG(pp.fixed_hotness > 0, "Invalid fixed hotness");
      break;
    case NVE_SPARSE_CSR:
      NVE_CHECK_ARG(pp.csr_offsets != nullptr, "CSR offsets are required for pooling");
      NVE_CHECK_ARG(pp.num_csr_offsets >= 2, "CSR pooling requires at least two offsets");
      break;
    default:
      NVE_CHECK_ARG(false, "Unsupported sparse type ", pp.sparse_type);
  }
}

int64_t lookup_output_rows(int64_t num_keys, const PoolingParams* pp) {
  NVE_CHECK_ARG(num_keys >= 0, "Invalid number of keys");
  if (pp == nullptr || pp->pooling_type == NVE_POOL_CONCATENATE) return num_keys;
  if (pp->sparse_type == NVE_SPARSE_FIXED) {
    NVE_CHECK_ARG(pp->fixed_hotness > 0, "Invalid fixed hotness");
    NVE_CHECK_ARG(num_keys % pp->fixed_hotness == 0,
                  "Number of keys does not divide by fixed hotness");
    return num_keys / pp->fixed_hotness;
  }
  NVE_CHECK_ARG(pp->sparse_type == NVE_SPARSE_CSR, "Unsupported sparse type ", pp->sparse_type);
  NVE_CHECK_ARG(pp->csr_offsets != nullptr, "CSR offsets are required for pooling");
  NVE_CHECK_ARG(pp->num_csr_offsets >= 2, "CSR pooling requires at least two offsets");
  return pp->num_csr_offsets - 1;
}

// ---------------------------------------------------------------------------
// layer base: modify operations a layer does not support
// ---------------------------------------------------------------------------
void EmbeddingLayer::insert(ExecutionContext&, int64_t, const void*, int64_t, int64_t, const void*,
                            int64_t) {
  NVE_NOT_IMPLEMENTED("insert is not supported by this layer");
}
void EmbeddingLayer::update(ExecutionContext&, int64_t, const void*, int64_t, int64_t, const void*,
                            int64_t) {
  NVE_NOT_IMPLEMENTED("update is not supported by this layer");
}
void EmbeddingLayer::accumulate(ExecutionContext&, int64_t, const void*, int64_t, int64_t,
                                const void*, int, int64_t) {
  NVE_NOT_IMPLEMENTED("accumulate is not supported by this layer");
}
void EmbeddingLayer::clear(ExecutionContext&) {
  NVE_NOT_IMPLEMENTED("clear is not supported by this layer");
}
void EmbeddingLayer::erase(ExecutionContext&, int64_t, const void*, int64_t) {
  NVE_NOT_IMPLEMENTED("erase is not supported by this layer");
}

std::shared_ptr<ExecutionContext> EmbeddingLayer::create_execution_context(
    hipStream_t lookup, hipStream_t modify, std::shared_ptr<ThreadPool> pool) {
  auto ctx = std::make_shared<ExecutionContext>(device_, lookup, modify, std::move(pool));
  if (auto streams = lookup_streams()) ctx->watch(streams);
  return ctx;
}

// ---------------------------------------------------------------------------
// GPUEmbeddingLayer (gpu_embedding_layer.cu:296-499)
// ---------------------------------------------------------------------------
namespace {

// Value count of a quantized row (gpu_embedding_layer.cu:45-50).
int64_t quant_value_count(int dtype, int64_t width) {
  const int64_t meta = meta_bytes(dtype);
  NVE_CHECK(width > meta, "Quantized GPU embedding rows must contain values in addition to metadata");
  return (width - meta) / value_elem_bytes(dtype);
}

// Output types a rowwise row may be dequantized to: the metadata precision for
// the reference's types; f16 or f32 for this build's extension types.
bool quant_output_ok(int dtype, int out) {
  if (dtype == kXI8AF32 || dtype == kXE4M3F32) return out == kF32 || out == kF16;
  return out == native_out(dtype);
}

// gpu_embedding_layer.cu:57-90
void validate_quant_pool(int dtype, int64_t width, const PoolingParams& pp, int64_t stride) {
  NVE_CHECK_ARG(quant_output_ok(dtype, pp.output_type),
                "Quantized GPU embedding output type must match the quantization metadata precision");
  NVE_CHECK_ARG(stride == quant_value_count(dtype, width) * dtype_size(pp.output_type),
                "Invalid dequantized output stride for quantized GPU embedding table");
  if (pp.pooling_type == NVE_POOL_CONCATENATE) return;
  if (is_weighted_pooling(pp.pooling_type))
    NVE_CHECK_ARG(pp.weight_type == kF32 || pp.weight_type == kF16,
                  "Quantized GPU embedding weights must be Float32 or Float16");
}

}  // namespace

GPUEmbeddingLayer::GPUEmbeddingLayer(int key_bytes, const GPUEmbeddingLayerConfig& cfg)
    : EmbeddingLayer(key_bytes, cfg.device_id), cfg_(cfg) {
  NVE_CHECK(cfg_.embedding_table != nullptr, "Invalid embedding table");
  NVE_CHECK(cfg_.num_embeddings > 0, "Invalid number of embeddings");
  NVE_CHECK(cfg_.value_dtype == kF32 || cfg_.value_dtype == kF16 || is_rowwise(cfg_.value_dtype),
            "Unsupported GPU embedding table value type");
  NVE_CHECK(cfg_.embedding_width_in_bytes > 0, "Invalid embedding width");
  if (is_rowwise(cfg_.value_dtype)) {
    NVE_CHECK(cfg_.embedding_width_in_bytes % 2 == 0, "Quantized GPU embedding row width must be even");
    (void)quant_value_count(cfg_.value_dtype, cfg_.embedding_width_in_bytes);
  } else {
    NVE_CHECK(cfg_.embedding_width_in_bytes % dtype_size(cfg_.value_dtype) == 0,
              "Embedding width must be a whole number of elements");
  }
  const uint64_t kmax = key_bytes == 4 ? (uint64_t)INT32_MAX : (uint64_t)INT64_MAX;
  NVE_CHECK((uint64_t)cfg_.num_embeddings <= kmax,
            "Number of embeddings cannot be represented by the layer key type");
  NVE_CHECK(cfg_.default_row_index < cfg_.num_embeddings,
            "Default row index must be less than num_embeddings");
}

void GPUEmbeddingLayer::lookup(ExecutionContext& ctx, int64_t num_keys, const void* keys,
                               void* output, int64_t output_stride, uint64_t* hitmask,
                               const PoolingParams* pp, float* hitrates) {
  ScopedDevice sd(cfg_.device_id);
  NVE_CHECK_ARG(num_keys >= 0, "Invalid num_keys");
  NVE_CHECK_ARG(keys != nullptr, "Invalid keys buffer");
  NVE_CHECK_ARG(output != nullptr, "Invalid output buffer");
  NVE_CHECK_ARG(hitmask == nullptr, "Hitmask is not supported for GPU embedding layer");
  NVE_CHECK_ARG(num_keys <= INT_MAX, "Number of keys exceeding max int value is not supported");

  const int vdt = cfg_.value_dtype;
  const int64_t width = cfg_.embedding_width_in_bytes;
  const bool quant = is_rowwise(vdt);
  const bool concat = pp && pp->pooling_type == NVE_POOL_CONCATENATE;
  const bool raw_concat = concat && pp->output_type == vdt;
  if (pp) {
    validate_pool_params(*pp);
    if (raw_concat) {
      NVE_CHECK_ARG(output_stride == width,
                    "Raw Concatenate output stride must be the same as the stored row width");
    } else if (quant) {
      validate_quant_pool(vdt, width, *pp, output_stride);
    } else {
      NVE_CHECK_ARG(output_stride == width, "Output stride must be the same as embedding width");
      NVE_CHECK_ARG(pp->output_type == vdt,
                    "GPU embedding layer requires pooled output type to match the table value type");
      if (!concat && pp->weights != nullptr)
        NVE_CHECK_ARG(pp->weight_type == vdt,
                      "GPU embedding layer requires weight type to match the table value type");
    }
  } else {
    NVE_CHECK_ARG(output_stride == width, "Output stride must be the same as embedding width");
  }

  const hipStream_t stream = ctx.lookup_stream();
  const int64_t out_rows = lookup_output_rows(num_keys, pp);
  const size_t out_bytes = (size_t)out_rows * (size_t)output_stride;
  const void* d_keys = device_input(ctx, "keys", keys, (size_t)num_keys * key_bytes_, stream);
  if (cfg_.default_row_index >= 0 && num_keys > 0) {
    void* s = ctx.buffer("sanitized_keys", (size_t)num_keys * key_bytes_);
    NVE_HIP(launch_sanitize(d_keys, s, num_keys, key_bytes_, (uint64_t)cfg_.num_embeddings,
                            cfg_.default_row_index, stream));
    d_keys = s;
  }
  void* d_out = device_output(ctx, "output", output, out_bytes);

  RowSource src{};
  src.table = static_cast<const uint8_t*>(cfg_.embedding_table);
  src.row_bytes = (uint64_t)width;
  src.load_indices = 1;
  // keys outside the table (no default row configured) read nothing: the
  // gather leaves their output rows alone and pooling adds a zero row
  src.num_rows = (uint64_t)cfg_.num_embeddings;

  {
    std::lock_guard<std::mutex> lk(launch_mu_);
    if (!pp || raw_concat) {
      GatherLaunch g{};
      g.keys = d_keys;
      g.key_bytes = key_bytes_;
      g.n = num_keys;
      g.src = src;
      g.stored_dtype = vdt;
      g.raw = 1;
      g.out = d_out;
      g.out_stride = output_stride;
      NVE_HIP(launch_gather(g, stream));
    } else if (concat) {
      // rowwise rows dequantized per key (find_and_dequant)
      GatherLaunch g{};
      g.keys = d_keys;
      g.key_bytes = key_bytes_;
      g.n = num_keys;
      g.src = src;
      g.stored_dtype = vdt;
      g.count = quant_value_count(vdt, width);
      g.raw = 0;
      g.out = d_out;
      g.out_stride = output_stride;
      g.out_dtype = pp->output_type;
      NVE_HIP(launch_gather(g, stream));
    } else {
      PoolLaunch p{};
      p.keys = d_keys;
      p.key_bytes = key_bytes_;
      p.num_keys = num_keys;
      if (pp->sparse_type == NVE_SPARSE_CSR) {
        p.offsets = device_input(ctx, "offsets", pp->csr_offsets,
                                 (size_t)pp->num_csr_offsets * key_bytes_, stream);
        p.num_bags = pp->num_csr_offsets - 1;
      } else {
        p.hotness = pp->fixed_hotness;
        p.num_bags = num_keys / pp->fixed_hotness;
      }
      p.weighted = is_weighted_pooling(pp->pooling_type);
      p.mean = is_mean_pooling(pp->pooling_type);
      if (p.weighted) {
        NVE_CHECK_ARG(pp->weight_type == kF32 || pp->weight_type == kF16,
                      "Unsupported weight type ", pp->weight_type);
        p.weights = device_input(ctx, "weights", pp->weights,
                                 (size_t)num_keys * dtype_size(pp->weight_type), stream);
        p.weight_dtype = pp->weight_type;
      }
      p.src = src;
      p.stored_dtype = vdt;
      p.count = quant ? quant_value_count(vdt, width) : width / dtype_size(vdt);
      p.out = d_out;
      p.out_stride = output_stride;
      p.out_dtype = pp->output_type;
      NVE_HIP(launch_pool(p, stream));
    }
  }
  finish_output(output, d_out, out_bytes, stream);
  if (hitrates) hitrates[0] = 1.0f;
}

// ---------------------------------------------------------------------------
// insert heuristics
// ---------------------------------------------------------------------------
DefaultInsertHeuristic::DefaultInsertHeuristic(std::vector<float> thresholds)
    : thresholds_(std::move(thresholds)), gen_(98437598437ULL), dis_(0.0, 1.0) {}

bool DefaultInsertHeuristic::insert_needed(float hitrate, size_t table_id) {
  std::lock_guard<std::mutex> lk(mu_);
  NVE_CHECK(table_id < thresholds_.size(), "Invalid table index");
  const float warm = 1.0f - hitrate;
  const float steady = warm * warm * warm;
  return hitrate < thresholds_[table_id] ? dis_(gen_) < warm : dis_(gen_) < steady;
}

}  // namespace nve_amd

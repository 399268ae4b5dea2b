"""pynve.torch: torch modules and custom ops over the HIP lookup library.

The two ops of the reference's torch library (torch_binding.cpp:85-92) are
defined here with the same schemas and implemented for HIP tensors (torch's
"CUDA" dispatch key on ROCm) and for host tensors ("CPU": host layers):

    nve_ops::embedding_lookup(Tensor marker, Tensor keys, int embedding_size,
                              int dtype) -> Tensor
    nve_ops::embedding_lookup_with_pooling(Tensor marker, Tensor keys,
        Tensor offsets, Tensor? weights, int pooling_type, int embedding_size,
        int dtype) -> Tensor

The layer is found through the marker tensor's data_ptr in the binding
registry (nve_registry.cu:25-50).  Shape inference (the fake kernels) uses
only the baked `embedding_size` and `dtype` arguments, as the reference's
pynve/torch/__init__.py does.
"""
import torch

from .. import nve

HAS_TORCH_OPS = True

_DEF = torch.library.Library("nve_ops", "DEF")
_DEF.define("embedding_lookup(Tensor marker, Tensor keys, int embedding_size, int dtype) -> Tensor")
_DEF.define("embedding_lookup_with_pooling(Tensor marker, Tensor keys, Tensor offsets, "
            "Tensor? weights, int pooling_type, int embedding_size, int dtype) -> Tensor")


def _out_dtype(dtype_tag):
    t = nve.DataType_t(dtype_tag)
    if t == nve.DataType_t.Float32:
        return torch.float32
    if t == nve.DataType_t.Float16:
        return torch.float16
    raise ValueError(f"Invalid data type: {t}")


def _check_index_tensor(t, name):
    # nve_torch_ops_checks.hpp:27-45
    if t.dtype != torch.int64:
        raise RuntimeError(f"nve-torch-ops: {name} must be an int64 tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"nve-torch-ops: {name} must be contiguous")


def _check_pooling_weights(w, num_keys):
    if not w.is_contiguous():
        raise RuntimeError("nve-torch-ops: weights must be contiguous")
    if w.numel() != num_keys:
        raise RuntimeError("nve-torch-ops: weights must have one element per key")
    if w.dtype == torch.float32:
        return int(nve.DataType_t.Float32)
    if w.dtype == torch.float16:
        return int(nve.DataType_t.Float16)
    raise RuntimeError("nve-torch-ops: weights must be a float32 or float16 tensor")


def _stream_for(t):
    """The stream a lookup on tensor t's device runs on (0 for host tensors:
    a host layer runs on the calling threads)."""
    return torch.cuda.current_stream(t.device).cuda_stream if t.is_cuda else 0


def _embedding_lookup_impl(marker, keys, embedding_size, dtype):
    """nve_torch_ops.cu:67-98 / nve_torch_ops_cpu.cpp:59-90: [num_keys, dim]
    rows of the layer's dtype, on the keys' device."""
    _check_index_tensor(keys, "keys")
    binding = nve.get_binding(marker.data_ptr())
    n = keys.numel()
    out = torch.empty((n, binding.get_embedding_dim()), dtype=_out_dtype(int(binding.get_data_type())),
                      device=keys.device)
    binding.lookup(n, keys.data_ptr(), out.data_ptr(), _stream_for(keys))
    return out


def _embedding_lookup_with_pooling_impl(marker, keys, offsets, weights, pooling_type,
                                        embedding_size, dtype):
    """nve_torch_ops.cu:100-146 / nve_torch_ops_cpu.cpp:92-133: [num_bags, dim]
    pooled rows, CSR offsets with num_bags + 1 entries."""
    _check_index_tensor(keys, "keys")
    _check_index_tensor(offsets, "offsets")
    if offsets.numel() < 2:
        raise RuntimeError("nve-torch-ops: offsets must have at least two entries "
                           "(num_bags + 1, include_last_offset=True convention)")
    binding = nve.get_binding(marker.data_ptr())
    num_bags = offsets.numel() - 1
    out = torch.empty((num_bags, binding.get_embedding_dim()),
                      dtype=_out_dtype(int(binding.get_data_type())), device=keys.device)
    wdt, wptr = int(nve.DataType_t.Unknown), 0
    if weights is not None:
        wdt = _check_pooling_weights(weights, keys.numel())
        wptr = weights.data_ptr()
    binding.lookup_with_pooling(keys.numel(), keys.data_ptr(), out.data_ptr(), int(pooling_type),
                                offsets.numel(), offsets.data_ptr(), wdt, wptr, _stream_for(keys))
    return out


# one implementation for both dispatch keys: the binding of the marker decides
# where the lookup runs (HIP kernels, or CPU threads for a host layer), and
# buffers on the other side are staged by the layer
for _key in ("CUDA", "CPU"):
    _DEF.impl("embedding_lookup", _embedding_lookup_impl, _key)
    _DEF.impl("embedding_lookup_with_pooling", _embedding_lookup_with_pooling_impl, _key)


@torch.library.register_fake("nve_ops::embedding_lookup")
def _embedding_lookup_fake(marker, keys, embedding_size, dtype):
    return keys.new_empty((keys.size(0), embedding_size), dtype=_out_dtype(dtype))


@torch.library.register_fake("nve_ops::embedding_lookup_with_pooling")
def _embedding_lookup_with_pooling_fake(marker, keys, offsets, weights, pooling_type,
                                        embedding_size, dtype):
    torch._check(offsets.size(0) >= 2,
                 lambda: "offsets must have at least two entries (num_bags + 1, "
                         "include_last_offset=True convention)")
    return offsets.new_empty((offsets.size(0) - 1, embedding_size), dtype=_out_dtype(dtype))

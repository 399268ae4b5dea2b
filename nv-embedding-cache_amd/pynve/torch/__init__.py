"""pynve.torch: torch modules and custom ops over the HIP lookup library.

The two ops of the reference's torch library (torch_binding.cpp:85-92) are
defined and implemented natively, in libnve_torch_ops.so (built beside
libnve_amd.so from csrc/torch_ops/nve_torch_ops.cpp), for HIP tensors (torch's
"CUDA" dispatch key on ROCm) and host tensors ("CPU": host layers):

    nve_ops::embedding_lookup(Tensor marker, Tensor keys, int embedding_size,
                              int dtype) -> Tensor
    nve_ops::embedding_lookup_with_pooling(Tensor marker, Tensor keys,
        Tensor offsets, Tensor? weights, int pooling_type, int embedding_size,
        int dtype) -> Tensor

Each call goes from the dispatcher straight to the C ABI, with no Python on
the way.  The layer is found through the marker tensor's data_ptr in the
library's registry (nve_registry.cu:25-50), which pynve.nve.register_for_torch
fills.  Shape inference (the fake kernels) uses only the baked
`embedding_size` and `dtype` arguments, as the reference's
pynve/torch/__init__.py does.
"""
import ctypes
import os

import torch

from .. import nve
from .._lib import LIB_PATH

HAS_TORCH_OPS = True

OPS_LIB_PATH = os.path.join(os.path.dirname(LIB_PATH), "libnve_torch_ops.so")


class _NativeOps:
    """ctypes view of the ops library's registry entry points."""

    def __init__(self, path):
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing: build the package (make -C nv-embedding-cache_amd) "
                              "before importing pynve.torch")
        torch.ops.load_library(path)  # registers nve_ops::* with the dispatcher
        lib = ctypes.CDLL(path)
        P, I32, I64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        self._register = lib.nve_torch_ops_register
        self._register.argtypes, self._register.restype = [P, P, I64, I32, P, I64], I32
        self._unregister = lib.nve_torch_ops_unregister
        self._unregister.argtypes, self._unregister.restype = [P], I32
        self._release = lib.nve_torch_ops_release_layer
        self._release.argtypes, self._release.restype = [P], I32
        self._num_contexts = lib.nve_torch_ops_num_contexts
        self._num_contexts.argtypes, self._num_contexts.restype = [P, ctypes.POINTER(I64)], I32

    def register(self, marker_ptr, binding):
        modify = binding._modify_stream.cuda_stream if binding._modify_stream is not None else 0
        dtype = int(binding.data_type_)
        if dtype not in (int(nve.DataType_t.Float32), int(nve.DataType_t.Float16)):
            raise ValueError(f"torch ops serve float32 and float16 layers, not {binding.data_type_!r}")
        rc = self._register(marker_ptr, binding._layer, binding.row_size_in_bytes_, dtype, modify,
                            binding.logging_interval_)
        if rc != 0:
            raise RuntimeError(f"nve_torch_ops_register refused marker {marker_ptr:#x}")

    def unregister(self, marker_ptr):
        self._unregister(marker_ptr)

    def release_layer(self, layer):
        self._release(layer)

    def num_contexts(self, marker_ptr):
        """Execution contexts the ops made for a marker's layer (one per stream)."""
        n = ctypes.c_int64()
        if self._num_contexts(marker_ptr, ctypes.byref(n)) != 0:
            raise RuntimeError(f"no binding registered for marker_ptr={marker_ptr:#x}")
        return n.value


nve._native_ops = _NativeOps(OPS_LIB_PATH)


def _out_dtype(dtype_tag):
    t = nve.DataType_t(dtype_tag)
    if t == nve.DataType_t.Float32:
        return torch.float32
    if t == nve.DataType_t.Float16:
        return torch.float16
    raise ValueError(f"Invalid data type: {t}")


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

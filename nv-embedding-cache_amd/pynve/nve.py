"""pynve.nve: layer bindings over the C ABI of libnve_amd.so.

Mirrors the reference's pybind11 module `pynve.nve`
(python/pynve/bindings/python_binding.cu:149-392, binding_layers.hpp:50-788):
the same class names, constructor arguments, method names and argument
meaning.  Keys are int64; every pointer argument is a raw address (an int),
streams are `hipStream_t` values (`torch.cuda.current_stream().cuda_stream`
on ROCm).  Lookups take one execution context per stream, created on first
use, as `NVEmbedBinding::get_exec_context` does (binding_layers.hpp:352-366).

Memory blocks: device memory comes from torch's allocator, host memory from
`hipHostMalloc` (pinned and mapped into the GPU's address space).  A
`ManagedMemBlock` (reference: cudaMallocManaged + preferred location host +
accessed-by the GPUs, memblock.cpp:111-134) is pinned host memory here: with
XNACK off, that is the memory the MI355X reads over the host link without
page faults, which is what the reference's advice arranges.

Table checkpoints (`TensorFileFormat`, `write_tensor_to_stream`,
`load_tensor_from_stream`) read and write the reference's .nve container.

Out of this build (raise NotImplementedInBuild): the HierarchicalEmbedding
layer, the parameter-server tables and the multi-process memory blocks
(NVL / MPI / Dist*).
"""
import ctypes
import json
import sys
import threading
from enum import IntEnum

from . import _lib


class DataType_t(IntEnum):
    """nve::DataType_t (nve_types.hpp:59-72), the ids the C ABI uses."""
    Unknown = 0
    Float32 = 1
    BFloat = 2
    Float16 = 3
    E4M3 = 4
    E5M2 = 5
    Float64 = 6


class PoolingType_t(IntEnum):
    """nve::PoolingType_t (python_binding.cu:204-210)."""
    Concatenate = 0
    Sum = 1
    Mean = 2
    WeightedSum = 3
    WeightedMean = 4


class MemBlockType(IntEnum):
    """nve::MemBlockType (memblock.hpp:29-36)."""
    Linear = 0
    NVL = 1
    MPI = 2
    Managed = 3
    User = 4
    Host = 5


_DTYPE_SIZE = {DataType_t.Float32: 4, DataType_t.BFloat: 2, DataType_t.Float16: 2,
               DataType_t.E4M3: 1, DataType_t.E5M2: 1, DataType_t.Float64: 8}


def dtype_size(dtype):
    """Bytes per element (nve_types.hpp dtype_size)."""
    try:
        return _DTYPE_SIZE[DataType_t(dtype)]
    except (KeyError, ValueError):
        raise _lib.InvalidArgument(_lib.INVALID_ARGUMENT, f"dtype {dtype!r} has no element size")


def _library_alive():
    """Whether libnve_amd.so is loaded and still reachable: at interpreter
    exit the module globals are cleared before the last objects are
    collected, and their handles are then left to the process's end."""
    return _lib is not None and getattr(_lib, "_lib", None) is not None


class EmbedLayerConfig:
    """Per-layer options (binding_layers.hpp:50-65); same fields and defaults."""

    _FIELDS = ("logging_interval", "kernel_mode", "kernel_mode_value_1", "kernel_mode_value_2",
               "max_modify_size", "default_row_index", "default_embedding")

    def __init__(self):
        self.logging_interval = -1
        self.kernel_mode = 0
        self.kernel_mode_value_1 = 0
        self.kernel_mode_value_2 = 0
        self.max_modify_size = 0
        self.default_row_index = -1
        self.default_embedding = []

    def to_json(self):
        return json.dumps({f: getattr(self, f) for f in self._FIELDS})


# ---------------------------------------------------------------------------
# memory blocks (memblock.hpp / memblock.cpp)
# ---------------------------------------------------------------------------

_hip = None


def _hip_lib():
    global _hip
    if _hip is None:
        h = ctypes.CDLL("libamdhip64.so")
        h.hipHostMalloc.restype = ctypes.c_int
        h.hipHostMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t, ctypes.c_uint]
        h.hipHostFree.restype = ctypes.c_int
        h.hipHostFree.argtypes = [ctypes.c_void_p]
        h.hipMemcpy.restype = ctypes.c_int
        h.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        h.hipDeviceSynchronize.restype = ctypes.c_int
        h.hipDeviceSynchronize.argtypes = []
        _hip = h
    return _hip


class MemBlock:
    """A block of memory a layer reads its rows from; the layer keeps a
    reference so the block outlives it (binding_layers.hpp:529-788)."""

    def __init__(self, kind, ptr, size):
        self._type = MemBlockType(kind)
        self._ptr = int(ptr)
        self._size = int(size)

    def get_ptr(self):
        return self._ptr

    def get_handle(self):
        return self._ptr

    def get_type(self):
        return self._type

    def get_size_in_bytes(self):
        return self._size

    def copy_from(self, src):
        """Copy a C-contiguous buffer (numpy array, bytes, ...) into the block,
        bounds-checked (python_binding.cu:235-261)."""
        mv = memoryview(src)
        if not mv.c_contiguous:
            raise _lib.InvalidArgument(_lib.INVALID_ARGUMENT,
                                       "copy_from: source buffer must be C-contiguous")
        nbytes = mv.nbytes
        if nbytes > self._size:
            raise IndexError(f"copy_from: source is {nbytes} bytes but memblock holds "
                             f"{self._size} bytes")
        if nbytes == 0:
            return
        import numpy as np
        src_bytes = np.frombuffer(mv.cast("B"), dtype=np.uint8)
        rc = _hip_lib().hipMemcpy(self._ptr, src_bytes.ctypes.data, nbytes, 4)  # hipMemcpyDefault
        if rc == 0:
            # from pageable memory the copy may still be in flight when hipMemcpy
            # returns; lookups on other streams must see the whole block
            rc = _hip_lib().hipDeviceSynchronize()
        if rc != 0:
            raise _lib.NVEError(_lib.HIP_ERROR, f"copy_from: hipMemcpy failed ({rc})")


class UserMemBlock(MemBlock):
    """Caller-owned memory (memblock.hpp UserMemBlock): nothing is freed."""

    def __init__(self, ptr, size):
        super().__init__(MemBlockType.User, ptr, size)


class _PinnedHost(MemBlock):
    def __init__(self, kind, size):
        p = ctypes.c_void_p()
        if size > 0:
            rc = _hip_lib().hipHostMalloc(ctypes.byref(p), size, 0)
            if rc != 0 or not p.value:
                raise _lib.NVEError(_lib.OUT_OF_MEMORY,
                                    f"hipHostMalloc of {size} bytes failed ({rc})")
        super().__init__(kind, p.value or 0, size)

    def __del__(self, _finalizing=sys.is_finalizing):
        if _finalizing():
            return
        if getattr(self, "_ptr", 0) and _hip is not None:
            _hip.hipHostFree(self._ptr)
            self._ptr = 0


class _PlainHost(MemBlock):
    """Ordinary (pageable) host memory, for a host layer on a machine without a
    GPU driver: the rows live in a numpy buffer this block owns."""

    def __init__(self, kind, size):
        import numpy as np
        self._buf = np.zeros(max(int(size), 1), dtype=np.uint8)
        super().__init__(kind, self._buf.ctypes.data, size)


class HostMemBlock(_PinnedHost):
    """Pinned host memory (memblock.cpp:93-105)."""

    def __init__(self, row_size, num_embeddings, dtype):
        super().__init__(MemBlockType.Host, int(row_size) * int(num_embeddings) * dtype_size(dtype))


class ManagedMemBlock(_PinnedHost):
    """Host-resident memory the GPUs read directly (memblock.cpp:111-134);
    pinned and GPU-mapped on this build (see the module docstring)."""

    def __init__(self, row_size, num_embeddings, dtype, gpu_ids=()):
        self.gpu_ids = list(gpu_ids)
        super().__init__(MemBlockType.Managed, int(row_size) * int(num_embeddings) * dtype_size(dtype))


class LinearMemBlock(MemBlock):
    """Device memory of `device_id`, or pinned host memory when it is negative
    (memblock.cpp:27-50)."""

    def __init__(self, row_size, num_embeddings, dtype, device_id=-1):
        size = int(row_size) * int(num_embeddings) * dtype_size(dtype)
        self.device_id = int(device_id)
        if self.device_id < 0:
            self._host = _PinnedHost(MemBlockType.Linear, size)
            super().__init__(MemBlockType.Linear, self._host.get_ptr(), size)
        else:
            import torch
            self._tensor = torch.empty(size, dtype=torch.uint8, device=f"cuda:{self.device_id}")
            super().__init__(MemBlockType.Linear, self._tensor.data_ptr(), size)


def resolve_memblock_devices(type, def_index, override=()):
    """GPU ids to rebuild a memory block with (memblock.cpp:144-165): `override`
    when given, else every GPU from def_index on for an NVL block, else
    [def_index]."""
    if len(override):
        return list(override)
    if MemBlockType(type) == MemBlockType.NVL:
        import torch
        n = torch.cuda.device_count()
        if not 0 <= int(def_index) < n:
            raise _lib.NVEError(_lib.RUNTIME, f"resolve_memblock_devices: def_index={def_index} "
                                f"out of range, system has {n} GPUs")
        return list(range(int(def_index), n))
    return [int(def_index)]


def _not_in_build(what):
    raise _lib.NotImplementedInBuild(_lib.NOT_IMPLEMENTED, f"{what} is not part of this build")


class NVLMemBlock(MemBlock):
    def __init__(self, *args, **kwargs):
        _not_in_build("NVLMemBlock (multi-GPU shared tables)")


class MPIMemBlock(MemBlock):
    def __init__(self, *args, **kwargs):
        _not_in_build("MPIMemBlock (multi-process shared tables)")


class Table:
    """Opaque table handle (python_binding.cu:194); only the parameter-server
    tables derive from it in the reference, and those are not in this build."""


# ---------------------------------------------------------------------------
# layer bindings (binding_layers.hpp)
# ---------------------------------------------------------------------------

_ELEM = {DataType_t.Float32: 4, DataType_t.Float16: 2}


class NVEmbedBinding:
    """Common surface of the layer bindings (binding_layers.hpp:67-408)."""

    def __init__(self, device_id, row_size, dtype, config):
        self.device_id_ = int(device_id)
        self.data_type_ = DataType_t(dtype)
        # binding_layers.hpp:306-307: 4-byte elements for Float32, 2 otherwise
        self.row_size_in_bytes_ = int(row_size) * (4 if self.data_type_ == DataType_t.Float32 else 2)
        self.logging_interval_ = int(config.logging_interval) if config is not None else -1
        self.logging_counter_ = 0
        self._layer = None
        self._contexts = {}
        self._ctx_mu = threading.Lock()
        self._modify_stream = None
        if self.device_id_ >= 0:
            import torch
            self._modify_stream = torch.cuda.Stream(device=self.device_id_)

    # accessors used by the torch ops (binding_layers.hpp:71-84)
    def get_embedding_dim(self):
        if self.data_type_ not in _ELEM:
            raise _lib.InvalidArgument(_lib.INVALID_ARGUMENT, "Invalid data type")
        return self.row_size_in_bytes_ // _ELEM[self.data_type_]

    def get_data_type(self):
        return self.data_type_

    def _ctx(self, stream):
        # one context per lookup stream; calls with no stream (host work) get
        # one per calling thread, as a context is not thread-safe
        stream = int(stream or 0)
        key = stream if stream else ("thread", threading.get_ident())
        with self._ctx_mu:
            ctx = self._contexts.get(key)
            if ctx is None:
                h = ctypes.c_void_p()
                modify = self._modify_stream.cuda_stream if self._modify_stream is not None else 0
                _lib.call("nve_layer_create_execution_context", self._layer, ctypes.byref(h),
                          ctypes.c_void_p(stream), ctypes.c_void_p(modify), None, None)
                ctx = self._contexts[key] = h.value
            return ctx

    def _log_hit_rates(self, hr):
        # every logging_interval-th lookup, at the library logger's perf level
        # (binding_layers.hpp:370-387)
        if self.logging_interval_ > 0:
            if self.logging_counter_ % self.logging_interval_ == 0:
                msg = "Hit rates: " + ", ".join(f"{v:g}" for v in hr)
                _lib.call("nve_amd_log_message", 30, msg.encode())
            self.logging_counter_ += 1

    def lookup(self, num_keys, keys, output, stream):
        """One output row per key (binding_layers.hpp:86-101)."""
        hr = (ctypes.c_float * 3)()
        ctx = self._ctx(stream)
        _lib.call("nve_layer_lookup", self._layer, ctx, int(num_keys), ctypes.c_void_p(keys),
                  ctypes.c_void_p(output), self.row_size_in_bytes_, None, hr)
        self._log_hit_rates(list(hr))

    def lookup_with_pooling(self, num_keys, keys, output, pooling_type, num_offsets, offsets,
                            weight_data_type, weights, stream):
        """CSR-pooled lookup, output in the table's dtype (binding_layers.hpp:103-129)."""
        hr = (ctypes.c_float * 3)()
        ctx = self._ctx(stream)
        _lib.call("nve_layer_lookup_pooled", self._layer, ctx, int(num_keys), ctypes.c_void_p(keys),
                  ctypes.c_void_p(output), self.row_size_in_bytes_, None, int(pooling_type),
                  _lib.SPARSE_CSR, ctypes.c_void_p(offsets), int(num_offsets), 0,
                  ctypes.c_void_p(weights), int(weight_data_type), int(self.data_type_), hr)
        self._log_hit_rates(list(hr))

    def insert(self, num_keys, keys, values, table_id, stream):
        ctx = self._ctx(stream)
        _lib.call("nve_layer_insert", self._layer, ctx, int(num_keys), ctypes.c_void_p(keys),
                  self.row_size_in_bytes_, self.row_size_in_bytes_, ctypes.c_void_p(values),
                  int(table_id))

    def update(self, num_keys, keys, updates, stream):
        ctx = self._ctx(stream)
        _lib.call("nve_layer_update", self._layer, ctx, int(num_keys), ctypes.c_void_p(keys),
                  self.row_size_in_bytes_, self.row_size_in_bytes_, ctypes.c_void_p(updates), -1)

    def accumulate(self, num_keys, keys, updates, stream):
        ctx = self._ctx(stream)
        _lib.call("nve_layer_accumulate", self._layer, ctx, int(num_keys), ctypes.c_void_p(keys),
                  self.row_size_in_bytes_, self.row_size_in_bytes_, ctypes.c_void_p(updates),
                  int(self.data_type_), -1)

    def clear(self, stream):
        _lib.call("nve_layer_clear", self._layer, self._ctx(stream))

    def erase(self, num_keys, keys, table_id, stream):
        _lib.call("nve_layer_erase", self._layer, self._ctx(stream), int(num_keys),
                  ctypes.c_void_p(keys), int(table_id))

    def _backprop(self, what, num_keys, keys, grads, unique_keys, output_grads, pooling_type,
                  num_bags, offsets, weight_type, weights, stream):
        if self.device_id_ < 0:
            raise _lib.InvalidArgument(
                _lib.INVALID_ARGUMENT,
                f"{what} is not supported on a host-only layer (device_id < 0). "
                "Gradient computation requires a GPU device; HostLayer is inference-only.")
        import torch
        dim = self.get_embedding_dim()
        need = ctypes.c_uint64()
        _lib.call("nve_amd_backprop_workspace_size", int(num_keys), int(num_bags), dim, ctypes.byref(need))
        ws = getattr(self, "_bp_ws", None)
        if ws is None or ws.numel() < need.value:
            ws = self._bp_ws = torch.empty(max(int(need.value), 1), dtype=torch.uint8,
                                           device=f"cuda:{self.device_id_}")
        nu = ctypes.c_int64()
        _lib.call("nve_amd_pooling_backprop", _lib.KEY_INT64, int(num_keys), ctypes.c_void_p(keys),
                  int(pooling_type), _lib.SPARSE_CSR, ctypes.c_void_p(offsets),
                  int(num_bags) + 1 if offsets else 0, 0, ctypes.c_void_p(weights), int(weight_type),
                  ctypes.c_void_p(grads), int(self.data_type_), dim, ctypes.c_void_p(unique_keys),
                  ctypes.c_void_p(output_grads), ctypes.byref(nu), ctypes.c_void_p(ws.data_ptr()),
                  need.value, ctypes.c_void_p(int(stream or 0)))
        return nu.value

    def concat_backprop(self, num_keys, keys, grads, unique_keys, output_grads, stream):
        """Sparse gradient of a per-key lookup (binding_layers.hpp:131-189): the
        unique keys ascending into unique_keys and, per unique key, the sum of
        the gradient rows of its positions into output_grads (the table's
        dtype); returns the number of unique keys."""
        return self._backprop("concat_backprop", num_keys, keys, grads, unique_keys, output_grads,
                              PoolingType_t.Concatenate, 0, 0, DataType_t.Unknown, 0, stream)

    def pooling_backprop(self, num_keys, keys, grads, unique_keys, output_grads, pooling_type,
                         num_offsets, offsets, data_type, weights, stream):
        """Sparse gradient of a CSR-pooled lookup (binding_layers.hpp:191-250):
        grads holds one row per bag (num_offsets bags, offsets of num_offsets + 1
        int64 entries); weights (weighted modes) are per key, of data_type or,
        when that is not a float type, of the table's dtype."""
        wt = DataType_t(data_type) if int(data_type) in (int(DataType_t.Float32),
                                                          int(DataType_t.Float16)) else self.data_type_
        return self._backprop("pooling_backprop", num_keys, keys, grads, unique_keys, output_grads,
                              pooling_type, num_offsets, offsets, wt if weights else DataType_t.Unknown,
                              weights, stream)

    def get_num_tables(self):
        out = ctypes.c_int64()
        _lib.call("nve_layer_get_num_tables", self._layer, ctypes.byref(out))
        return out.value

    def release_contexts(self):
        """Wait for and destroy every context (binding_layers.hpp:339-350),
        those the native torch ops made for this layer included."""
        if _native_ops is not None and self._layer is not None:
            _native_ops.release_layer(self._layer)
        with self._ctx_mu:
            for ctx in self._contexts.values():
                _lib.call("nve_context_wait", ctx)
                _lib.call("nve_context_destroy", ctx)
            self._contexts.clear()

    def _destroy(self):
        if getattr(self, "_layer", None) is None or not _library_alive():
            return
        try:
            self.release_contexts()
        finally:
            _lib._lib.nve_layer_destroy(self._layer)
            self._layer = None

    def __del__(self, _finalizing=sys.is_finalizing):
        # at interpreter exit the module's globals may already be gone: the
        # process's end releases the native handles then
        if not _finalizing():
            self._destroy()


class GPUEmbedding(NVEmbedBinding):
    """Linear table in GPU memory, no cache (binding_layers.hpp:660-728)."""

    def __init__(self, row_size, num_embeddings, dtype, mem_block, device_id, config=None):
        config = config if config is not None else EmbedLayerConfig()
        super().__init__(device_id, row_size, dtype, config)
        self.num_embeddings_ = int(num_embeddings)
        self.row_size_ = int(row_size)
        self.mem_block_ = mem_block
        cfg = _lib.load().nve_gpu_embedding_layer_config_default()
        cfg.layer_name = b"gpu_layer"
        cfg.device_id = self.device_id_
        cfg.embedding_table = mem_block.get_ptr()
        cfg.num_embeddings = self.num_embeddings_
        cfg.embedding_width_in_bytes = self.row_size_in_bytes_
        cfg.value_dtype = int(self.data_type_)
        cfg.default_row_index = int(config.default_row_index)
        h = ctypes.c_void_p()
        _lib.call("nve_gpu_embedding_layer_create", ctypes.byref(h), _lib.KEY_INT64,
                  ctypes.byref(cfg), None)
        self._layer = h.value


class LinearUVMEmbedding(NVEmbedBinding):
    """GPU cache in front of a host-resident linear table
    (binding_layers.hpp:529-657)."""

    def __init__(self, row_size, num_embeddings, dtype, mem_block, gpu_cache_size,
                 use_private_stream, device_id, config=None):
        config = config if config is not None else EmbedLayerConfig()
        super().__init__(device_id, row_size, dtype, config)
        self.num_embeddings_ = int(num_embeddings)
        self.mem_block_ = mem_block
        self.row_size_ = int(row_size)
        self._table = None
        self._private_stream = None
        cfg = _lib.load().nve_gpu_table_config_default()
        cfg.device_id = self.device_id_
        cfg.cache_size = int(gpu_cache_size)
        cfg.row_size_in_bytes = self.row_size_in_bytes_
        cfg.value_dtype = int(self.data_type_)
        cfg.count_misses = 1
        if config.max_modify_size > 0:
            cfg.max_modify_size = int(config.max_modify_size)
        if use_private_stream:
            import torch
            self._private_stream = torch.cuda.Stream(device=self.device_id_)
            cfg.private_stream = self._private_stream.cuda_stream
        cfg.uvm_table = mem_block.get_ptr()
        cfg.uvm_num_rows = self.num_embeddings_
        # lookup modes (binding_layers.hpp:565-576; KernelType, gpu_table.hpp:37-42):
        # 0 direct below 2^20 keys else SortGather, 1 direct, 2 SortGather
        # (value: tile size), 3 PipelineGather (value: pointer to
        # {task_size, num_aux_streams}, read when the table is created)
        cfg.kernel_mode_type = int(config.kernel_mode)
        if config.kernel_mode == 2:
            cfg.kernel_mode_value = int(config.kernel_mode_value_1) if config.kernel_mode_value_1 > 0 else 1024
        elif config.kernel_mode == 3:
            self._pipeline_params = (ctypes.c_uint64 * 2)(
                int(config.kernel_mode_value_1) if config.kernel_mode_value_1 > 0 else 1024,
                int(config.kernel_mode_value_2) if config.kernel_mode_value_2 > 0 else 16)
            cfg.kernel_mode_value = ctypes.addressof(self._pipeline_params)
        t = ctypes.c_void_p()
        _lib.call("nve_gpu_table_create", ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(cfg), None)
        self._table = t.value
        try:
            lcfg = _lib.load().nve_linear_uvm_layer_config_default()
            lcfg.layer_name = b"uvm_layer"
            lcfg.default_row_index = int(config.default_row_index)
            h = ctypes.c_void_p()
            _lib.call("nve_linear_uvm_layer_create", ctypes.byref(h), _lib.KEY_INT64,
                      ctypes.byref(lcfg), self._table, None)
            self._layer = h.value
        except Exception:
            _lib._lib.nve_table_destroy(self._table)
            self._table = None
            raise

    def get_table_tensor(self):
        """The backing table as a [num_embeddings, row_size] host tensor that
        shares the block's memory (the reference hands out a DLPack view,
        binding_layers.hpp:588-617)."""
        import torch
        tdt = torch.float32 if self.data_type_ == DataType_t.Float32 else torch.float16
        n = self.num_embeddings_ * self.row_size_
        if n == 0:
            return torch.empty((self.num_embeddings_, self.row_size_), dtype=tdt)
        buf = (ctypes.c_char * (n * tdt.itemsize)).from_address(self.mem_block_.get_ptr())
        t = torch.frombuffer(buf, dtype=tdt).view(self.num_embeddings_, self.row_size_)
        t._nve_owner = self  # keep the binding (and its memory block) alive
        return t

    def _destroy(self):
        try:
            super()._destroy()
        finally:
            if getattr(self, "_table", None) is not None and _library_alive():
                if self._private_stream is not None:
                    self._private_stream.synchronize()
                _lib._lib.nve_table_destroy(self._table)
                self._table = None


class HostEmbedding(NVEmbedBinding):
    """Host-only layer (binding_layers.hpp:730-789): a LinearHostTable over the
    memory block's rows and the host embedding layer on top of it.  Lookups,
    pooling and updates run on CPU threads inside libnve_amd.so; with host
    buffers (device_id < 0) nothing touches a GPU.  Inference only: the
    backprop entries raise."""

    def __init__(self, row_size, num_embeddings, dtype, mem_block, device_id=-1, config=None):
        config = config if config is not None else EmbedLayerConfig()
        super().__init__(device_id, row_size, dtype, config)
        self.num_embeddings_ = int(num_embeddings)
        self.row_size_ = int(row_size)
        self.mem_block_ = mem_block
        self._table = None
        L = _lib.load()
        tcfg = L.nve_host_table_config_default()
        tcfg.key_size = 8
        tcfg.max_value_size = self.row_size_in_bytes_
        tcfg.value_dtype = int(self.data_type_)
        t = ctypes.c_void_p()
        _lib.call("nve_amd_linear_host_table_create", ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(tcfg),
                  ctypes.c_void_p(mem_block.get_ptr()), self.num_embeddings_, 0)
        self._table = t.value
        try:
            lcfg = L.nve_host_embedding_layer_config_default()
            lcfg.layer_name = b"host_layer"
            default = bytes(bytearray(config.default_embedding))
            self._default_row = ctypes.create_string_buffer(default, len(default) or 1)
            if default:
                lcfg.default_embedding = ctypes.cast(self._default_row, ctypes.c_void_p)
                lcfg.default_embedding_size = len(default)
            h = ctypes.c_void_p()
            _lib.call("nve_host_embedding_layer_create", ctypes.byref(h), _lib.KEY_INT64, ctypes.byref(lcfg),
                      self._table, None)
            self._layer = h.value
        except Exception:
            _lib._lib.nve_table_destroy(self._table)
            self._table = None
            raise

    def _destroy(self):
        try:
            super()._destroy()
        finally:
            if getattr(self, "_table", None) is not None and _library_alive():
                _lib._lib.nve_table_destroy(self._table)
                self._table = None


class HierarchicalEmbedding(NVEmbedBinding):
    def __init__(self, *args, **kwargs):
        _not_in_build("HierarchicalEmbedding (host / remote tiers)")


# ---------------------------------------------------------------------------
# table checkpoints: the .nve container (serialization.hpp:100-140,
# serialization.cpp:234-300) over a Python binary stream
# ---------------------------------------------------------------------------

class _PyStream:
    """A binary Python stream as the format reads and writes it
    (binding_serialization.cpp:22-70): `write` repeats until the stream has
    taken every byte, `read` repeats `readinto` until it returns 0."""

    def __init__(self, stream):
        self._s = stream

    def write(self, data):
        mv = memoryview(data).cast("B")
        done = 0
        while done < len(mv):
            n = self._s.write(mv[done:])
            done += len(mv) - done if n is None else int(n)

    def read_into(self, mv):
        mv = memoryview(mv).cast("B")
        total = 0
        while total < len(mv):
            n = self._s.readinto(mv[total:])
            if not n:
                break
            total += int(n)
        return total

    def seek(self, pos):
        return self._s.seek(int(pos))

    def tell(self):
        return int(self._s.tell())

    def size(self):
        cur = self._s.tell()
        end = self._s.seek(0, 2)
        self._s.seek(cur)
        return int(end)

    def flush(self):
        self._s.flush()


class TensorFileFormat:
    """The NVE table file (serialization.hpp:110-140): a 12-byte header
    {u32 magic 0x4E564500, u32 version major 0, u32 minor 2} at offset 0, then
    entries, each a 32-byte record {u64 key1, u64 name, u64 offset of the next
    record, u64 length} followed by `length` bytes of row-major table data.
    key1 packs the row width in elements (bits 0-15), the element size in bytes
    (bits 16-19) and the row count (bits 20-63).  All fields little-endian,
    the byte order the reference writes on x86 and aarch64 hosts."""

    MAGIC_NUMBER = 0x4E564500
    VERSION_MAJOR = 0
    VERSION_MINOR = 2
    ROW_SIZE_BITS = 16
    DATA_TYPE_BITS = 4
    ROWS_BITS = 64 - (ROW_SIZE_BITS + DATA_TYPE_BITS)
    HEADER_BYTES = 12
    ENTRY_BYTES = 32

    @staticmethod
    def _io(stream):
        return stream if isinstance(stream, _PyStream) else _PyStream(stream)

    def write_table_file_header(self, stream):
        """serialization.cpp:234-241: header at offset 0, then flush."""
        import struct
        s = self._io(stream)
        s.seek(0)
        s.write(struct.pack("<III", self.MAGIC_NUMBER, self.VERSION_MAJOR, self.VERSION_MINOR))
        s.flush()

    def verify_table_header(self, stream):
        """serialization.cpp:243-252: True when offset 0 holds this header;
        leaves the stream at the first entry."""
        import struct
        s = self._io(stream)
        s.seek(0)
        buf = bytearray(self.HEADER_BYTES)
        if s.read_into(buf) != self.HEADER_BYTES:
            return False
        return struct.unpack("<III", buf) == (self.MAGIC_NUMBER, self.VERSION_MAJOR,
                                               self.VERSION_MINOR)

    def make_key(self, rows, cols, element_size):
        """key1 of an entry, with the reference's limits (serialization.cpp:284-293)."""
        rows, cols, element_size = int(rows), int(cols), int(element_size)
        if not 0 <= cols < (1 << self.ROW_SIZE_BITS):
            raise _lib.NVEError(_lib.RUNTIME, "nve support max 16 bit row size")
        if not 0 <= rows < (1 << self.ROWS_BITS):
            raise _lib.NVEError(_lib.RUNTIME, "nve support max 44 bit rows")
        if not 0 <= element_size < (1 << self.DATA_TYPE_BITS):
            raise _lib.NVEError(_lib.RUNTIME, "nve support max 2 bit data type")
        return cols | (element_size << self.ROW_SIZE_BITS) | (rows << (self.ROW_SIZE_BITS +
                                                                      self.DATA_TYPE_BITS))

    def write_tensor_to_stream(self, stream, name, rows, cols, element_size, chunks):
        """Append one entry at the stream's position (serialization.cpp:254-264);
        `chunks` yields the rows*cols*element_size data bytes in order."""
        import struct
        s = self._io(stream)
        name = _u64_name(name)
        key1 = self.make_key(rows, cols, element_size)
        sz = int(rows) * int(cols) * int(element_size)
        s.write(struct.pack("<QQQQ", key1, name, sz + self.ENTRY_BYTES + s.tell(), sz))
        written = 0
        for c in chunks:
            s.write(c)
            written += memoryview(c).nbytes
        if written != sz:
            raise _lib.NVEError(_lib.RUNTIME, f"tensor source gave {written} of {sz} bytes")
        s.flush()

    def find_tensor(self, stream, name, rows, cols, element_size):
        """The search of load_tensor_from_stream (serialization.cpp:266-282):
        verify the header, then walk the entries from the first; on the entry
        named `name` check its length and return it with the stream at its data.
        Returns None when the stream ends first (no error, as in the reference)."""
        import struct
        s = self._io(stream)
        name = _u64_name(name)
        if not self.verify_table_header(s):
            raise _lib.NVEError(_lib.RUNTIME, "Incorrect file version")
        sz = int(rows) * int(cols) * int(element_size)
        rec = bytearray(self.ENTRY_BYTES)
        got = s.read_into(rec)
        while got != 0:
            if got != self.ENTRY_BYTES:
                raise _lib.NVEError(_lib.RUNTIME, "Problem reading table entry")
            key1, key2, offset, length = struct.unpack("<QQQQ", rec)
            if key2 == name:
                if length != sz:
                    raise _lib.NVEError(_lib.RUNTIME, "Incorrect tensor size")
                # a truncated entry fails here, before the destination is touched
                if s.tell() + length > s.size():
                    raise _lib.NVEError(_lib.RUNTIME, "Problem reading tensor")
                return (key1, key2, offset, length)
            s.seek(offset)
            got = s.read_into(rec)
        return None


def _u64_name(name):
    name = int(name)
    if not 0 <= name < (1 << 64):
        raise _lib.InvalidArgument(_lib.INVALID_ARGUMENT, f"tensor name {name} is not a uint64")
    return name


_STAGE_BYTES = 64 << 20


def _host_view(ptr, nbytes):
    return memoryview((ctypes.c_char * nbytes).from_address(ptr)).cast("B") if nbytes else memoryview(b"")


def _table_geometry(layer):
    """(rows, row width in elements, element size, base address) of the table a
    layer checkpoints: the backing table of a LinearUVMEmbedding (element size
    4 for Float32 tables, else 2: binding_layers.hpp:586-590) or the device
    table of a GPUEmbedding (dtype_size: binding_layers.hpp:677-680)."""
    if isinstance(layer, LinearUVMEmbedding):
        esize = 4 if layer.data_type_ == DataType_t.Float32 else 2
        return layer.num_embeddings_, layer.row_size_, esize, layer.mem_block_.get_ptr()
    if isinstance(layer, (GPUEmbedding, HostEmbedding)):
        return (layer.num_embeddings_, layer.row_size_, dtype_size(layer.data_type_),
                layer.mem_block_.get_ptr())
    raise TypeError("write_tensor_to_stream / load_tensor_from_stream take a LinearUVMEmbedding, "
                    f"a GPUEmbedding or a HostEmbedding, not {type(layer).__name__}")


def _device_chunks(layer, base, nbytes):
    """The GPU table's bytes in order, through a pinned staging buffer (bounded
    host memory, unlike the reference's one full-size copy)."""
    import torch
    torch.cuda.synchronize(layer.device_id_)  # pending lookups / updates land first
    stage = _PinnedHost(MemBlockType.Host, min(nbytes, _STAGE_BYTES))
    view = _host_view(stage.get_ptr(), stage.get_size_in_bytes())
    done = 0
    while done < nbytes:
        n = min(nbytes - done, _STAGE_BYTES)
        rc = _hip_lib().hipMemcpy(stage.get_ptr(), base + done, n, 4)
        if rc != 0:
            raise _lib.NVEError(_lib.HIP_ERROR, f"table read: hipMemcpy failed ({rc})")
        yield view[:n]
        done += n


def write_tensor_to_stream(layer, stream, name):
    """Append the layer's table to `stream` as one entry named `name`
    (python_binding.cu:83-99; binding_layers.hpp:626-630 and 693-703).  The
    stream must already hold the header (TensorFileFormat.write_table_file_header)."""
    rows, cols, esize, base = _table_geometry(layer)
    nbytes = rows * cols * esize
    fmt = TensorFileFormat()
    if isinstance(layer, (LinearUVMEmbedding, HostEmbedding)):  # host memory, written in place
        fmt.write_tensor_to_stream(stream, name, rows, cols, esize, [_host_view(base, nbytes)])
    else:
        fmt.write_tensor_to_stream(stream, name, rows, cols, esize, _device_chunks(layer, base, nbytes))


def load_tensor_from_stream(layer, stream, name):
    """Fill the layer's table from the entry named `name` of `stream`
    (python_binding.cu:89-105; binding_layers.hpp:632-636 and 705-716).

    Errors as in the reference: a wrong header, a short entry record or an entry
    of another size raise.  A stream without the name leaves a LinearUVMEmbedding's
    table as it was and zero-fills a GPUEmbedding's table (the reference copies
    its zero-initialised host buffer to the device either way).  Rows already in
    a LinearUVMEmbedding's GPU cache are not refreshed, as in the reference."""
    rows, cols, esize, base = _table_geometry(layer)
    nbytes = rows * cols * esize
    s = _PyStream(stream)
    found = TensorFileFormat().find_tensor(s, name, rows, cols, esize)
    if isinstance(layer, (LinearUVMEmbedding, HostEmbedding)):
        if found is not None and s.read_into(_host_view(base, nbytes)) != nbytes:
            raise _lib.NVEError(_lib.RUNTIME, "Problem reading tensor")
        return
    import torch
    torch.cuda.synchronize(layer.device_id_)
    stage = _PinnedHost(MemBlockType.Host, min(nbytes, _STAGE_BYTES))
    view = _host_view(stage.get_ptr(), stage.get_size_in_bytes())
    if found is None:
        ctypes.memset(stage.get_ptr(), 0, stage.get_size_in_bytes()) if nbytes else None
    done = 0
    while done < nbytes:
        n = min(nbytes - done, _STAGE_BYTES)
        if found is not None and s.read_into(view[:n]) != n:
            raise _lib.NVEError(_lib.RUNTIME, "Problem reading tensor")
        rc = _hip_lib().hipMemcpy(base + done, stage.get_ptr(), n, 4)
        if rc != 0:
            raise _lib.NVEError(_lib.HIP_ERROR, f"table write: hipMemcpy failed ({rc})")
        done += n


def get_dl_tensor(layer, dtype=None):
    """View of a LinearUVMEmbedding's backing table (python_binding.cu:65-81);
    a torch tensor, which `torch.utils.dlpack.from_dlpack` accepts as is."""
    if not isinstance(layer, LinearUVMEmbedding):
        raise _lib.InvalidArgument(_lib.INVALID_ARGUMENT, "get_dl_tensor takes a LinearUVMEmbedding")
    return layer.get_table_tensor()


# ---------------------------------------------------------------------------
# marker-tensor registry of the torch ops (nve_registry.cu:25-50)
# ---------------------------------------------------------------------------

_registry = {}
_registry_mu = threading.Lock()
# the native ops library's own registry (marker -> layer handle, contexts per
# stream); pynve.torch installs it when it loads that library
_native_ops = None


def register_for_torch(marker_ptr, binding):
    with _registry_mu:
        _registry[int(marker_ptr)] = binding
    if _native_ops is not None and getattr(binding, "_layer", None) is not None:
        _native_ops.register(int(marker_ptr), binding)


def unregister_from_torch(marker_ptr):
    with _registry_mu:
        _registry.pop(int(marker_ptr), None)
    if _native_ops is not None:
        _native_ops.unregister(int(marker_ptr))


def get_binding(marker_ptr):
    with _registry_mu:
        b = _registry.get(int(marker_ptr))
    if b is None:
        raise RuntimeError(f"NVELayerRegistry: no binding registered for marker_ptr={int(marker_ptr):#x}")
    return b

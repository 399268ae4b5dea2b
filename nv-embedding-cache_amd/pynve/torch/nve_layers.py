"""torch modules over the NVE layer bindings.

Interface kept from the reference's python/pynve/torch/nve_layers.py:110-556:
`LayerType` (same member values), `NVEmbedding` (torch.nn.Embedding over a
layer) and `NVEmbeddingBag` (torch.nn.EmbeddingBag with
include_last_offset=True: 'sum', 'mean' and 'concat'), their constructor
arguments, the `weight` / `marker_tensor` / `emb_layer` attributes the export
path reads, and `config_to_nve_config`.

How a layer is made here: the constructor arguments are first folded into a
`_Plan`, which validates everything that can be validated without memory or a
device; then the builder registered for the layer type allocates the table's
storage and the binding.  Layer types:

  GPULayer   table in HBM (HIP kernels of libnve_amd.so)
  LinearUVM  8-way GPU cache over a host-resident table (HIP kernels)
  HostLayer  table in host memory, looked up by CPU threads of libnve_amd.so
             (inference only; device='cpu' needs no GPU at all)
  Hierarchical  not part of this build (NotImplementedInBuild)
"""
import builtins
import sys
from enum import Enum
from typing import Optional

import torch

from .. import _lib, nve
from . import HAS_TORCH_OPS
from . import nve_ops
from .nve_tensors import CachedTable

_TORCH_OF = {nve.DataType_t.Float32: torch.float32, nve.DataType_t.Float16: torch.float16}
_NVE_OF = {v: k for k, v in _TORCH_OF.items()}

# integer fields of nve.EmbedLayerConfig a config dict may set
_CONFIG_FIELDS = ("kernel_mode", "logging_interval", "kernel_mode_value_1", "kernel_mode_value_2",
                  "max_modify_size", "default_row_index")


def nve_type_to_torch_type(nve_type):
    if nve_type in _TORCH_OF:
        return _TORCH_OF[nve_type]
    raise ValueError(f"{nve_type!r} has no torch counterpart among the table dtypes (float32, float16)")


def torch_type_to_nve_type(torch_type):
    if torch_type in _NVE_OF:
        return _NVE_OF[torch_type]
    raise ValueError(f"{torch_type} is not a table dtype of this build (float32, float16)")


def config_to_nve_config(config):
    """A dict of layer options -> nve.EmbedLayerConfig.  `default_embedding` may
    be a tensor (its bytes are taken) or an iterable of byte values."""
    out = nve.EmbedLayerConfig()
    for field in _CONFIG_FIELDS:
        if config and field in config:
            setattr(out, field, config[field])
    if config and "default_embedding" in config:
        row = config["default_embedding"]
        if isinstance(row, torch.Tensor):
            row = row.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()
        out.default_embedding = [int(b) for b in row]
    return out


def _check_forward_inputs(keys, offsets=None, per_sample_weights=None):
    """Types and layout the binding relies on (it reads raw pointers).  Offset
    values are checked by the layer at lookup time, where reading them does
    not break tracing."""
    if keys.dtype != torch.int64:
        raise TypeError(f"keys: expected torch.int64, got {keys.dtype}")
    if not keys.is_contiguous():
        raise ValueError("keys: a contiguous tensor is required")
    if offsets is not None:
        if offsets.dtype != torch.int64:
            raise TypeError(f"offsets: expected torch.int64, got {offsets.dtype}")
        if not offsets.is_contiguous():
            raise ValueError("offsets: a contiguous tensor is required")
        if offsets.numel() < 2:
            raise ValueError(f"offsets: {offsets.numel()} entries given, a batch needs num_bags + 1 >= 2 "
                             "(the last entry is len(keys))")
    if per_sample_weights is not None:
        if per_sample_weights.dtype not in (torch.float32, torch.float16):
            raise TypeError(f"per_sample_weights: expected float32 or float16, got {per_sample_weights.dtype}")
        if not per_sample_weights.is_contiguous():
            raise ValueError("per_sample_weights: a contiguous tensor is required")
        if per_sample_weights.numel() != keys.numel():
            raise ValueError(f"per_sample_weights: {per_sample_weights.numel()} values for "
                             f"{keys.numel()} keys (one per key is required)")


class LayerType(Enum):
    """Where a layer keeps its table (values as in the reference)."""
    GPULayer = 1
    LinearUVM = 2
    Hierarchical = 3
    HostLayer = 4


class _Plan:
    """Validated constructor arguments of a layer; nothing is allocated yet."""

    def __init__(self, num_embeddings, embedding_size, data_type, layer_type, gpu_cache_size,
                 host_cache_size, storage, weight_init, optimize_for_training, device, uid, config):
        if not isinstance(layer_type, LayerType):
            raise ValueError(f"layer_type must be a LayerType, got {layer_type!r}")
        self.layer_type = layer_type
        self.num_embeddings = int(num_embeddings)
        self.embedding_size = int(embedding_size)
        self.data_type = data_type
        self.nve_type = torch_type_to_nve_type(data_type)
        self.row_bytes = self.embedding_size * torch.empty(0, dtype=data_type).element_size()
        self.gpu_cache_size = gpu_cache_size
        self.host_cache_size = host_cache_size
        self.storage = storage
        self.weight_init = weight_init
        self.optimize_for_training = optimize_for_training
        self.uid = uid
        self.config = self._layer_config(config)
        self.device, self.device_index = self._placement(device)

    def _layer_config(self, config):
        row = config.get("default_embedding") if config else None
        if isinstance(row, torch.Tensor) and row.dtype != self.data_type:
            raise ValueError(f"default_embedding is {row.dtype}, the table holds {self.data_type}")
        cfg = config_to_nve_config(config)
        given = len(cfg.default_embedding)
        if given not in (0, self.row_bytes):
            raise ValueError(f"default_embedding has {given} bytes; one row of this table is "
                             f"{self.row_bytes} bytes ({self.embedding_size} x {self.data_type})")
        keeps_default = self.layer_type in (LayerType.HostLayer, LayerType.Hierarchical)
        if given and not keeps_default:
            raise ValueError(f"{self.layer_type.name} has no default embedding (a default row "
                             "index serves that purpose); only HostLayer and Hierarchical take one")
        if keeps_default and not given:
            cfg.default_embedding = [0] * self.row_bytes  # missed keys read zeros
        return cfg

    def _placement(self, device):
        dev = torch.device(device) if device is not None else torch.device("cuda")
        if dev.type == "cpu":
            if self.layer_type != LayerType.HostLayer:
                raise ValueError(f"a {self.layer_type.name} layer lives on a GPU; only HostLayer can be "
                                 "placed on device='cpu'")
            return dev, -1
        if dev.type != "cuda":
            raise ValueError(f"device {dev} is neither a GPU ('cuda') nor 'cpu'")
        return dev, dev.index if dev.index is not None else torch.cuda.current_device()


def _need_memblock_or_none(plan):
    if plan.storage is not None and not isinstance(plan.storage, nve.MemBlock):
        raise ValueError(f"storage of a {plan.layer_type.name} layer must be an nve.MemBlock (or None), "
                         f"got {type(plan.storage).__name__}")


def _build_gpu(plan):
    _need_memblock_or_none(plan)
    if plan.weight_init is not None:
        table = plan.weight_init.detach().clone().to(plan.device)
    else:
        table = torch.empty(plan.num_embeddings, plan.embedding_size, dtype=plan.data_type, device=plan.device)
    block = plan.storage or nve.UserMemBlock(table.data_ptr(), table.nbytes)
    binding = nve.GPUEmbedding(plan.embedding_size, plan.num_embeddings, plan.nve_type, block,
                               plan.device_index, plan.config)
    return binding, table, block, {0: "gpu"}


def _build_uvm(plan):
    if not plan.gpu_cache_size:
        raise ValueError("a LinearUVM layer needs gpu_cache_size > 0 (bytes of HBM for its cache)")
    _need_memblock_or_none(plan)
    block = plan.storage or nve.ManagedMemBlock(plan.embedding_size, plan.num_embeddings, plan.nve_type,
                                                [plan.device_index])
    binding = nve.LinearUVMEmbedding(plan.embedding_size, plan.num_embeddings, plan.nve_type, block,
                                     plan.gpu_cache_size, plan.optimize_for_training, plan.device_index,
                                     plan.config)
    table = torch.utils.dlpack.from_dlpack(nve.get_dl_tensor(binding, plan.nve_type))
    if plan.weight_init is not None:
        table.copy_(plan.weight_init)
    return binding, table, block, {0: "gpu_cache"}


def _build_hierarchical(plan):
    raise _lib.NotImplementedInBuild(_lib.NOT_IMPLEMENTED, "Hierarchical layers (host cache and remote "
                                     "parameter-server tiers) are not part of this build")


def _build_host(plan):
    if plan.optimize_for_training:
        raise ValueError("a HostLayer cannot be trained (its gradient would need a GPU): pass "
                         "optimize_for_training=False")
    _need_memblock_or_none(plan)
    if plan.storage is not None:
        if plan.storage.get_type() in (nve.MemBlockType.NVL, nve.MemBlockType.MPI):
            raise ValueError(f"a HostLayer reads its rows on the host; a {plan.storage.get_type().name} "
                             "memory block is not host memory")
        block = plan.storage
        if plan.weight_init is not None:
            src = plan.weight_init.detach().to("cpu", plan.data_type).contiguous()
            block.copy_from(src.view(torch.uint8).numpy())
        # the rows live in the caller's block: the weight is a shape-only placeholder
        table = torch.sparse_coo_tensor(size=(plan.num_embeddings, plan.embedding_size),
                                        dtype=plan.data_type, device=plan.device)
    else:
        if plan.weight_init is not None:
            table = plan.weight_init.detach().to("cpu", plan.data_type).contiguous()
        else:
            table = torch.empty(plan.num_embeddings, plan.embedding_size, dtype=plan.data_type)
        if plan.device.type == "cuda":  # GPU keys and outputs stage through pinned rows faster
            table = table.pin_memory()
        block = nve.UserMemBlock(table.data_ptr(), table.nbytes)
    binding = nve.HostEmbedding(plan.embedding_size, plan.num_embeddings, plan.nve_type, block,
                                plan.device_index, plan.config)
    return binding, table, block, {0: "host"}


_BUILDERS = {LayerType.GPULayer: _build_gpu, LayerType.LinearUVM: _build_uvm,
             LayerType.Hierarchical: _build_hierarchical, LayerType.HostLayer: _build_host}


class NVEmbeddingBase(torch.nn.Module):
    """State shared by NVEmbedding and NVEmbeddingBag.

    Arguments: num_embeddings, embedding_size, data_type (torch.float32 /
    torch.float16), layer_type, and keyword-only gpu_cache_size (bytes of HBM,
    LinearUVM), host_cache_size (unused here), storage (an nve.MemBlock holding
    the rows), weight_init (initial rows), optimize_for_training (keep the
    backprop path; LinearUVM table work on a private stream), device, id (the
    checkpoint entry name; defaults to the module's id()) and config (a dict of
    EmbedLayerConfig fields)."""

    def __init__(self, num_embeddings: int, embedding_size: int, data_type: torch.dtype,
                 layer_type: LayerType, *, gpu_cache_size: int = 0, host_cache_size: int = 0,
                 storage=None, weight_init: Optional[torch.Tensor] = None,
                 optimize_for_training: bool = True, device: Optional[torch.device] = None,
                 id: Optional[int] = None, config: Optional[dict] = None):
        super().__init__()
        plan = _Plan(num_embeddings, embedding_size, data_type, layer_type, gpu_cache_size, host_cache_size,
                     storage, weight_init, optimize_for_training, device,
                     id if id is not None else builtins.id(self), config)
        binding, table, block, table_ids = _BUILDERS[plan.layer_type](plan)
        # attributes read by the export / checkpoint code and by users
        self.layer_type = plan.layer_type
        self.num_embeddings = plan.num_embeddings
        self.embedding_size = plan.embedding_size
        self.data_type = plan.data_type
        self.layer_data_type = plan.nve_type
        self.gpu_cache_size = plan.gpu_cache_size
        self.host_cache_size = plan.host_cache_size
        self.optimize_for_training = plan.optimize_for_training
        self.device = plan.device
        self.device_index = plan.device_index
        self.id = plan.uid
        self.config = plan.config
        self.emb_layer = binding
        self.storage = block
        self.memblock_type = block.get_type()
        self.table_ids = table_ids
        self.dtype_tag = int(plan.nve_type)
        self.weight = CachedTable(table, cache=binding)
        # identity of the layer for the ops: its data_ptr keys the binding
        # registry; a graph constant under torch.export, outside state_dict
        self.register_buffer("marker_tensor", torch.tensor([self.id], dtype=torch.int64, device=self.device),
                             persistent=False)
        if HAS_TORCH_OPS:
            nve.register_for_torch(self.marker_tensor.data_ptr(), binding)

    def __del__(self, _finalizing=sys.is_finalizing):
        if _finalizing():  # the registry goes with the process
            return
        marker = getattr(self, "_buffers", {}).get("marker_tensor")
        if HAS_TORCH_OPS and marker is not None:
            nve.unregister_from_torch(marker.data_ptr())

    def to(self, *args, **kwargs):
        """Moves what the layer owns besides its rows: the table (`weight`) stays
        where the binding reads it and the marker stays where it was registered."""
        device, dtype, non_blocking, _ = torch._C._nn._parse_to(*args, **kwargs)
        pinned = {"weight", "marker_tensor"}
        for name, t in list(self.named_parameters()) + list(self.named_buffers()):
            if name not in pinned:
                t.data = t.data.to(device, dtype or t.dtype, non_blocking)
        return self

    def _stream(self):
        return 0 if self.device.type == "cpu" else torch.cuda.current_stream(self.device).cuda_stream

    def update(self, keys: torch.Tensor, updates: torch.Tensor):
        """Overwrite the rows of `keys` (asynchronous on the current stream)."""
        self.emb_layer.update(keys.numel(), keys.data_ptr(), updates.data_ptr(), self._stream())

    def insert(self, keys: torch.Tensor, values: torch.Tensor, table_id: int):
        """Offer rows to table `table_id` of the layer (a cache may decline)."""
        self.emb_layer.insert(keys.numel(), keys.data_ptr(), values.data_ptr(), table_id, self._stream())

    def clear(self):
        self.emb_layer.clear(self._stream())

    def erase(self, keys: torch.Tensor, table_id: int):
        self.emb_layer.erase(keys.numel(), keys.data_ptr(), table_id, self._stream())

    def load_from_stream(self, stream):
        """Fill the table from the .nve entry named after this module's id."""
        nve.load_tensor_from_stream(self.emb_layer, stream, self.id)

    # -- lookups --------------------------------------------------------------
    def _rows(self, keys):
        if self.optimize_for_training:
            return nve_ops.NVEmbeddingOpTraining.apply(self.marker_tensor, keys, self.weight,
                                                       self.embedding_size, self.dtype_tag)
        # an inference layer's op takes no weight, so its output has no autograd
        # history: call the op itself and spare the autograd.Function's cost
        return torch.ops.nve_ops.embedding_lookup(self.marker_tensor, keys, self.embedding_size, self.dtype_tag)

    def _bags(self, keys, offsets, per_sample_weights, pooling_type):
        if self.optimize_for_training:
            return nve_ops.NVEmbeddingBagOpTraining.apply(self.marker_tensor, keys, self.weight, offsets,
                                                          per_sample_weights, pooling_type,
                                                          self.embedding_size, self.dtype_tag)
        return torch.ops.nve_ops.embedding_lookup_with_pooling(self.marker_tensor, keys, offsets,
                                                               per_sample_weights, pooling_type,
                                                               self.embedding_size, self.dtype_tag)


class NVEmbedding(NVEmbeddingBase):
    """torch.nn.Embedding over an NVE layer: one row per key."""

    def __init__(self, num_embeddings: int, embedding_size: int, data_type: torch.dtype,
                 layer_type: LayerType, *, gpu_cache_size: int = 0, host_cache_size: int = 0,
                 storage=None, weight_init: Optional[torch.Tensor] = None,
                 optimize_for_training: bool = True, device: Optional[torch.device] = None,
                 id: Optional[int] = None, config: Optional[dict] = None):
        super().__init__(num_embeddings, embedding_size, data_type, layer_type, gpu_cache_size=gpu_cache_size,
                         host_cache_size=host_cache_size, storage=storage, weight_init=weight_init,
                         optimize_for_training=optimize_for_training, device=device, id=id, config=config)

    def forward(self, keys: torch.Tensor):
        _check_forward_inputs(keys)
        return self._rows(keys)


class NVEmbeddingBag(NVEmbeddingBase):
    """torch.nn.EmbeddingBag over an NVE layer, offsets in the
    include_last_offset=True convention (num_bags + 1 entries ending at
    len(input)).  mode 'sum' or 'mean' pools each bag (weighted when
    per_sample_weights are given); 'concat' returns one row per key."""

    def __init__(self, num_embeddings: int, embedding_size: int, data_type: torch.dtype,
                 layer_type: LayerType, mode: str, *, gpu_cache_size: int = 0,
                 host_cache_size: int = 0, storage=None,
                 weight_init: Optional[torch.Tensor] = None, optimize_for_training: bool = True,
                 device: Optional[torch.device] = None, id: Optional[int] = None,
                 config: Optional[dict] = None):
        if mode != "concat":
            nve_ops.pooling_type_from_mode(mode, False)  # reject before any allocation
        super().__init__(num_embeddings, embedding_size, data_type, layer_type, gpu_cache_size=gpu_cache_size,
                         host_cache_size=host_cache_size, storage=storage, weight_init=weight_init,
                         optimize_for_training=optimize_for_training, device=device, id=id, config=config)
        self.mode = mode

    def forward(self, input: torch.Tensor, offsets: torch.Tensor,
                per_sample_weights: Optional[torch.Tensor] = None):
        _check_forward_inputs(input, offsets, per_sample_weights)
        if self.mode == "concat":
            return self._rows(input)
        pooling = int(nve_ops.pooling_type_from_mode(self.mode, per_sample_weights is not None))
        return self._bags(input, offsets, per_sample_weights, pooling)

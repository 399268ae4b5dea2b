"""torch modules over the NVE layer bindings (python/pynve/torch/nve_layers.py).

`NVEmbedding` (like torch.nn.Embedding) and `NVEmbeddingBag` (like
torch.nn.EmbeddingBag with include_last_offset=True) with the reference's
constructor arguments, validation and forward routing.  The GPU layer
(`LayerType.GPULayer`: table in HBM) and the cached layer
(`LayerType.LinearUVM`: 8-way GPU cache over a host-resident table) run on the
HIP kernels of libnve_amd.so; the host and hierarchical layers are not part of
this build and raise NotImplementedInBuild when constructed.
"""
import builtins
from enum import Enum
from typing import Optional

import torch

from .. import nve
from . import HAS_TORCH_OPS
from . import nve_ops
from .nve_tensors import CachedTable


def nve_type_to_torch_type(nve_type):
    if nve_type == nve.DataType_t.Float32:
        return torch.float32
    if nve_type == nve.DataType_t.Float16:
        return torch.float16
    raise ValueError(f"Invalid data type: {nve_type}")


def torch_type_to_nve_type(torch_type):
    if torch_type == torch.float32:
        return nve.DataType_t.Float32
    if torch_type == torch.float16:
        return nve.DataType_t.Float16
    raise ValueError(f"Invalid data type: {torch_type}")


def _check_forward_inputs(keys, offsets=None, per_sample_weights=None):
    """dtype / contiguity checks before the raw data_ptr handoff
    (nve_layers.py:42-71).  Offset values are checked by the layer."""
    if keys.dtype != torch.int64:
        raise TypeError(f"keys must be an int64 tensor, got {keys.dtype}")
    if not keys.is_contiguous():
        raise ValueError("keys must be contiguous")
    if offsets is not None:
        if offsets.dtype != torch.int64:
            raise TypeError(f"offsets must be an int64 tensor, got {offsets.dtype}")
        if not offsets.is_contiguous():
            raise ValueError("offsets must be contiguous")
        if offsets.numel() < 2:
            raise ValueError("offsets must have at least two entries (num_bags + 1, "
                             "include_last_offset=True convention)")
    if per_sample_weights is not None:
        if per_sample_weights.dtype not in (torch.float32, torch.float16):
            raise TypeError(f"per_sample_weights must be a float32 or float16 tensor, "
                            f"got {per_sample_weights.dtype}")
        if not per_sample_weights.is_contiguous():
            raise ValueError("per_sample_weights must be contiguous")
        if per_sample_weights.numel() != keys.numel():
            raise ValueError(f"per_sample_weights must have one element per key: "
                             f"got {per_sample_weights.numel()} weights for {keys.numel()} keys")


def _current_stream_handle(device):
    if device.type == "cpu":
        return 0
    return torch.cuda.current_stream(device).cuda_stream


def config_to_nve_config(config):
    """dict -> nve.EmbedLayerConfig (nve_layers.py:84-108)."""
    embed_config = nve.EmbedLayerConfig()
    if config is None:
        return embed_config
    for f in ("kernel_mode", "logging_interval", "kernel_mode_value_1", "kernel_mode_value_2",
              "max_modify_size", "default_row_index"):
        if f in config:
            setattr(embed_config, f, config[f])
    if "default_embedding" in config:
        value = config["default_embedding"]
        if isinstance(value, torch.Tensor):
            value = value.detach().to("cpu").contiguous().view(torch.uint8).numpy().tobytes()
        embed_config.default_embedding = list(value)
    return embed_config


class LayerType(Enum):
    """Layer implementations (nve_layers.py:110-122)."""
    GPULayer = 1
    LinearUVM = 2
    Hierarchical = 3
    HostLayer = 4


class NVEmbeddingBase(torch.nn.Module):
    """Common constructor of NVEmbedding / NVEmbeddingBag (nve_layers.py:124-383).

    Args follow the reference: num_embeddings, embedding_size, data_type
    (torch.float32 / torch.float16), layer_type, and keyword-only
    gpu_cache_size (bytes, LinearUVM), host_cache_size, storage (an
    nve.MemBlock), weight_init, optimize_for_training (LinearUVM: the table
    work runs on a private stream), device, id, config (dict of
    EmbedLayerConfig fields).
    """

    def __init__(self, num_embeddings: int, embedding_size: int, data_type: torch.dtype,
                 layer_type: LayerType, *, gpu_cache_size: int = 0, host_cache_size: int = 0,
                 storage=None, weight_init: Optional[torch.Tensor] = None,
                 optimize_for_training: bool = True, device: Optional[torch.device] = None,
                 id: Optional[int] = None, config: Optional[dict] = None):
        super().__init__()
        if (config is not None and isinstance(config.get("default_embedding"), torch.Tensor)
                and config["default_embedding"].dtype != data_type):
            raise ValueError(f"config['default_embedding'] dtype {config['default_embedding'].dtype} "
                             f"does not match layer data_type {data_type}")
        self.config = config_to_nve_config(config)
        self.layer_type = layer_type
        self.num_embeddings = num_embeddings
        self.embedding_size = embedding_size
        self.data_type = data_type
        self.layer_data_type = torch_type_to_nve_type(data_type)
        row_bytes = embedding_size * torch.empty(0, dtype=data_type).element_size()
        if len(self.config.default_embedding) not in (0, row_bytes):
            raise ValueError(f"config['default_embedding'] must hold one row ({embedding_size} "
                             f"elements of {data_type} = {row_bytes} bytes), got "
                             f"{len(self.config.default_embedding)} bytes")
        if layer_type in (LayerType.HostLayer, LayerType.Hierarchical):
            if config is None or "default_embedding" not in config:
                self.config.default_embedding = [0] * row_bytes
        elif len(self.config.default_embedding) > 0:
            raise ValueError(f"config['default_embedding'] is only supported for HostLayer and "
                             f"Hierarchical layers, got layer_type={layer_type}")
        self.gpu_cache_size = gpu_cache_size
        self.host_cache_size = host_cache_size
        self.optimize_for_training = optimize_for_training
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        if self.device.type == "cpu":
            if layer_type != LayerType.HostLayer:
                raise ValueError(f"device='cpu' is only supported with LayerType.HostLayer, "
                                 f"got layer_type={layer_type}")
            self.device_index = -1
        elif self.device.type == "cuda":
            self.device_index = (self.device.index if self.device.index is not None
                                 else torch.cuda.current_device())
        else:
            raise ValueError(f"NV Embedding only supports cuda or cpu devices, got {self.device.type}")
        self.id = id if id is not None else builtins.id(self)
        self.table_ids = {}

        if layer_type == LayerType.GPULayer:
            if storage is not None and not isinstance(storage, nve.MemBlock):
                raise ValueError("GPULayer requires storage to be a MemBlock or None")
            if weight_init is not None:
                tensor_storage = weight_init.detach().clone().to(self.device)
            else:
                tensor_storage = torch.empty(num_embeddings, embedding_size, dtype=data_type,
                                             device=self.device)
            memblock = storage if storage is not None else nve.UserMemBlock(
                tensor_storage.data_ptr(), tensor_storage.nbytes)
            self.memblock_type = memblock.get_type()
            self.storage = memblock
            self.emb_layer = nve.GPUEmbedding(embedding_size, num_embeddings, self.layer_data_type,
                                              memblock, self.device_index, self.config)
            self.table_ids = {0: "gpu"}
        elif layer_type == LayerType.LinearUVM:
            if gpu_cache_size == 0:
                raise ValueError("GPU cache size > 0 is required for UVM embedding")
            if storage is not None and not isinstance(storage, nve.MemBlock):
                raise ValueError("LinearUVM requires storage to be a MemBlock or None")
            memblock = storage if storage is not None else nve.ManagedMemBlock(
                embedding_size, num_embeddings, self.layer_data_type, [self.device_index])
            self.memblock_type = memblock.get_type()
            self.storage = memblock
            self.emb_layer = nve.LinearUVMEmbedding(embedding_size, num_embeddings,
                                                    self.layer_data_type, memblock, gpu_cache_size,
                                                    optimize_for_training, self.device_index,
                                                    self.config)
            tensor_storage = torch.utils.dlpack.from_dlpack(
                nve.get_dl_tensor(self.emb_layer, self.layer_data_type))
            if weight_init is not None:
                tensor_storage.copy_(weight_init)
            self.table_ids = {0: "gpu_cache"}
        elif layer_type == LayerType.Hierarchical:
            if storage is None or not isinstance(storage, nve.Table):
                raise ValueError("Hierarchical requires storage to be a Table or NVEParameterServer")
            if gpu_cache_size == 0:
                raise ValueError("GPU cache size > 0 is required for hierarchical embedding")
            if weight_init is not None:
                raise ValueError("Weight init is not supported for hierarchical embedding")
            self.emb_layer = nve.HierarchicalEmbedding()
        elif layer_type == LayerType.HostLayer:
            if optimize_for_training:
                raise ValueError(
                    "HostLayer is inference-only and does not support training. "
                    "Pass optimize_for_training=False when using LayerType.HostLayer.")
            if storage is not None and not isinstance(storage, nve.MemBlock):
                raise ValueError("HostLayer requires storage to be a MemBlock or None")
            self.emb_layer = nve.HostEmbedding()
        else:
            raise ValueError(f"Unknown layer_type: {layer_type}")
        self.weight = CachedTable(tensor_storage, cache=self.emb_layer)
        # Per-layer identity marker: its data_ptr is the registry key the ops
        # dispatch on; it stays out of state_dict and never moves.
        self.register_buffer("marker_tensor",
                             torch.tensor([self.id], dtype=torch.int64, device=self.device),
                             persistent=False)
        self.dtype_tag = int(self.layer_data_type)
        if HAS_TORCH_OPS:
            nve.register_for_torch(self.marker_tensor.data_ptr(), self.emb_layer)

    def __del__(self):
        if HAS_TORCH_OPS and "marker_tensor" in getattr(self, "_buffers", {}):
            nve.unregister_from_torch(self._buffers["marker_tensor"].data_ptr())

    def to(self, *args, **kwargs):
        """Moves parameters and buffers except the table (`weight`, which stays
        where its layer reads it) and the identity marker (nve_layers.py:339-354)."""
        device, dtype, non_blocking, _ = torch._C._nn._parse_to(*args, **kwargs)
        for name, param in self.named_parameters():
            if name != "weight":
                param.data = param.data.to(device, dtype if dtype else param.dtype, non_blocking)
        for name, buf in self.named_buffers():
            if name == "marker_tensor":
                continue
            buf.data = buf.data.to(device, dtype if dtype else buf.dtype, non_blocking)
        return self

    def update(self, keys: torch.Tensor, updates: torch.Tensor):
        self.emb_layer.update(torch.numel(keys), keys.data_ptr(), updates.data_ptr(),
                              _current_stream_handle(self.device))

    def insert(self, keys: torch.Tensor, values: torch.Tensor, table_id: int):
        """Best-effort insert of rows into table `table_id` of the layer
        (nve_layers.py:369-382), asynchronous on the current stream."""
        self.emb_layer.insert(torch.numel(keys), keys.data_ptr(), values.data_ptr(), table_id,
                              _current_stream_handle(self.device))

    def clear(self):
        self.emb_layer.clear(_current_stream_handle(self.device))

    def erase(self, keys: torch.Tensor, table_id: int):
        self.emb_layer.erase(torch.numel(keys), keys.data_ptr(), table_id,
                             _current_stream_handle(self.device))

    def load_from_stream(self, stream):
        """Fill the table from the .nve entry named by this module's id
        (nve_layers.py:400-401)."""
        nve.load_tensor_from_stream(self.emb_layer, stream, self.id)


class NVEmbedding(NVEmbeddingBase):
    """torch.nn.Embedding over an NVE layer (nve_layers.py:386-453)."""

    def __init__(self, num_embeddings: int, embedding_size: int, data_type: torch.dtype,
                 layer_type: LayerType, *, gpu_cache_size: int = 0, host_cache_size: int = 0,
                 storage=None, weight_init: Optional[torch.Tensor] = None,
                 optimize_for_training: bool = True, device: Optional[torch.device] = None,
                 id: Optional[int] = None, config: Optional[dict] = None):
        super().__init__(num_embeddings, embedding_size, data_type, layer_type,
                         gpu_cache_size=gpu_cache_size, host_cache_size=host_cache_size,
                         storage=storage, weight_init=weight_init,
                         optimize_for_training=optimize_for_training, device=device, id=id,
                         config=config)

    def forward(self, keys: torch.Tensor):
        _check_forward_inputs(keys)
        if self.optimize_for_training:
            return nve_ops.NVEmbeddingOpTraining.apply(self.marker_tensor, keys, self.weight,
                                                       self.embedding_size, self.dtype_tag)
        return nve_ops.NVEmbeddingOp.apply(self.marker_tensor, keys, self.embedding_size,
                                           self.dtype_tag)


class NVEmbeddingBag(NVEmbeddingBase):
    """torch.nn.EmbeddingBag over an NVE layer (nve_layers.py:455-556): modes
    'sum', 'mean' and 'concat' ('max' is not implemented); offsets follow
    include_last_offset=True (num_bags + 1 entries ending at len(input))."""

    def __init__(self, num_embeddings: int, embedding_size: int, data_type: torch.dtype,
                 layer_type: LayerType, mode: str, *, gpu_cache_size: int = 0,
                 host_cache_size: int = 0, storage=None,
                 weight_init: Optional[torch.Tensor] = None, optimize_for_training: bool = True,
                 device: Optional[torch.device] = None, id: Optional[int] = None,
                 config: Optional[dict] = None):
        if mode != "concat":
            nve_ops.pooling_type_from_mode(mode, weighted=False)
        super().__init__(num_embeddings, embedding_size, data_type, layer_type,
                         gpu_cache_size=gpu_cache_size, host_cache_size=host_cache_size,
                         storage=storage, weight_init=weight_init,
                         optimize_for_training=optimize_for_training, device=device, id=id,
                         config=config)
        self.mode = mode

    def forward(self, input: torch.Tensor, offsets: torch.Tensor,
                per_sample_weights: Optional[torch.Tensor] = None):
        _check_forward_inputs(input, offsets, per_sample_weights)
        if self.mode == "concat":
            if self.optimize_for_training:
                return nve_ops.NVEmbeddingOpTraining.apply(self.marker_tensor, input, self.weight,
                                                           self.embedding_size, self.dtype_tag)
            return nve_ops.NVEmbeddingOp.apply(self.marker_tensor, input, self.embedding_size,
                                               self.dtype_tag)
        pooling_type = int(nve_ops.pooling_type_from_mode(
            self.mode, weighted=per_sample_weights is not None))
        if self.optimize_for_training:
            return nve_ops.NVEmbeddingBagOpTraining.apply(
                self.marker_tensor, input, self.weight, offsets, per_sample_weights, pooling_type,
                self.embedding_size, self.dtype_tag)
        return nve_ops.NVEmbeddingBagOp.apply(self.marker_tensor, input, offsets,
                                              per_sample_weights, pooling_type,
                                              self.embedding_size, self.dtype_tag)

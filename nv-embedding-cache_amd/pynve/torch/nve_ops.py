"""Autograd wrappers of the nve_ops custom ops (python/pynve/torch/nve_ops.py).

Forward goes through torch.ops.nve_ops.* (traceable).  Backward: the
inference ops raise as in the reference (nve_ops.py:83-86); the training ops
(nve_ops.py:89-128, :157-226) take the CachedTable weight as an unused forward
input and return its gradient as a sparse COO tensor (unique keys x rows),
computed on the GPU by the layer binding's concat_backprop / pooling_backprop.
"""
import torch

from .. import nve
from . import HAS_TORCH_OPS  # noqa: F401  (ops are registered on import)


def _stream_handle(device):
    if device.type == "cpu":
        return 0
    return torch.cuda.current_stream(device).cuda_stream


def pooling_type_from_mode(mode, weighted):
    """'sum' / 'mean' (weighted or not) -> PoolingType_t (nve_ops.py:32-50);
    every other mode ('concat' is routed separately, 'max' is unsupported) raises."""
    if mode == "sum":
        return nve.PoolingType_t.WeightedSum if weighted else nve.PoolingType_t.Sum
    if mode == "mean":
        return nve.PoolingType_t.WeightedMean if weighted else nve.PoolingType_t.Mean
    raise ValueError(f"Unsupported pooling mode {mode!r}; expected 'sum' or 'mean' "
                     "('concat' is handled separately). 'max' pooling is not implemented.")


class NVEmbeddingOp(torch.autograd.Function):
    @staticmethod
    def forward(marker, keys, embedding_size, dtype):
        return torch.ops.nve_ops.embedding_lookup(marker, keys, embedding_size, dtype)

    @staticmethod
    def setup_context(ctx, inputs, output):
        pass

    @staticmethod
    def backward(ctx, grad_output):
        raise RuntimeError("NVEmbeddingOp does not support backward. "
                           "Use optimize_for_training=True to enable gradient computation.")


class NVEmbeddingOpTraining(torch.autograd.Function):
    @staticmethod
    def forward(marker, keys, weight, embedding_size, dtype):
        return torch.ops.nve_ops.embedding_lookup(marker, keys, embedding_size, dtype)

    @staticmethod
    def setup_context(ctx, inputs, output):
        marker, keys, weight, embedding_size, dtype = inputs
        ctx.save_for_backward(keys, weight)

    @staticmethod
    def backward(ctx, grad_output):
        keys, weight = ctx.saved_tensors
        keys_flat = keys.reshape((1, -1))
        num_keys = keys_flat.numel()
        embed_dim = grad_output.shape[-1]
        grad = grad_output.reshape(-1, embed_dim).contiguous()
        unique_keys = torch.empty(num_keys, dtype=torch.int64, device=keys.device)
        result = torch.empty(num_keys, embed_dim, dtype=grad_output.dtype, device=keys.device)
        num_unique = weight.emb_layer.concat_backprop(
            num_keys, keys_flat.data_ptr(), grad.data_ptr(), unique_keys.data_ptr(),
            result.data_ptr(), _stream_handle(keys.device))
        grad_weight = torch.sparse_coo_tensor(unique_keys[:num_unique].reshape((1, -1)),
                                              result[:num_unique], weight.shape, device=weight.device)
        return None, None, grad_weight, None, None


class NVEmbeddingBagOp(torch.autograd.Function):
    @staticmethod
    def forward(marker, keys, offsets, per_sample_weights, pooling_type, embedding_size, dtype):
        return torch.ops.nve_ops.embedding_lookup_with_pooling(
            marker, keys, offsets, per_sample_weights, pooling_type, embedding_size, dtype)

    @staticmethod
    def setup_context(ctx, inputs, output):
        pass

    @staticmethod
    def backward(ctx, grad_output):
        raise RuntimeError("NVEmbeddingBagOp does not support backward. "
                           "Use optimize_for_training=True to enable gradient computation.")


class NVEmbeddingBagOpTraining(torch.autograd.Function):
    @staticmethod
    def forward(marker, keys, weight, offsets, per_sample_weights, pooling_type, embedding_size,
                dtype):
        return torch.ops.nve_ops.embedding_lookup_with_pooling(
            marker, keys, offsets, per_sample_weights, pooling_type, embedding_size, dtype)

    @staticmethod
    def setup_context(ctx, inputs, output):
        (marker, keys, weight, offsets, per_sample_weights, pooling_type,
         embedding_size, dtype) = inputs
        ctx.pooling_type = pooling_type
        ctx.has_per_sample_weights = per_sample_weights is not None
        if ctx.has_per_sample_weights:
            ctx.save_for_backward(keys, weight, offsets, per_sample_weights)
        else:
            ctx.save_for_backward(keys, weight, offsets)

    @staticmethod
    def backward(ctx, grad_output):
        if ctx.has_per_sample_weights:
            keys, weight, offsets, per_sample_weights = ctx.saved_tensors
        else:
            keys, weight, offsets = ctx.saved_tensors
            per_sample_weights = None
        num_keys = keys.numel()
        embed_dim = grad_output.shape[-1]
        grad = grad_output.contiguous()
        unique_keys = torch.empty(num_keys, dtype=torch.int64, device=keys.device)
        result = torch.empty(num_keys, embed_dim, dtype=grad_output.dtype, device=keys.device)
        weight_dtype = nve.DataType_t.Unknown
        weight_ptr = 0
        if per_sample_weights is not None:
            per_sample_weights = per_sample_weights.contiguous()
            weight_dtype = (nve.DataType_t.Float32 if per_sample_weights.dtype == torch.float32
                            else nve.DataType_t.Float16)
            weight_ptr = per_sample_weights.data_ptr()
        num_unique = weight.emb_layer.pooling_backprop(
            num_keys, keys.data_ptr(), grad.data_ptr(), unique_keys.data_ptr(), result.data_ptr(),
            ctx.pooling_type, offsets.numel() - 1, offsets.data_ptr(), weight_dtype, weight_ptr,
            _stream_handle(keys.device))
        grad_weight = torch.sparse_coo_tensor(unique_keys[:num_unique].reshape((1, -1)),
                                              result[:num_unique], weight.shape, device=weight.device)
        return None, None, grad_weight, None, None, None, None, None

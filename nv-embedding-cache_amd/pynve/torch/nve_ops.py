"""Autograd wrappers of the nve_ops custom ops (python/pynve/torch/nve_ops.py).

Forward goes through torch.ops.nve_ops.* (traceable).  Backward: the
inference ops raise as in the reference (nve_ops.py:83-86); the training ops
keep the reference's signature (the CachedTable weight is an input) but the
gradient kernels are not part of this build, so their backward raises
NotImplementedInBuild.
"""
import torch

from .. import _lib
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


def _no_training():
    raise _lib.NotImplementedInBuild(
        _lib.NOT_IMPLEMENTED, "Gradients of NVEmbedding lookups (training) are not part of this build")


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
        pass

    @staticmethod
    def backward(ctx, grad_output):
        _no_training()


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
        pass

    @staticmethod
    def backward(ctx, grad_output):
        _no_training()

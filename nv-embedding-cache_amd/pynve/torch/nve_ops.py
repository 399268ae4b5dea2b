"""Autograd over the nve_ops custom ops.

Interface kept from the reference's python/pynve/torch/nve_ops.py: the four
autograd functions NVEmbeddingOp / NVEmbeddingOpTraining (one row per key) and
NVEmbeddingBagOp / NVEmbeddingBagOpTraining (pooled bags), and
pooling_type_from_mode.  The forward of every function is the traceable
torch.ops.nve_ops call.

Gradients.  An inference function (a layer built with
optimize_for_training=False) has none and says so when asked.  A training
function takes the layer's `weight` (a CachedTable) as an extra forward input
only so that autograd reaches it; its gradient is a sparse COO tensor over the
table's rows: the unique keys of the batch and, for each, the sum over its
positions of (its weight in the bag) x (the output gradient of its bag),
computed on the GPU by the layer binding's backprop entry
(nve_amd_pooling_backprop).
"""
import torch

from .. import nve
from . import HAS_TORCH_OPS  # noqa: F401  (importing registers the ops)

# (mode, weighted) -> pooling type of the C ABI
_MODES = {
    ("sum", False): nve.PoolingType_t.Sum,
    ("sum", True): nve.PoolingType_t.WeightedSum,
    ("mean", False): nve.PoolingType_t.Mean,
    ("mean", True): nve.PoolingType_t.WeightedMean,
}


def pooling_type_from_mode(mode, weighted):
    """The pooling type of an EmbeddingBag mode: 'sum' or 'mean', weighted when
    per-sample weights are given.  'concat' never pools (the caller routes it to
    the per-key lookup) and 'max' has no kernel: both raise ValueError."""
    try:
        return _MODES[(mode, bool(weighted))]
    except (KeyError, TypeError):
        raise ValueError(f"pooling mode {mode!r} cannot be computed here: use 'sum' or 'mean' "
                         "(or route 'concat' to the per-key lookup)") from None


def _stream_of(t):
    return torch.cuda.current_stream(t.device).cuda_stream if t.is_cuda else 0


def _no_gradient(name):
    raise RuntimeError(f"{name}: this layer was built for inference (optimize_for_training=False) "
                       "and has no gradient; build it with optimize_for_training=True to train it")


def _table_gradient(weight, keys, grad_rows, backprop):
    """Runs `backprop(unique_out, rows_out)` (one of the binding's backprop
    entries, returning the unique-key count) and wraps its result as the sparse
    gradient of `weight`."""
    n = keys.numel()
    dim = grad_rows.shape[-1]
    unique = torch.empty(n, dtype=torch.int64, device=keys.device)
    rows = torch.empty((n, dim), dtype=grad_rows.dtype, device=keys.device)
    u = backprop(unique, rows)
    return torch.sparse_coo_tensor(unique[:u].unsqueeze(0), rows[:u], weight.shape, device=weight.device)


class NVEmbeddingOp(torch.autograd.Function):
    """Per-key lookup without a gradient."""

    @staticmethod
    def forward(marker, keys, embedding_size, dtype):
        return torch.ops.nve_ops.embedding_lookup(marker, keys, embedding_size, dtype)

    @staticmethod
    def setup_context(ctx, inputs, output):
        return None

    @staticmethod
    def backward(ctx, grad_output):
        _no_gradient("NVEmbeddingOp")


class NVEmbeddingOpTraining(torch.autograd.Function):
    """Per-key lookup whose gradient is the sparse table gradient: each unique
    key gets the sum of the output-gradient rows of its positions."""

    @staticmethod
    def forward(marker, keys, weight, embedding_size, dtype):
        return torch.ops.nve_ops.embedding_lookup(marker, keys, embedding_size, dtype)

    @staticmethod
    def setup_context(ctx, inputs, output):
        _, keys, weight, _, _ = inputs
        ctx.save_for_backward(keys, weight)

    @staticmethod
    def backward(ctx, grad_output):
        keys, weight = ctx.saved_tensors
        flat_keys = keys.reshape(-1)
        g = grad_output.reshape(flat_keys.numel(), -1).contiguous()
        binding = weight.emb_layer

        def run(unique, rows):
            return binding.concat_backprop(flat_keys.numel(), flat_keys.data_ptr(), g.data_ptr(),
                                           unique.data_ptr(), rows.data_ptr(), _stream_of(flat_keys))

        return None, None, _table_gradient(weight, flat_keys, g, run), None, None


class NVEmbeddingBagOp(torch.autograd.Function):
    """Pooled lookup (CSR bags) without a gradient."""

    @staticmethod
    def forward(marker, keys, offsets, per_sample_weights, pooling_type, embedding_size, dtype):
        return torch.ops.nve_ops.embedding_lookup_with_pooling(
            marker, keys, offsets, per_sample_weights, pooling_type, embedding_size, dtype)

    @staticmethod
    def setup_context(ctx, inputs, output):
        return None

    @staticmethod
    def backward(ctx, grad_output):
        _no_gradient("NVEmbeddingBagOp")


class NVEmbeddingBagOpTraining(torch.autograd.Function):
    """Pooled lookup whose gradient is the sparse table gradient: key k of bag b
    receives w_k x grad[b], w_k being 1 (Sum), its per-sample weight
    (WeightedSum), 1 / |b| (Mean) or its weight over the bag's weight sum
    (WeightedMean)."""

    @staticmethod
    def forward(marker, keys, weight, offsets, per_sample_weights, pooling_type, embedding_size, dtype):
        return torch.ops.nve_ops.embedding_lookup_with_pooling(
            marker, keys, offsets, per_sample_weights, pooling_type, embedding_size, dtype)

    @staticmethod
    def setup_context(ctx, inputs, output):
        _, keys, weight, offsets, psw, pooling_type, _, _ = inputs
        ctx.pooling_type = int(pooling_type)
        ctx.weighted = psw is not None
        saved = (keys, weight, offsets) + ((psw,) if psw is not None else ())
        ctx.save_for_backward(*saved)

    @staticmethod
    def backward(ctx, grad_output):
        keys, weight, offsets, *rest = ctx.saved_tensors
        psw = rest[0].contiguous() if ctx.weighted else None
        g = grad_output.contiguous()
        binding = weight.emb_layer
        wtype, wptr = nve.DataType_t.Unknown, 0
        if psw is not None:
            wtype = nve.DataType_t.Float16 if psw.dtype == torch.float16 else nve.DataType_t.Float32
            wptr = psw.data_ptr()

        def run(unique, rows):
            return binding.pooling_backprop(keys.numel(), keys.data_ptr(), g.data_ptr(), unique.data_ptr(),
                                            rows.data_ptr(), ctx.pooling_type, offsets.numel() - 1,
                                            offsets.data_ptr(), wtype, wptr, _stream_of(keys))

        return None, None, _table_gradient(weight, keys, g, run), None, None, None, None, None

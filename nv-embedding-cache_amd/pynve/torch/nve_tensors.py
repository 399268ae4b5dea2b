"""CachedTable: the `weight` Parameter of the NVEmbedding layers
(python/pynve/torch/nve_tensors.py:18-80).

It wraps the table's storage and keeps a reference to the layer binding
(`emb_layer`).  `add_` is the optimizer's update hook: a sparse row-gradient
is accumulated into the layer's table and caches (nve_tensors.py:64-80).
"""
import torch

from .. import _lib


class CachedTable(torch.nn.parameter.Parameter):
    def __new__(cls, *args, **kwargs):
        if "cache" not in kwargs:
            raise Exception("building a CachedTable Tensor require a viable cache argument")
        cache = kwargs.pop("cache")
        instance = super().__new__(cls, *args, **kwargs)
        instance.emb_layer = cache
        return instance

    def __getstate__(self):
        # the binding holds native handles and cannot be pickled
        state = dict(self.__dict__)
        state["emb_layer"] = None
        return state

    def add_(self, other, *, alpha=1):
        """self += alpha * other for a sparse `other` over rows (its nonzero
        rows go to the layer's accumulate, which updates the table and every
        cache that holds them)."""
        if not other.is_sparse:
            raise _lib.InvalidArgument(_lib.INVALID_ARGUMENT, "add_ takes a sparse row tensor")
        factored = (other * alpha).coalesce()
        keys = factored.indices()[0].contiguous()
        values = factored.values().to(self.dtype).contiguous()
        stream = torch.cuda.current_stream().cuda_stream
        self.emb_layer.accumulate(factored._nnz(), keys.data_ptr(), values.data_ptr(), stream)
        torch.cuda.current_stream().synchronize()  # keys / values are temporaries
        return self

"""CachedTable: the `weight` Parameter of the NVEmbedding layers
(python/pynve/torch/nve_tensors.py:18-80).

It wraps the table's storage and keeps a reference to the layer binding
(`emb_layer`).  Only lookups are in this build, so `add_` -- the optimizer's
update hook in the reference, which accumulates into the caches -- raises.
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
        raise _lib.NotImplementedInBuild(
            _lib.NOT_IMPLEMENTED, "Optimizer updates of an NVEmbedding table (accumulate) "
            "are not part of this build")

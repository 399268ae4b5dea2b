"""CachedTable: the `weight` Parameter of the NVEmbedding layers (the role of
the reference's python/pynve/torch/nve_tensors.py:18-80).

The parameter's data is the layer's table as torch sees it; the native layer
binding that owns the table and its caches rides along as `emb_layer`.  Two
things differ from a plain Parameter:

* the binding is a process-local native handle, so it is left out of the
  pickled state (torch.export.save pickles the module's parameters; the
  exported graph reaches the layer through its marker tensor instead);
* `add_` is the optimizer's update hook: a sparse row gradient is sent to the
  layer's accumulate, which updates the table and every cache holding a row.
"""
import torch

from .. import _lib


class CachedTable(torch.nn.parameter.Parameter):
    # attributes that only mean something inside this process
    _PROCESS_LOCAL = ("emb_layer",)

    def __new__(cls, data=None, requires_grad=True, *, cache):
        # `cache` is keyword-only and has no default: a CachedTable without a
        # layer binding behind it cannot apply an update, so there is none
        if cache is None:
            raise _lib.InvalidArgument(_lib.INVALID_ARGUMENT,
                                       "CachedTable needs the layer binding that owns the table (cache=)")
        param = super().__new__(cls, data, requires_grad)
        param.emb_layer = cache
        return param

    def __getstate__(self):
        # a copy: the live parameter keeps its binding after being pickled
        return {k: (None if k in self._PROCESS_LOCAL else v) for k, v in self.__dict__.items()}

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

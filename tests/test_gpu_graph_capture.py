"""The fused find-and-pool of the GPU layer captured into a HIP graph and
replayed: a serving loop that replays one captured lookup over fresh keys.
The layer's context is made on the capturing stream and warmed up first (its
first call sizes its buffers); a captured call then allocates nothing and
waits for nothing.  Each replay, with eager work and synchronizations between
replays, must equal the eager lookup of the same keys bit for bit."""
import ctypes

import numpy as np
import pytest

from nve_helpers import float_table, to_dev, vp
from oracle import oracle as O
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("bags,hot", [(256, 1024), (2048, 20)], ids=["long_bags", "short_bags"])
def test_captured_pooled_lookup_replays_match_eager(bags, hot):
    rng = np.random.default_rng(bags + hot)
    rows, dim = 100000, 128
    tb = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    d_table = to_dev(tb.reshape(-1))
    L = _lib.load()
    cfg = L.nve_gpu_embedding_layer_config_default()
    cfg.layer_name = b"graph"
    cfg.embedding_table = d_table.data_ptr()
    cfg.num_embeddings = rows
    cfg.embedding_width_in_bytes = dim * 2
    cfg.value_dtype = _lib.DT_F16
    layer = ctypes.c_void_p()
    _lib.call("nve_gpu_embedding_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(cfg), None)
    s = torch.cuda.Stream()
    ctx = ctypes.c_void_p()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(ctx), ctypes.c_void_p(s.cuda_stream),
              ctypes.c_void_p(s.cuda_stream), None, None)
    n = bags * hot
    keys = torch.zeros(n, dtype=torch.int64, device="cuda")
    out = torch.zeros((bags, dim), dtype=torch.float16, device="cuda")

    def lookup(k, o):
        _lib.call("nve_layer_lookup_pooled", layer, ctx, n, vp(k), vp(o), dim * 2, None, _lib.POOL_SUM,
                  _lib.SPARSE_FIXED, None, 0, hot, None, 0, _lib.DT_F16, None)

    with torch.cuda.stream(s):
        keys.copy_(torch.from_numpy(rng.integers(0, rows, size=n)).cuda())
        lookup(keys, out)  # warm-up: the first call sizes the context's buffers
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        lookup(keys, out)
    eager = torch.zeros_like(out)
    for r in range(4):
        batch = torch.from_numpy((rng.zipf(1.05, size=n) % rows).astype(np.int64)).cuda()
        with torch.cuda.stream(s):
            keys.copy_(batch)
            g.replay()
            got = out.clone()
            lookup(batch, eager)  # eager call of the same keys between replays
        s.synchronize()
        assert torch.equal(got, eager), r
        ref = O.pool(O.linear_row_ptrs(batch.cpu().numpy(), np.ascontiguousarray(tb).reshape(-1), dim * 2),
                     O.F16, dim, O.FIXED, O.SUM, n, None, bags, hot, None, 0, O.F16)
        if hot <= 32:  # one lane group per bag: the oracle's order
            assert np.array_equal(got.cpu().numpy().view(np.uint16), ref), r
    del g
    _lib.call("nve_context_wait", ctx)
    _lib.call("nve_context_destroy", ctx)
    _lib.call("nve_layer_destroy", layer)

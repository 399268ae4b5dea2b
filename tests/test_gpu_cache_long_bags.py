"""GPU parity of pooling over a set-associative cache, long bags (the cache
variant of the split kernel: cache slots and backing-table rows as 32-bit
codes) and short bags (the general pool kernel); find_and_combine over a
GpuTable, find_and_combine_kernel.cuh:40-154, reached through a LinearUVM
layer, linear_embedding_layer.cu:91-209.

* With the cache holding exact copies of backing rows, a pooled lookup must
  equal the same lookup over the linear table bit for bit (same bag cut, same
  summation order), whatever mix of hits and misses the keys make.
* With every cached value negated, a wrong hit / miss decision changes the
  output: the result is compared with the oracle's cache model (fp32
  tolerance: the oracle adds a bag in key order).
* The reported hit rate is exact; keys outside the backing table read
  nothing."""
import ctypes

import numpy as np
import pytest

from nve_helpers import float_table, rel_close, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib
from test_gpu_cache_lookup import CachedTable
from test_gpu_find_and_pool import run_pool

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DT = {O.F16: _lib.DT_F16, O.F32: _lib.DT_F32}


def layer_over(ct, key_bytes):
    L = _lib.load()
    never = ctypes.c_void_p()
    _lib.call("nve_heuristic_create_never", ctypes.byref(never))
    lc = L.nve_linear_uvm_layer_config_default()
    lc.insert_heuristic = never.value
    layer = ctypes.c_void_p()
    kt = _lib.KEY_INT32 if key_bytes == 4 else _lib.KEY_INT64
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), kt, ctypes.byref(lc), ct.table, None)
    _lib.call("nve_heuristic_destroy", never)
    lctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(lctx), s, s, None, None)
    return layer, lctx


def pooled(layer, lctx, keys, dim, dtype, pooling, off, bags, hot, w):
    es = 2 if dtype == O.F16 else 4
    out = torch.zeros((bags, dim * es), dtype=torch.uint8, device="cuda")
    hr = (ctypes.c_float * 1)()
    d_keys = to_dev(keys)
    d_off = to_dev(off) if off is not None else None
    d_w = to_dev(w) if w is not None else None
    sparse = _lib.SPARSE_CSR if off is not None else _lib.SPARSE_FIXED
    _lib.call("nve_layer_lookup_pooled", layer, lctx, keys.size, vp(d_keys), vp(out), dim * es, None, pooling,
              sparse, vp(d_off), 0 if off is None else off.size, hot, vp(d_w),
              _lib.DT_F32 if w is not None else _lib.DT_UNKNOWN, DT[dtype], hr)
    _lib.call("nve_context_wait", lctx)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16 if dtype == O.F16 else np.float32).reshape(bags, dim), hr[0]


def close(layer, lctx, ct):
    _lib.call("nve_context_destroy", lctx)
    _lib.call("nve_layer_destroy", layer)
    ct.close()


@pytest.mark.parametrize("shape", [(48, 600), (1500, 24)], ids=["long", "short"])
@pytest.mark.parametrize("key_bytes", [4, 8])
@pytest.mark.parametrize("dtype", [O.F16, O.F32])
@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_MEAN, _lib.POOL_WSUM])
def test_cached_copies_equal_the_linear_table_bitwise(shape, key_bytes, dtype, pooling):
    rng = np.random.default_rng(900 + key_bytes + 10 * dtype + pooling + shape[1])
    rows, dim = 20000, 128
    bags, hot = shape
    tb = float_table(rng, rows, dim, dtype, dyadic_values=False)
    ct = CachedTable(tb, 1 << 20, key_bytes, value_dtype=DT[dtype])
    kt = np.int64 if key_bytes == 8 else np.int32
    ct.model.insert_keys(rng.choice(6000, size=5000).astype(kt), uvm=ct.uvm_np.reshape(-1))
    ct.load_model()
    keys = np.where(rng.uniform(size=bags * hot) < 0.7, rng.integers(0, 6000, size=bags * hot),
                    rng.integers(0, rows, size=bags * hot)).astype(kt)
    keys[rng.uniform(size=keys.size) < 0.01] = rows + 3  # outside the backing table: nothing
    w = rng.uniform(0, 1, size=keys.size).astype(np.float32) if pooling == _lib.POOL_WSUM else None
    layer, lctx = layer_over(ct, key_bytes)
    got, hr = pooled(layer, lctx, keys, dim, dtype, pooling, None, bags, hot, w)
    ref = run_pool(tb, dtype, keys.astype(np.int64), pooling, _lib.SPARSE_FIXED, None, bags, hot, w, O.F32,
                   dtype)
    bits = np.uint16 if dtype == O.F16 else np.uint32
    assert np.array_equal(got.view(bits), ref.view(bits))
    _, _, misses = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
    assert abs(hr - (1.0 - misses / keys.size)) < 1e-6
    assert 0.0 < hr < 1.0
    close(layer, lctx, ct)


@pytest.mark.parametrize("lens", [(300, 1500), (1, 40)], ids=["long", "short"])
def test_hit_miss_decisions_against_the_cache_model(lens):
    """Cached values negated: every key's source shows in the output.  CSR bags
    of 300 to 1500 keys (or 1 to 40), one empty."""
    rng = np.random.default_rng(918 + lens[0])
    rows, dim, bags = 30000, 128, 40 if lens[0] > 1 else 600
    tb = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(tb, 2 << 20, 8)
    ct.model.insert_keys(rng.choice(8000, size=9000).astype(np.int64), uvm=ct.uvm_np.reshape(-1))
    d = ct.model.data()
    d.reshape(-1, 4)[:, 3] ^= np.uint8(0x80)
    ct.load_model()
    lens = rng.integers(lens[0], lens[1], size=bags)
    lens[5] = 0
    off = np.zeros(bags + 1, np.int64)
    off[1:] = np.cumsum(lens)
    n = int(off[-1])
    keys = np.where(rng.uniform(size=n) < 0.8, rng.integers(0, 8000, size=n),
                    rng.integers(0, rows, size=n)).astype(np.int64)
    layer, lctx = layer_over(ct, 8)
    got, hr = pooled(layer, lctx, keys, dim, O.F32, _lib.POOL_SUM, off, bags, 0, None)
    rows_ptr, _, misses = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
    ref = O.pool(rows_ptr, O.F32, dim, O.CSR, _lib.POOL_SUM, n, off, bags, 0, None, O.F32, O.F32)
    assert rel_close(got, ref.reshape(bags, dim), 1e-5)
    assert np.all(got[5] == 0)
    assert abs(hr - (1.0 - misses / n)) < 1e-6
    close(layer, lctx, ct)

"""LinearUVM layer cases of the reference's tests/embedding_layer/
uvm_layer_test.cpp not held elsewhere: a collection that switches between
plain and pooled lookups while the last lookup holds more keys than the
collection still needs (InflightInsertPoolingMixed and its reverse,
:1166-1240), the layer's validation of its backing table (UVMValidation,
:1033-1072), and insert / update / accumulate with a padded value stride
(UVMPaddedStride, :1366-1415).

The collections are held to the oracle's cache model: the insert takes the
first min_insert_size_gpu collected keys, from the backing table once a
pooled lookup has joined, and the whole cache state must match."""
import ctypes

import numpy as np
import pytest

from nve_helpers import dyadic, float_table, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib
from test_gpu_auto_insert_rows import Layer
from test_gpu_cache_insert import assert_same_state
from test_gpu_cache_lookup import CachedTable

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("first_kind", ["plain", "pooled"])
def test_collection_switching_kinds_takes_the_first_keys_it_needs(first_kind):
    """512 keys by one kind of lookup, then 1,536 by the other: the collection
    of 1,024 takes the first 512 of the second lookup, is promoted from the
    backing table (a pooled lookup took part), and those 1,024 keys then hit."""
    rng = np.random.default_rng(11 if first_kind == "plain" else 12)
    rows, dim = 20000, 32
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 16 << 20, 8)
    lay = Layer(ct, min_size=1024)
    keys = rng.permutation(rows)[:2048].astype(np.int64)
    a, b = keys[:512], keys[512:]
    (lay.plain if first_kind == "plain" else lay.pooled)(a)
    assert lay.hr[0] == 0.0
    (lay.pooled if first_kind == "plain" else lay.plain)(b)
    lay.wait()
    collected = keys[:1024]
    ct.model.insert_keys(collected, uvm=ct.uvm_np.reshape(-1))
    assert_same_state(ct)
    got = lay.plain(collected)
    assert lay.hr[0] > 0.9
    assert np.array_equal(got, uvm[collected])
    lay.close()
    ct.close()


def test_layer_rejects_a_backing_table_its_keys_cannot_address():
    """uvm_layer_test.cpp:1033-1072: a default row outside the backing table,
    and a backing table of 2^31 rows under int32 keys."""
    L = _lib.load()
    buf = torch.zeros(64, dtype=torch.uint8).pin_memory()
    for kt, num_rows, default_row, msg in ((_lib.KEY_INT64, 2, 2, "Default row index"),
                                           (_lib.KEY_INT32, 1 << 31, -1, "cannot be represented")):
        cfg = L.nve_gpu_table_config_default()
        cfg.cache_size, cfg.row_size_in_bytes, cfg.value_dtype = 1 << 16, 32, _lib.DT_F32
        cfg.uvm_table, cfg.uvm_num_rows = buf.data_ptr(), num_rows
        t = ctypes.c_void_p()
        _lib.call("nve_gpu_table_create", ctypes.byref(t), kt, ctypes.byref(cfg), None)
        lc = L.nve_linear_uvm_layer_config_default()
        lc.default_row_index = default_row
        lay = ctypes.c_void_p()
        st = L.nve_linear_uvm_layer_create(ctypes.byref(lay), kt, ctypes.byref(lc), t, None)
        assert st != _lib.SUCCESS
        assert msg in _lib.last_error()
        _lib.call("nve_table_destroy", t)


def test_insert_update_accumulate_with_a_padded_value_stride():
    """uvm_layer_test.cpp:1366-1415: 512 unique keys, 256-byte fp32 rows
    given at a 320-byte stride (the padding holds 0xEE); after each call the
    layer's lookups return the rows as packed.  Values are dyadic fractions,
    so the accumulate is exact."""
    rng = np.random.default_rng(21)
    rows, dim, n = 50000, 64, 512
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, 16 << 20, 8)
    L = _lib.load()
    never = ctypes.c_void_p()
    _lib.call("nve_heuristic_create_never", ctypes.byref(never))
    lc = L.nve_linear_uvm_layer_config_default()
    lc.insert_heuristic = never
    lay = ctypes.c_void_p()
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(lay), _lib.KEY_INT64, ctypes.byref(lc), ct.table, None)
    _lib.call("nve_heuristic_destroy", never)
    ctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", lay, ctypes.byref(ctx), s, s, None, None)
    keys = rng.permutation(rows)[:n].astype(np.int64)
    row, stride = dim * 4, dim * 4 + 64

    def padded(vals):
        p = np.full((n, stride), 0xEE, np.uint8)
        p[:, :row] = vals.view(np.uint8).reshape(n, row)
        return p

    def lookup():
        out = torch.zeros((n, row), dtype=torch.uint8, device="cuda")
        _lib.call("nve_layer_lookup", lay, ctx, n, vp(to_dev(keys)), vp(out), row, None, None)
        torch.cuda.synchronize()
        return out.cpu().numpy().view(np.float32)

    vals = dyadic(rng, (n, dim)).astype(np.float32)
    pv = padded(vals)  # kept alive across the call
    _lib.call("nve_layer_insert", lay, ctx, n, ctypes.c_void_p(keys.ctypes.data), stride, row,
              ctypes.c_void_p(pv.ctypes.data), 0)
    assert np.array_equal(lookup(), vals)
    upd = dyadic(rng, (n, dim)).astype(np.float32)
    pu = padded(upd)
    _lib.call("nve_layer_update", lay, ctx, n, ctypes.c_void_p(keys.ctypes.data), stride, row,
              ctypes.c_void_p(pu.ctypes.data), 0)
    assert np.array_equal(lookup(), upd)
    _lib.call("nve_layer_accumulate", lay, ctx, n, ctypes.c_void_p(keys.ctypes.data), stride, row,
              ctypes.c_void_p(pu.ctypes.data), _lib.DT_F32, 0)
    assert np.array_equal(lookup(), upd + upd)
    # the backing rows took the update and the accumulate too
    assert np.array_equal(ct.h_uvm.numpy().reshape(rows, row)[keys].view(np.float32), upd + upd)
    _lib.call("nve_context_wait", ctx)
    _lib.call("nve_context_destroy", ctx)
    _lib.call("nve_layer_destroy", lay)
    ct.close()

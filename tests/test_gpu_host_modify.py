"""GPU parity of the host-metadata cache (GPUTableConfig.modify_on_gpu =
false, the reference's CacheSAHostModify) against the oracle's model of that
policy.

After every modify the table's tags, way counters (bitwise), set timestamps,
insert clock and cached rows must equal the model's.  Cases follow
gpu_table_test.cpp / uvm_layer_test.cpp with modify_on_gpu = false: insert
with repeated keys, insert_from_uvm, erase (the way's counter survives), clear,
max_modify_size, int32 keys, keys handed over in host memory, and lookups
through the cache the host policy filled."""
import ctypes

import numpy as np
import pytest

from nve_helpers import float_table, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib
from test_gpu_cache_insert import assert_same_state, table_insert
from test_gpu_cache_lookup import CachedTable

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def test_num_sets_has_no_counter_term():
    # per set align16(8*8) + align16(8*256) = 2112 bytes: counters live on the host
    ct = CachedTable(np.zeros((10, 256), np.uint8), 2112 * 1000 + 2111, modify_on_gpu=False)
    assert ct.num_sets == 1000
    ct.close()


@pytest.mark.parametrize("key_bytes", [8, 4])
def test_insert_sequence_matches_model(key_bytes):
    rng = np.random.default_rng(301 + key_bytes)
    rows, dim = 50000, 16
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 96 * 1024, key_bytes, modify_on_gpu=False)  # ~ 370 sets: contention
    kdt = np.int64 if key_bytes == 8 else np.int32
    for step in range(6):
        keys = (rng.zipf(1.3, size=3000) % 20000).astype(kdt)
        vals = uvm[keys.astype(np.int64)]
        table_insert(ct, keys, vals, ct.width)
        ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
        assert_same_state(ct)
    ct.close()


def test_insert_from_uvm_erase_clear_sequence():
    """insert_from_uvm, then erase (the erased way keeps its counter, which the
    next insert must still see), more inserts with decay over skipped calls,
    then clear (counters, timestamps and the clock back to 0)."""
    rng = np.random.default_rng(307)
    rows, dim = 30000, 32
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 64 * 1024, 8, modify_on_gpu=False)

    def insert_uvm(keys):
        d_keys = to_dev(keys)
        _lib.call("nve_amd_table_insert_from_uvm", ct.table, ct.ctx, keys.size, vp(d_keys))
        ct.model.insert_keys(keys, uvm=ct.uvm_np.reshape(-1))

    for step in range(3):
        insert_uvm((rng.zipf(1.2, size=4000) % 10000).astype(np.int64))
        assert_same_state(ct)
    resident = [k for k in range(10000) if ct.model.find_way(k) >= 0]
    erase = np.array(resident[:40], np.int64)
    d_erase = to_dev(erase)
    _lib.call("nve_table_erase", ct.table, ct.ctx, erase.size, vp(d_erase))
    assert ct.model.erase(erase) == 40
    assert_same_state(ct)
    for step in range(3):
        insert_uvm((rng.zipf(1.2, size=4000) % 10000).astype(np.int64))
        assert_same_state(ct)
    _lib.call("nve_table_clear", ct.table, ct.ctx)
    ct.model.clear()
    assert_same_state(ct)
    insert_uvm((rng.zipf(1.2, size=2000) % 10000).astype(np.int64))
    assert_same_state(ct)
    ct.close()


def test_keys_and_values_in_host_memory_first_occurrence_rows():
    """Keys and values handed over in pageable host memory; each occurrence of
    a key carries a different row and the first one is inserted."""
    rng = np.random.default_rng(311)
    rows, dim = 2000, 12
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, 64 * 1024, 8, modify_on_gpu=False)
    keys = rng.integers(0, 300, size=1500).astype(np.int64)
    stride = ct.width + 16
    vals = rng.integers(0, 256, size=(keys.size, stride), dtype=np.uint8)
    _lib.call("nve_table_insert", ct.table, ct.ctx, keys.size, keys.ctypes.data_as(ctypes.c_void_p),
              stride, ct.width, vals.ctypes.data_as(ctypes.c_void_p))
    ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=stride)
    assert_same_state(ct)
    ct.close()


def test_max_modify_size_stops_the_policy():
    rng = np.random.default_rng(313)
    rows, dim = 8000, 8
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, 64 * 1024, 8, modify_on_gpu=False, max_modify_size=100)
    keys = rng.integers(0, 5000, size=4000).astype(np.int64)
    vals = uvm[keys]
    table_insert(ct, keys, vals, ct.width)
    ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width, max_modify_size=100)
    assert_same_state(ct)
    assert (ct.model.tags() != -1).sum() == 100
    ct.close()


def test_lookups_through_host_policy_cache():
    """find over the backing table after host-policy inserts: cached rows are
    the inserted values (here: negated rows), the rest come from the host."""
    rng = np.random.default_rng(317)
    rows, dim = 20000, 32
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 256 * 1024, 8, modify_on_gpu=False)
    keys = rng.integers(0, 4000, size=6000).astype(np.int64)
    vals = (-uvm.view(np.float32)[keys]).view(np.uint8)  # cache rows differ from the host rows
    table_insert(ct, keys, vals, ct.width)
    ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
    assert_same_state(ct)
    q = rng.integers(0, rows, size=5000).astype(np.int64)
    out = torch.zeros((q.size, ct.width), dtype=torch.uint8, device="cuda")
    d_q = to_dev(q)
    _lib.call("nve_table_find", ct.table, ct.ctx, q.size, vp(d_q), None, ct.width, vp(out), None)
    torch.cuda.synchronize()
    rows_ptr, _, misses = ct.model.resolve(q, ct.uvm_np.reshape(-1))
    ref = np.stack([np.frombuffer(ctypes.string_at(int(p), ct.width), np.uint8) for p in rows_ptr])
    assert np.array_equal(out.cpu().numpy(), ref)
    assert 0 < misses < q.size
    ct.close()


def test_uvm_layer_auto_insert_with_host_policy():
    """LinearUVM layer over a host-policy table: every pooled lookup equals
    the plain backing-table result while auto-insert fills the cache."""
    rng = np.random.default_rng(319)
    rows, dim, bags, hot = 40000, 64, 512, 16
    uvm = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    ct = CachedTable(uvm, 4 * 1024 * 1024, 8, value_dtype=_lib.DT_F16, modify_on_gpu=False)
    L = _lib.load()
    lc = L.nve_linear_uvm_layer_config_default()
    lc.min_insert_size_gpu = 4096
    layer = ctypes.c_void_p()
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), ct.table, None)
    lctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(lctx), s, s, None, None)
    keys = (rng.zipf(1.2, size=bags * hot) % rows).astype(np.int64)
    d_keys = to_dev(keys)
    ref = O.pool(O.linear_row_ptrs(keys, np.ascontiguousarray(uvm).reshape(-1), dim * 2), O.F16, dim,
                 O.FIXED, O.SUM, keys.size, None, bags, hot, None, 0, O.F16)
    out = torch.zeros((bags, dim), dtype=torch.float16, device="cuda")
    hr = (ctypes.c_float * 1)()
    rates = []
    for it in range(10):
        _lib.call("nve_layer_lookup_pooled", layer, lctx, keys.size, vp(d_keys), vp(out), dim * 2, None,
                  _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, hot, None, 0, _lib.DT_F16, hr)
        _lib.call("nve_context_wait", lctx)
        assert np.array_equal(out.cpu().numpy().view(np.uint16), ref)
        rates.append(hr[0])
    assert rates[0] == 0.0 and rates[-1] > 0.5, rates
    _lib.call("nve_context_destroy", lctx)
    _lib.call("nve_layer_destroy", layer)
    ct.close()

"""GPU parity of the cache insert (histogram -> per-set replacement ->
invalidate / copy / commit) against the oracle's lane-exact model of
SetReplaceDataKernel.

After every insert the GPU table's tags, way counters (bitwise), set
timestamps and cached rows must equal the model's.  Cases follow
tests/kernels/gpu_insert_tests.cu (random priorities, repeated inserts with
decay between them) and gpu_table_test.cpp (insert / insert_from_uvm,
duplicate keys, int32 keys, max_modify_size)."""
import ctypes

import numpy as np
import pytest

from nve_helpers import float_table, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib
from test_gpu_cache_lookup import CachedTable

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def gpu_state(ct):
    kdt = np.int32 if ct.key_bytes == 4 else np.int64
    tags = np.zeros(ct.num_sets * 8, kdt)
    ctr = np.zeros(ct.num_sets * 8, np.float32)
    ts = np.zeros(ct.num_sets, np.int64)
    gts = ctypes.c_int64()
    _lib.call("nve_amd_gpu_table_export_state", ct.table, tags.ctypes.data_as(ctypes.c_void_p),
              ctr.ctypes.data_as(ctypes.c_void_p), ts.ctypes.data_as(ctypes.c_void_p), ctypes.byref(gts))
    data = np.zeros(ct.num_sets * 8 * ct.width, np.uint8)
    ptr = ctypes.c_void_p()
    _lib.call("nve_amd_gpu_table_data", ct.table, ctypes.byref(ptr))
    from nve_helpers import hip_memcpy
    hip_memcpy(data.ctypes.data, ptr.value, data.nbytes)
    return tags.astype(np.int64), ctr, ts, gts.value, data


def assert_same_state(ct):
    tags, ctr, ts, gts, data = gpu_state(ct)
    assert np.array_equal(tags, ct.model.tags())
    assert np.array_equal(ctr.view(np.uint32), ct.model.counters().view(np.uint32))
    assert np.array_equal(ts, ct.model.set_ts())
    assert gts == ct.model.c.global_ts
    # cached rows: compare only occupied ways (empty ways hold whatever was there)
    mt = ct.model.tags()
    occ = np.repeat(mt != -1, ct.width)
    assert np.array_equal(data[occ], ct.model.data()[occ])


def table_insert(ct, keys, values, stride):
    d_keys = to_dev(keys)
    d_vals = to_dev(values.reshape(-1))
    _lib.call("nve_table_insert", ct.table, ct.ctx, keys.size, vp(d_keys), stride, ct.width, vp(d_vals))


@pytest.mark.parametrize("key_bytes", [8, 4])
def test_insert_sequence_matches_model(key_bytes):
    rng = np.random.default_rng(101 + key_bytes)
    rows, dim = 50000, 16
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 96 * 1024, key_bytes)  # ~ 350 sets: heavy contention
    kdt = np.int64 if key_bytes == 8 else np.int32
    for step in range(6):
        # Zipf-like repeats: counts differ, many ties among singletons
        keys = (rng.zipf(1.3, size=3000) % 20000).astype(kdt)
        vals = uvm[keys.astype(np.int64)]
        table_insert(ct, keys, vals, ct.width)
        ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
        assert_same_state(ct)
    ct.close()


def test_insert_all_ties_and_duplicates():
    """Every key once (all priorities equal): the networks' tie rules decide."""
    rng = np.random.default_rng(7)
    rows, dim = 10000, 8
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, 16 * 1024, 8)
    for step in range(4):
        keys = rng.permutation(rows)[:2000].astype(np.int64)
        vals = uvm[keys]
        table_insert(ct, keys, vals, ct.width)
        ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
        assert_same_state(ct)
    ct.close()


@pytest.mark.parametrize("case", ["below_bit_32", "bit_32_once", "wide_int64", "negative_int32", "single_key"])
def test_insert_key_sort_bits_first_assumed_then_checked(case):
    """The histogram's key sort first assumes that the keys differ only below
    bit 32 (four 8-bit passes, no host round trip before them) and checks that
    with the unique count; keys that differ higher up are sorted again on
    their exact bits.  Cache keys are any integers, not only row indices."""
    rng = np.random.default_rng(["below_bit_32", "bit_32_once", "wide_int64", "negative_int32",
                                 "single_key"].index(case) + 40)
    rows, dim = 4000, 8
    uvm = float_table(rng, rows, dim, O.F32)
    kb = 4 if case == "negative_int32" else 8
    ct = CachedTable(uvm, 64 * 1024, kb)
    n = 3000
    base = rng.zipf(1.2, size=n) % 700
    if case == "below_bit_32":
        keys = (base * 6_000_011 % (2**32)).astype(np.int64)
        keys[:2] = [0, 2**32 - 1]
    elif case == "bit_32_once":
        keys = (base * 6_000_011 % (2**32)).astype(np.int64)
        keys[n // 2] = 2**32
    elif case == "wide_int64":
        keys = (base.astype(np.int64) * 0x1E3779B97F4A7C15 % (2**62)).astype(np.int64) - 2**61
    elif case == "negative_int32":
        keys = (base - 350).astype(np.int32) * 3_000_017
    else:
        keys = np.array([2**40 + 3], np.int64)
    vals = rng.integers(0, 256, size=(keys.size, ct.width), dtype=np.uint8)
    table_insert(ct, keys, vals, ct.width)
    ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
    assert_same_state(ct)
    ct.close()


def test_insert_values_use_first_occurrence_and_padded_stride():
    rng = np.random.default_rng(9)
    rows, dim = 2000, 12
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, 64 * 1024, 8)
    keys = rng.integers(0, 300, size=1500).astype(np.int64)
    stride = ct.width + 16
    vals = rng.integers(0, 256, size=(keys.size, stride), dtype=np.uint8)  # each occurrence differs
    table_insert(ct, keys, vals, stride)
    ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=stride)
    assert_same_state(ct)
    ct.close()


def test_max_modify_size_truncates_histogram():
    rng = np.random.default_rng(13)
    rows, dim = 8000, 8
    uvm = float_table(rng, rows, dim, O.F32)
    L = _lib.load()
    ct = CachedTable(uvm, 64 * 1024, 8)
    ct.close()
    # rebuild with a small max_modify_size
    cfg = L.nve_gpu_table_config_default()
    cfg.cache_size = 64 * 1024
    cfg.row_size_in_bytes = uvm.shape[1]
    cfg.value_dtype = _lib.DT_F32
    cfg.max_modify_size = 100
    table = ctypes.c_void_p()
    _lib.call("nve_gpu_table_create", ctypes.byref(table), _lib.KEY_INT64, ctypes.byref(cfg), None)
    ctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_table_create_execution_context", table, ctypes.byref(ctx), s, s, None, None)
    model = O.Cache(64 * 1024, uvm.shape[1], 8)
    keys = rng.integers(0, 5000, size=4000).astype(np.int64)
    vals = uvm[keys]
    d_keys, d_vals = to_dev(keys), to_dev(vals.reshape(-1))
    _lib.call("nve_table_insert", table, ctx, keys.size, vp(d_keys), uvm.shape[1], uvm.shape[1], vp(d_vals))
    model.insert_keys(keys, values=vals.reshape(-1), value_stride=uvm.shape[1], max_modify_size=100)
    tags = np.zeros(model.num_sets * 8, np.int64)
    _lib.call("nve_amd_gpu_table_export_state", table, tags.ctypes.data_as(ctypes.c_void_p), None, None, None)
    assert np.array_equal(tags, model.tags())
    assert (tags != -1).sum() <= 100
    _lib.call("nve_context_destroy", ctx)
    _lib.call("nve_table_destroy", table)


def test_uvm_layer_auto_insert_raises_hit_rate_and_keeps_results():
    """Auto-insert promotes rows from the backing table, so every lookup must
    equal the plain linear-table result whatever is cached; the hit rate of a
    repeated Zipf batch climbs as inserts land (uvm_layer_test.cpp insert flow)."""
    rng = np.random.default_rng(17)
    rows, dim, bags = 40000, 64, 512
    uvm = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    ct = CachedTable(uvm, 4 * 1024 * 1024, 8, value_dtype=_lib.DT_F16)
    L = _lib.load()
    lc = L.nve_linear_uvm_layer_config_default()
    lc.min_insert_size_gpu = 4096
    layer = ctypes.c_void_p()
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), ct.table, None)
    lctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(lctx), s, s, None, None)
    hot = 16
    keys = (rng.zipf(1.2, size=bags * hot) % rows).astype(np.int64)
    d_keys = to_dev(keys)
    ref = O.pool(O.linear_row_ptrs(keys, np.ascontiguousarray(uvm).reshape(-1), dim * 2), O.F16, dim,
                 O.FIXED, O.SUM, keys.size, None, bags, hot, None, 0, O.F16)
    out = torch.zeros((bags, dim), dtype=torch.float16, device="cuda")
    hr = (ctypes.c_float * 1)()
    rates = []
    for it in range(12):
        _lib.call("nve_layer_lookup_pooled", layer, lctx, keys.size, vp(d_keys), vp(out), dim * 2, None,
                  _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, hot, None, 0, _lib.DT_F16, hr)
        _lib.call("nve_context_wait", lctx)  # joins a pending auto-insert
        assert np.array_equal(out.cpu().numpy().view(np.uint16), ref)
        rates.append(hr[0])
    assert rates[0] == 0.0
    assert rates[-1] > 0.5, rates
    _lib.call("nve_context_destroy", lctx)
    _lib.call("nve_layer_destroy", layer)
    ct.close()


@pytest.mark.parametrize("modify_on_gpu", [True, False])
@pytest.mark.parametrize("key_bytes", [8, 4])
def test_insert_from_uvm_keys_outside_the_backing_table(modify_on_gpu, key_bytes):
    """insert_from_uvm with keys below 0 or past the backing table: they have
    no source row and are never inserted (the reference would read past the
    table), while a resident one of them (put there by an insert with values)
    still gains its priority, under both policies."""
    rng = np.random.default_rng(61 + key_bytes + (0 if modify_on_gpu else 7))
    rows, dim = 3000, 16
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 48 * 1024, key_bytes, modify_on_gpu=modify_on_gpu)
    kdt = np.int64 if key_bytes == 8 else np.int32
    outside = np.array([rows + 5, -3], kdt)
    vals = rng.integers(0, 256, size=(outside.size, ct.width), dtype=np.uint8)
    table_insert(ct, outside[:1], vals[:1], ct.width)  # rows + 5 resident with its own values
    ct.model.insert_keys(outside[:1], values=vals[:1].reshape(-1), value_stride=ct.width)
    assert_same_state(ct)
    for step in range(3):
        keys = (rng.zipf(1.2, size=2500) % (rows + 400) - 100).astype(kdt)  # about 17 % outside
        keys[::50] = outside[step % 2]
        d_keys = to_dev(keys)
        _lib.call("nve_amd_table_insert_from_uvm", ct.table, ct.ctx, keys.size, vp(d_keys))
        ct.model.insert_keys(keys, uvm=ct.uvm_np.reshape(-1))
        assert_same_state(ct)
        tags = ct.model.tags()
        ways = np.nonzero(tags != -1)[0]
        resident = tags[ways] * ct.num_sets + ways // 8  # key = tag * num_sets + set
        assert np.all(((resident >= 0) & (resident < rows)) | (resident == rows + 5))
    assert ct.model.find_way(rows + 5) >= 0
    assert ct.model.find_way(-3) < 0
    ct.close()

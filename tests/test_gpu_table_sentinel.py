"""GpuTable cases of the reference's gpu_table_test.cpp that the other files
do not hold: a custom empty-way sentinel (GpuTableInvalidKey, :460-650) and
updates / accumulates of keys outside the backing table next to guard rows
(GpuTableOutOfRangeKeys, :652-775).

Sentinel: a table whose invalid_key is not -1 fills its empty ways with it; a
batch holding the sentinel itself inserts and finds its other keys; and -1
is then an ordinary key that round-trips.  The cache state after the insert
is also held to the oracle's model built with the same sentinel.

Guard rows: the host buffer holds 8 rows past uvm_num_rows; every 7th key
is negative or aimed at a guard row, and after update / update_accumulate
the whole buffer must equal the in-range keys applied alone."""
import ctypes

import numpy as np
import pytest

from nve_helpers import stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib
from test_gpu_cache_insert import gpu_state

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


class SentinelTable:
    """Cache-only GpuTable (1 MiB, 128-byte rows) with a given invalid_key."""

    def __init__(self, key_bytes, sentinel, modify_on_gpu=True):
        L = _lib.load()
        cfg = L.nve_gpu_table_config_default()
        cfg.cache_size = 1 << 20
        cfg.row_size_in_bytes = 128
        cfg.value_dtype = _lib.DT_F32
        cfg.invalid_key = sentinel
        cfg.modify_on_gpu = 1 if modify_on_gpu else 0
        self.table = ctypes.c_void_p()
        kt = _lib.KEY_INT64 if key_bytes == 8 else _lib.KEY_INT32
        _lib.call("nve_gpu_table_create", ctypes.byref(self.table), kt, ctypes.byref(cfg), None)
        self.ctx = ctypes.c_void_p()
        s = stream_ptr()
        _lib.call("nve_table_create_execution_context", self.table, ctypes.byref(self.ctx), s, s, None, None)
        ns = ctypes.c_int64()
        _lib.call("nve_amd_gpu_table_num_sets", self.table, ctypes.byref(ns))
        self.num_sets, self.width, self.key_bytes = ns.value, 128, key_bytes
        self.model = O.Cache(1 << 20, 128, key_bytes, sentinel=sentinel, host_modify=not modify_on_gpu)
        assert self.model.num_sets == self.num_sets

    def insert(self, keys, vals):
        d_keys, d_vals = to_dev(keys), to_dev(vals.reshape(-1))
        _lib.call("nve_table_insert", self.table, self.ctx, keys.size, vp(d_keys), 128, 128, vp(d_vals))
        self.model.insert_keys(keys, values=vals.reshape(-1), value_stride=128)

    def find(self, keys):
        out = torch.zeros((keys.size, 128), dtype=torch.uint8, device="cuda")
        mask = torch.zeros((keys.size + 63) // 64, dtype=torch.int64, device="cuda")
        d_keys = to_dev(keys)
        _lib.call("nve_table_find", self.table, self.ctx, keys.size, vp(d_keys), vp(mask), 128, vp(out), None)
        m = mask.cpu().numpy().view(np.uint64)
        hits = np.array([(int(m[i >> 6]) >> (i & 63)) & 1 for i in range(keys.size)], bool)
        return out.cpu().numpy(), hits

    def close(self):
        _lib.call("nve_context_wait", self.ctx)
        _lib.call("nve_context_destroy", self.ctx)
        _lib.call("nve_table_destroy", self.table)


def rows_for(n):
    """Row i holds float32 i * 1000 + j (gpu_table_test.cpp:488-494)."""
    v = np.arange(n)[:, None] * 1000.0 + np.arange(32)[None, :]
    return v.astype(np.float32).view(np.uint8)


def max_key(key_bytes):
    return (1 << 63) - 1 if key_bytes == 8 else (1 << 31) - 1


@pytest.mark.parametrize("key_bytes", [8, 4])
def test_custom_sentinel_fills_the_empty_ways(key_bytes):
    t = SentinelTable(key_bytes, 12345)
    tags = gpu_state(t)[0]
    assert np.all(tags == 12345)
    t.close()


@pytest.mark.parametrize("modify_on_gpu", [True, False])
@pytest.mark.parametrize("key_bytes", [8, 4])
def test_valid_keys_survive_a_batch_holding_the_sentinel(key_bytes, modify_on_gpu):
    sent = max_key(key_bytes)
    t = SentinelTable(key_bytes, sent, modify_on_gpu)
    kdt = np.int64 if key_bytes == 8 else np.int32
    keys = np.array([101, 202, sent, 404], kdt)
    vals = rows_for(4)
    t.insert(keys, vals)
    got, hits = t.find(keys)
    for i in (0, 1, 3):
        assert hits[i], i
        assert np.array_equal(got[i], vals[i])
    tags = gpu_state(t)[0]
    assert np.array_equal(tags, t.model.tags())
    t.close()


@pytest.mark.parametrize("modify_on_gpu", [True, False])
@pytest.mark.parametrize("key_bytes", [8, 4])
def test_minus_one_round_trips_when_the_sentinel_is_custom(key_bytes, modify_on_gpu):
    t = SentinelTable(key_bytes, max_key(key_bytes), modify_on_gpu)
    kdt = np.int64 if key_bytes == 8 else np.int32
    keys = np.array([101, -1, 303], kdt)
    vals = rows_for(3)
    t.insert(keys, vals)
    got, hits = t.find(keys)
    assert hits.all()
    assert np.array_equal(got, vals)
    tags = gpu_state(t)[0]
    assert np.array_equal(tags, t.model.tags())
    assert t.model.find_way(-1) >= 0
    t.close()


def guarded_table(key_bytes, num_rows, guard=8):
    """A GpuTable over a pinned host buffer of num_rows + guard float32 rows
    (value = its index), with uvm_num_rows = num_rows."""
    h = torch.arange((num_rows + guard) * 32, dtype=torch.float32).pin_memory()
    L = _lib.load()
    cfg = L.nve_gpu_table_config_default()
    cfg.cache_size = 1 << 20
    cfg.row_size_in_bytes = 128
    cfg.value_dtype = _lib.DT_F32
    cfg.uvm_table = h.data_ptr()
    cfg.uvm_num_rows = num_rows
    cfg.uvm_cpu_accumulate = 1
    table = ctypes.c_void_p()
    kt = _lib.KEY_INT64 if key_bytes == 8 else _lib.KEY_INT32
    _lib.call("nve_gpu_table_create", ctypes.byref(table), kt, ctypes.byref(cfg), None)
    ctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_table_create_execution_context", table, ctypes.byref(ctx), s, s, None, None)
    return h, table, ctx


@pytest.mark.parametrize("key_bytes,accumulate,num_keys", [(8, False, 64), (4, False, 64), (8, True, 64),
                                                           (8, True, 16 * 512), (4, True, 16 * 512)])
def test_update_and_accumulate_leave_rows_past_the_table_alone(key_bytes, accumulate, num_keys):
    rows = num_keys
    h, table, ctx = guarded_table(key_bytes, rows)
    kdt = np.int64 if key_bytes == 8 else np.int32
    i = np.arange(num_keys)
    keys = i.copy()
    keys[i % 7 == 1] = -(i[i % 7 == 1] + 1)
    keys[i % 7 == 3] = rows + (i[i % 7 == 3] % 8)
    keys = keys.astype(kdt)
    upd = (1000.0 + i[:, None] + np.arange(32)[None, :]).astype(np.float32)
    ref = h.numpy().reshape(rows + 8, 32).copy()
    inr = (keys >= 0) & (keys < rows)
    if accumulate:
        ref[keys[inr].astype(np.int64)] += upd[inr]
    else:
        ref[keys[inr].astype(np.int64)] = upd[inr]
    d_keys, d_upd = to_dev(keys), to_dev(upd.reshape(-1))
    if accumulate:
        _lib.call("nve_table_update_accumulate", table, ctx, num_keys, vp(d_keys), 128, 128, vp(d_upd),
                  _lib.DT_F32)
    else:
        _lib.call("nve_table_update", table, ctx, num_keys, vp(d_keys), 128, 128, vp(d_upd))
    _lib.call("nve_context_wait", ctx)
    torch.cuda.synchronize()
    got = h.numpy().reshape(rows + 8, 32)
    assert np.array_equal(got[rows:], ref[rows:]), "a guard row past the table was written"
    assert np.array_equal(got, ref)
    _lib.call("nve_context_destroy", ctx)
    _lib.call("nve_table_destroy", table)


def test_backing_table_without_a_row_count_is_rejected():
    """gpu_table_test.cpp:767-775: without uvm_num_rows every key would be out of range."""
    buf = torch.zeros(64 * 32, dtype=torch.float32).pin_memory()
    L = _lib.load()
    cfg = L.nve_gpu_table_config_default()
    cfg.cache_size = 1 << 20
    cfg.row_size_in_bytes = 128
    cfg.value_dtype = _lib.DT_F32
    cfg.uvm_table = buf.data_ptr()
    cfg.uvm_num_rows = 0
    t = ctypes.c_void_p()
    st = L.nve_gpu_table_create(ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(cfg), None)
    assert st != _lib.SUCCESS
    assert "uvm_num_rows" in _lib.last_error()

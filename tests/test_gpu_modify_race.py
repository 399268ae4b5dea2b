"""Lookups racing modifies on one table (the property the reference's insert
protocol exists for, ec_set_associative_device_modify.cuh:225-288,428-446,
tested there by tests/embedding_layer/uvm_layer_test.cpp:1091-1240).

A lookup thread reads every key's row on its own stream while a second thread
inserts or updates through another execution context of the same table.  Each
row is 256 words, all equal to (key << 8 | version): version 0 is the backing
row, each modify writes a new version.  Every row a lookup returns must be one
whole version of its own key -- never words of two versions or of two keys,
which is what a lookup reading a way while an insert copies over it returns.

The cache is small (64 sets) and each insert brings 1024 of 4096 keys, so
nearly every insert evicts rows that concurrent lookups resolved a moment
before; the inserts also run against a 2048-set cache, where they take the
hashed histogram."""
import ctypes
import threading

import numpy as np
import pytest

from nve_helpers import to_dev, vp
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

# Device buffers passed to the library are bound to names for the length of
# each call: a temporary tensor inside `vp(to_dev(...))` is freed as soon as
# vp returns, and its block can be handed to the next argument.

NK = 4096
WORDS = 256  # 1 KiB rows
PER_SET = 2144 - 8 * 256 + 8 * WORDS * 4  # tags + rows + counters per set (int64 keys)


def rows_of(keys, version):
    return ((keys.astype(np.uint32) << 8) | np.uint32(version))[:, None].repeat(WORDS, axis=1)


def check_rows(out, keys, max_version):
    """Every row whole (one word repeated), of its own key, a known version."""
    assert np.all(out == out[:, :1]), "a lookup returned a row mixing two versions"
    w = out[:, 0]
    assert np.array_equal(w >> 8, keys.astype(np.uint32)), "a lookup returned another key's row"
    assert np.all((w & 0xFF) <= max_version)
    return w & 0xFF


class RaceTable:
    def __init__(self, sets=64):
        self.backing = torch.from_numpy(rows_of(np.arange(NK), 0).reshape(-1).view(np.uint8).copy()).pin_memory()
        L = _lib.load()
        cfg = L.nve_gpu_table_config_default()
        cfg.cache_size = sets * PER_SET
        cfg.row_size_in_bytes = WORDS * 4
        cfg.value_dtype = _lib.DT_F32
        cfg.uvm_table = self.backing.data_ptr()
        cfg.uvm_num_rows = NK
        self.table = ctypes.c_void_p()
        _lib.call("nve_gpu_table_create", ctypes.byref(self.table), _lib.KEY_INT64, ctypes.byref(cfg), None)
        self.s_lookup = torch.cuda.Stream()
        self.s_modify = torch.cuda.Stream()
        self.ctx_lookup = self.context(self.s_lookup)
        self.ctx_modify = self.context(self.s_modify)

    def context(self, s):
        ctx = ctypes.c_void_p()
        p = ctypes.c_void_p(s.cuda_stream)
        _lib.call("nve_table_create_execution_context", self.table, ctypes.byref(ctx), p, p, None, None)
        return ctx

    def close(self):
        for c in (self.ctx_lookup, self.ctx_modify):
            _lib.call("nve_context_wait", c)
            _lib.call("nve_context_destroy", c)
        _lib.call("nve_table_destroy", self.table)


def run_race(modify_step, lookup, rounds=40, min_overlapped=5):
    """modify_step(i) runs on a second thread `rounds` times; lookup() runs on
    this thread until then and returns each time the versions it saw."""
    done = threading.Event()
    errors = []

    def modifier():
        try:
            torch.cuda.set_device(0)
            for i in range(rounds):
                modify_step(i)
        except Exception as e:  # noqa: BLE001 -- reported on the main thread
            errors.append(e)
        finally:
            done.set()

    t = threading.Thread(target=modifier)
    t.start()
    overlapped, seen = 0, set()
    try:
        while not done.is_set():
            seen |= set(np.unique(lookup()).tolist())
            overlapped += 1
    finally:
        t.join()
    assert not errors, errors
    seen |= set(np.unique(lookup()).tolist())  # after the last modify
    assert overlapped >= min_overlapped, f"only {overlapped} lookups overlapped the modifies"
    return seen


@pytest.mark.parametrize("sets", [64, 2048])
def test_table_find_racing_inserts(sets):
    """64 sets: the insert's sorted histogram; 2048 sets (more sets than the
    1024 keys of an insert): its hashed histogram."""
    rt = RaceTable(sets)
    rng = np.random.default_rng(5)
    keys = np.arange(NK, dtype=np.int64)
    d_keys = to_dev(keys)
    out = torch.zeros((NK, WORDS), dtype=torch.int32, device="cuda")

    def insert(i):
        pick = np.sort(rng.choice(NK, size=1024, replace=False)).astype(np.int64)
        d_pick, d_vals = to_dev(pick), to_dev(rows_of(pick, 1 + i).view(np.int32))  # alive for the call
        _lib.call("nve_table_insert", rt.table, rt.ctx_modify, pick.size, vp(d_pick), WORDS * 4, WORDS * 4,
                  vp(d_vals))

    def lookup():
        _lib.call("nve_table_find", rt.table, rt.ctx_lookup, NK, vp(d_keys), None, WORDS * 4, vp(out), None)
        rt.s_lookup.synchronize()
        return check_rows(out.cpu().numpy().view(np.uint32), keys, 40)

    seen = run_race(insert, lookup)
    assert 0 in seen and len(seen) > 2  # backing rows and inserted versions both read
    rt.close()


def test_table_find_racing_updates():
    """update rewrites the backing row and the resident cache row of each key:
    lookups see the old version or the new one, whole."""
    rt = RaceTable()
    rng = np.random.default_rng(6)
    keys = np.arange(NK, dtype=np.int64)
    d_keys = to_dev(keys)
    out = torch.zeros((NK, WORDS), dtype=torch.int32, device="cuda")
    # some rows resident first, so that updates hit cache rows as well
    first = np.arange(0, NK, 3, dtype=np.int64)[:1024]
    d_first, d_rows = to_dev(first), to_dev(rows_of(first, 0).view(np.int32))
    _lib.call("nve_table_insert", rt.table, rt.ctx_modify, first.size, vp(d_first), WORDS * 4, WORDS * 4,
              vp(d_rows))
    rt.s_modify.synchronize()

    def update(i):
        pick = np.sort(rng.choice(NK, size=1024, replace=False)).astype(np.int64)
        d_pick, d_vals = to_dev(pick), to_dev(rows_of(pick, 1 + i).view(np.int32))
        _lib.call("nve_table_update", rt.table, rt.ctx_modify, pick.size, vp(d_pick), WORDS * 4, WORDS * 4,
                  vp(d_vals))

    def lookup():
        _lib.call("nve_table_find", rt.table, rt.ctx_lookup, NK, vp(d_keys), None, WORDS * 4, vp(out), None)
        rt.s_lookup.synchronize()
        return check_rows(out.cpu().numpy().view(np.uint32), keys, 40)

    seen = run_race(update, lookup)
    assert len(seen) > 2
    rt.close()


def test_uvm_layer_lookup_racing_layer_inserts():
    """The same through a LinearUVM layer: one layer context looks up, another
    inserts (layer insert with values, table 0)."""
    rt = RaceTable()
    L = _lib.load()
    lc = L.nve_linear_uvm_layer_config_default()
    layer = ctypes.c_void_p()
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), rt.table, None)
    ctxs = []
    for s in (rt.s_lookup, rt.s_modify):
        c = ctypes.c_void_p()
        p = ctypes.c_void_p(s.cuda_stream)
        _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(c), p, p, None, None)
        ctxs.append(c)
    lctx, mctx = ctxs
    rng = np.random.default_rng(7)
    keys = np.arange(NK, dtype=np.int64)
    d_keys = to_dev(keys)
    out = torch.zeros((NK, WORDS), dtype=torch.int32, device="cuda")

    def insert(i):
        pick = np.sort(rng.choice(NK, size=1024, replace=False)).astype(np.int64)
        d_pick, d_vals = to_dev(pick), to_dev(rows_of(pick, 1 + i).view(np.int32))
        _lib.call("nve_layer_insert", layer, mctx, pick.size, vp(d_pick), WORDS * 4, WORDS * 4, vp(d_vals), 0)

    def lookup():
        _lib.call("nve_layer_lookup", layer, lctx, NK, vp(d_keys), vp(out), WORDS * 4, None, None)
        rt.s_lookup.synchronize()
        return check_rows(out.cpu().numpy().view(np.uint32), keys, 40)

    seen = run_race(insert, lookup)
    assert 0 in seen and len(seen) > 2
    for c in ctxs:
        _lib.call("nve_context_wait", c)
        _lib.call("nve_context_destroy", c)
    _lib.call("nve_layer_destroy", layer)
    rt.close()


def test_gpu_layer_lookup_racing_updates():
    """GPU layer (linear table in HBM): lookups on one context, updates of the
    table through another; rows old or new, whole."""
    table = to_dev(rows_of(np.arange(NK), 0).view(np.int32))
    L = _lib.load()
    cfg = L.nve_gpu_embedding_layer_config_default()
    cfg.layer_name = b"race"
    cfg.embedding_table = table.data_ptr()
    cfg.num_embeddings = NK
    cfg.embedding_width_in_bytes = WORDS * 4
    cfg.value_dtype = _lib.DT_F32
    layer = ctypes.c_void_p()
    _lib.call("nve_gpu_embedding_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(cfg), None)
    s_l, s_m = torch.cuda.Stream(), torch.cuda.Stream()
    ctxs = []
    for s in (s_l, s_m):
        c = ctypes.c_void_p()
        p = ctypes.c_void_p(s.cuda_stream)
        _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(c), p, p, None, None)
        ctxs.append(c)
    lctx, mctx = ctxs
    rng = np.random.default_rng(8)
    keys = np.arange(NK, dtype=np.int64)
    d_keys = to_dev(keys)
    out = torch.zeros((NK, WORDS), dtype=torch.int32, device="cuda")

    def update(i):
        pick = np.sort(rng.choice(NK, size=1024, replace=False)).astype(np.int64)
        d_pick, d_vals = to_dev(pick), to_dev(rows_of(pick, 1 + i).view(np.int32))
        _lib.call("nve_layer_update", layer, mctx, pick.size, vp(d_pick), WORDS * 4, WORDS * 4, vp(d_vals), 0)

    def lookup():
        _lib.call("nve_layer_lookup", layer, lctx, NK, vp(d_keys), vp(out), WORDS * 4, None, None)
        s_l.synchronize()
        return check_rows(out.cpu().numpy().view(np.uint32), keys, 40)

    seen = run_race(update, lookup)
    assert len(seen) > 2
    for c in ctxs:
        _lib.call("nve_context_wait", c)
        _lib.call("nve_context_destroy", c)
    _lib.call("nve_layer_destroy", layer)


def test_context_streams_are_registered_and_released():
    """Contexts add their lookup stream to the table's registry and remove it
    when destroyed: a modify after the lookup context is gone runs alone."""
    rt = RaceTable()
    keys = np.arange(64, dtype=np.int64)
    _lib.call("nve_context_wait", rt.ctx_lookup)
    _lib.call("nve_context_destroy", rt.ctx_lookup)
    d_keys, d_rows = to_dev(keys), to_dev(rows_of(keys, 3).view(np.int32))
    _lib.call("nve_table_insert", rt.table, rt.ctx_modify, keys.size, vp(d_keys), WORDS * 4, WORDS * 4, vp(d_rows))
    out = torch.zeros((keys.size, WORDS), dtype=torch.int32, device="cuda")
    _lib.call("nve_table_find", rt.table, rt.ctx_modify, keys.size, vp(d_keys), None, WORDS * 4, vp(out), None)
    rt.s_modify.synchronize()
    v = check_rows(out.cpu().numpy().view(np.uint32), keys, 3)
    assert np.all(v == 3)
    _lib.call("nve_context_wait", rt.ctx_modify)
    _lib.call("nve_context_destroy", rt.ctx_modify)
    _lib.call("nve_table_destroy", rt.table)

"""GPU parity of the lookup modes over a host-resident backing table
(get_kernel_mode, gpu_table.cu:271-287): LookupUVM, SortGather
(ec_set_associative.cuh:966-1057) and PipelineGather (pipeline_gather.cuh:203-412)
write the same rows -- each key's cache row on a hit, its backing row on a
miss, nothing for a key outside the table -- and count the same misses.
Checked against the oracle's cache model and across modes, bytewise."""
import ctypes

import numpy as np
import pytest

from nve_helpers import float_table, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib
from test_gpu_cache_lookup import CachedTable, warm

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

LOOKUP, SORT, PIPE = 1, 2, 3


def run_find(ct, keys, dim4, fill=0x5A):
    out = torch.full((keys.size, dim4), fill, dtype=torch.uint8, device="cuda")
    d_keys = to_dev(keys)
    _lib.call("nve_table_reset_lookup_counter", ct.table, ct.ctx)
    _lib.call("nve_table_find", ct.table, ct.ctx, keys.size, vp(d_keys), None, dim4, vp(out), None)
    cnt = ctypes.c_int64()
    _lib.call("nve_table_get_lookup_counter", ct.table, ct.ctx, ctypes.byref(cnt))
    return out.cpu().numpy(), cnt.value


def expected(ct, keys, dim4, fill=0x5A):
    """Cache slot on a hit, backing row on a miss, untouched for a key outside
    the table.  Hits come from the model's hit mask: the address the model
    gives a key outside the table lies past the backing array and can fall
    inside the model's cache array, so an address range cannot tell them apart."""
    rows_ptr, hits, misses = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
    data = ct.model.data().reshape(-1)
    base_d, base_u = data.ctypes.data, ct.uvm_np.ctypes.data
    exp = np.full((keys.size, dim4), fill, np.uint8)
    for i in range(keys.size):
        p = int(rows_ptr[i])
        if (int(hits[i >> 6]) >> (i & 63)) & 1:
            assert base_d <= p < base_d + data.nbytes
            exp[i] = data[p - base_d:p - base_d + dim4]
        elif 0 <= int(keys[i]) < ct.rows:
            exp[i] = ct.uvm_np.reshape(-1)[p - base_u:p - base_u + dim4]
    return exp, misses


@pytest.mark.parametrize("key_bytes", [8, 4])
@pytest.mark.parametrize("n", [3000, 70000])
def test_modes_write_the_same_rows(key_bytes, n):
    rng = np.random.default_rng(60 + n + key_bytes)
    rows, dim = 50000, 32
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    kdt = np.int64 if key_bytes == 8 else np.int32
    keys = rng.integers(0, rows, size=n).astype(kdt)
    keys[: n // 3] = rng.integers(0, 4000, size=n // 3)  # mostly cached
    keys[rng.random(n) < 0.01] = rows + 5                # outside the table
    keys[rng.random(n) < 0.01] = -3
    params = (ctypes.c_uint64 * 2)(97, 4)  # PipelineGather: 97 keys per host task
    outs = {}
    for mode, value in ((LOOKUP, 0), (SORT, 0), (PIPE, ctypes.addressof(params)), (0, 1000)):
        ct = CachedTable(uvm, 512 * 1024, key_bytes, kernel_mode_type=mode, kernel_mode_value=value)
        rng2 = np.random.default_rng(7)
        warm(ct, rng2, 6000, np.arange(0, 4000))
        got, misses = run_find(ct, keys, dim * 4)
        exp, exp_misses = expected(ct, keys, dim * 4)
        if not np.array_equal(got, exp):
            bad = np.nonzero(np.any(got != exp, axis=1))[0]
            rows_ptr, _, _ = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
            data = ct.model.data().reshape(-1)
            kind = ["cache" if data.ctypes.data <= int(rows_ptr[i]) < data.ctypes.data + data.nbytes
                    else ("backing" if 0 <= int(keys[i]) < rows else "none") for i in bad[:8]]
            first = bad[0]
            cols = np.nonzero(got[first] != exp[first])[0]
            pytest.fail(f"mode {mode}: {bad.size} rows differ, first {bad[:8].tolist()} keys "
                        f"{keys[bad[:8]].tolist()} expected from {kind}; row {first} differs in "
                        f"bytes {cols[:16].tolist()} (got {got[first][cols[:8]].tolist()}, "
                        f"expected {exp[first][cols[:8]].tolist()})")
        assert misses == exp_misses, f"mode {mode}"
        outs[mode] = got
        ct.close()
    assert all(np.array_equal(outs[LOOKUP], o) for o in outs.values())


def test_pipeline_default_params_and_all_misses():
    rng = np.random.default_rng(61)
    rows, dim = 20000, 64
    uvm = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    ct = CachedTable(uvm, 256 * 1024, 8, value_dtype=_lib.DT_F16, kernel_mode_type=PIPE)
    keys = rng.integers(0, rows, size=5000).astype(np.int64)  # empty cache: every key misses
    got, misses = run_find(ct, keys, dim * 2)
    assert misses == keys.size
    assert np.array_equal(got, uvm[keys])
    ct.close()


def test_unknown_kernel_mode_is_not_implemented_at_the_lookup():
    """c_api_boundary_test.cpp:103-131: a table with an unknown
    kernel_mode_type is created, and its first lookup over the backing table
    reports NVE_ERROR_NOT_IMPLEMENTED (get_kernel_mode, gpu_table.cu:271-287);
    a table without a backing table never asks for a mode."""
    L = _lib.load()
    h_uvm = torch.zeros(16 * 16, dtype=torch.float32).pin_memory()
    for with_uvm in (True, False):
        cfg = L.nve_gpu_table_config_default()
        cfg.cache_size, cfg.row_size_in_bytes, cfg.value_dtype = 1 << 20, 64, _lib.DT_F32
        cfg.kernel_mode_type = 99
        if with_uvm:
            cfg.uvm_table, cfg.uvm_num_rows = h_uvm.data_ptr(), 16
        t = ctypes.c_void_p()
        _lib.call("nve_gpu_table_create", ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(cfg), None)
        ctx = ctypes.c_void_p()
        s = stream_ptr()
        _lib.call("nve_table_create_execution_context", t, ctypes.byref(ctx), s, s, None, None)
        keys = torch.zeros(1, dtype=torch.int64, device="cuda")
        out = torch.zeros(64, dtype=torch.uint8, device="cuda")
        mask = torch.zeros(1, dtype=torch.int64, device="cuda")
        st = L.nve_table_find(t, ctx, 1, vp(keys), vp(mask), 64, vp(out), None)
        if with_uvm:
            assert st == _lib.NOT_IMPLEMENTED, _lib.last_error()
            assert "kernel_mode_type" in _lib.last_error()
        else:
            assert st == _lib.SUCCESS
            assert int(mask.cpu()[0]) == 0  # an empty cache: a miss
        torch.cuda.synchronize()
        _lib.call("nve_context_destroy", ctx)
        _lib.call("nve_table_destroy", t)


@pytest.mark.parametrize("mode", [LOOKUP, SORT, PIPE])
@pytest.mark.parametrize("key_bytes", [4, 8])
@pytest.mark.parametrize("modify_on_gpu", [False, True])
def test_mode_boundaries_empty_all_misses_all_hits(mode, key_bytes, modify_on_gpu):
    """pipeline_gather_boundary_tests.cu:147-205 for every lookup mode: an empty
    lookup writes nothing and counts nothing, 500 keys of an empty cache all
    miss and read the backing rows, and 32 inserted keys all hit.  The
    backing row of key i holds bytes (i + j) % 256; the inserted rows hold
    their complement, so a hit is seen to come from the cache."""
    rows, width = 100000, 32
    uvm = ((np.arange(rows)[:, None] + np.arange(width)[None, :]) % 256).astype(np.uint8)
    params = (ctypes.c_uint64 * 2)(4096, 4)
    ct = CachedTable(uvm, 1 << 20, key_bytes, value_dtype=_lib.DT_F32, kernel_mode_type=mode,
                     kernel_mode_value=ctypes.addressof(params) if mode == PIPE else 0,
                     modify_on_gpu=modify_on_gpu)
    kdt = np.int64 if key_bytes == 8 else np.int32
    empty = torch.zeros(1, dtype=torch.int64 if key_bytes == 8 else torch.int32, device="cuda")
    out = torch.full((1, width), 0x5A, dtype=torch.uint8, device="cuda")
    _lib.call("nve_table_reset_lookup_counter", ct.table, ct.ctx)
    _lib.call("nve_table_find", ct.table, ct.ctx, 0, vp(empty), None, width, vp(out), None)
    cnt = ctypes.c_int64()
    _lib.call("nve_table_get_lookup_counter", ct.table, ct.ctx, ctypes.byref(cnt))
    assert cnt.value == 0 and bool((out == 0x5A).all())

    keys = np.arange(500, dtype=kdt)
    got, misses = run_find(ct, keys, width)
    assert misses == 500
    assert np.array_equal(got, uvm[:500])

    hot = np.arange(32, dtype=kdt)
    from test_gpu_cache_insert import table_insert
    table_insert(ct, hot, ~uvm[:32], width)
    got, misses = run_find(ct, hot, width)
    assert misses == 0
    assert np.array_equal(got, ~uvm[:32])
    ct.close()

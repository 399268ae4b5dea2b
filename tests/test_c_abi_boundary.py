"""Conventions of the table C ABI at its edges, after the reference's
tests/c_api/c_api_boundary_test.cpp: keys is required once n > 0 (with the
reference's message, nve_c_api_tables.cpp:97-99 and the same check in insert,
update, update_accumulate and erase), getters reject a NULL out, hit_mask /
values / value_sizes of find are each optional, the lookup counter restarts
at 0 and a host table counts the keys it resolved, a GPU table's calls with
n = 0 are no-ops (gpu_table.cu:249,382,421,499,584,688,1057), and a HIP
failure is reported as NVE_ERROR_CUDA.

The LinearHostTable cases run on the CPU; the GpuTable ones are marked gpu."""
import ctypes

import numpy as np
import pytest

from pynve import _lib

ROWS = 16


def p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


@pytest.fixture
def host_table():
    """A LinearHostTable of 16 int64 rows (row i holds 10 * i) and a context."""
    L = _lib.load()
    data = (np.arange(ROWS, dtype=np.int64) * 10).reshape(ROWS, 1)
    tc = L.nve_host_table_config_default()
    tc.key_size = 8
    tc.max_value_size = 8
    tc.value_dtype = _lib.DT_F32  # two fp32 values per row; finds copy the row's bytes
    t, ctx = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("nve_amd_linear_host_table_create", ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(tc), p(data),
              ROWS, 0)
    _lib.call("nve_table_create_execution_context", t, ctypes.byref(ctx), None, None, None, None)
    yield t, ctx, data
    _lib.call("nve_context_destroy", ctx)
    _lib.call("nve_table_destroy", t)


def null_key_calls(L, t, ctx):
    one = np.ones(1, np.int64)
    upd = np.ones(1, np.float64)
    return {
        "find": lambda: L.nve_table_find(t, ctx, 1, None, None, 8, p(one), None),
        "insert": lambda: L.nve_table_insert(t, ctx, 1, None, 8, 8, p(one)),
        "update": lambda: L.nve_table_update(t, ctx, 1, None, 8, 8, p(one)),
        "update_accumulate": lambda: L.nve_table_update_accumulate(t, ctx, 1, None, 8, 8, p(upd), _lib.DT_F64),
        "erase": lambda: L.nve_table_erase(t, ctx, 1, None),
    }


def check_null_keys(t, ctx):
    for name, call in null_key_calls(_lib.load(), t, ctx).items():
        assert call() == _lib.INVALID_ARGUMENT, name
        assert _lib.last_error() == "keys must not be NULL when n > 0", name


def check_null_outs(t, ctx):
    L = _lib.load()
    assert L.nve_table_get_device_id(t, None) == _lib.INVALID_ARGUMENT
    assert L.nve_table_get_max_row_size(t, None) == _lib.INVALID_ARGUMENT
    assert L.nve_table_get_key_size(t, None) == _lib.INVALID_ARGUMENT
    assert L.nve_table_get_lookup_counter(t, ctx, None) == _lib.INVALID_ARGUMENT


def test_host_table_null_keys_with_positive_count_are_rejected(host_table):
    t, ctx, _ = host_table
    check_null_keys(t, ctx)


def test_host_table_getters_reject_null_out(host_table):
    t, ctx, _ = host_table
    check_null_outs(t, ctx)


def test_host_table_find_optional_arguments(host_table):
    """c_api_boundary_test.cpp:187-239 on a LinearHostTable: hit_mask and
    value_sizes may each be NULL; values may not, as the reference's linear
    host table checks them ("Invalid values", linear_host_table.hpp:86)."""
    t, ctx, data = host_table
    L = _lib.load()
    key = np.array([7], np.int64)
    out = np.full(1, -1, np.int64)
    sizes = np.full(1, -1, np.int64)
    mask = np.zeros(1, np.uint64)
    _lib.check(L.nve_table_find(t, ctx, 1, p(key), None, 8, p(out), p(sizes)))
    assert out[0] == data[7, 0]
    out[0] = -1
    _lib.check(L.nve_table_find(t, ctx, 1, p(key), p(mask), 8, p(out), None))
    assert out[0] == data[7, 0] and int(mask[0]) & 1 == 1
    assert L.nve_table_find(t, ctx, 1, p(key), p(mask), 8, None, None) != _lib.SUCCESS
    assert "Invalid values" in _lib.last_error()


def test_host_table_lookup_counter_counts_resolved_keys_after_reset(host_table):
    """c_api_boundary_test.cpp:259-290: reset reads 0; finding 3 present keys
    adds 3; keys past the table resolve nothing and add nothing."""
    t, ctx, _ = host_table
    L = _lib.load()
    _lib.check(L.nve_table_reset_lookup_counter(t, ctx))
    cnt = ctypes.c_int64(-1)
    _lib.check(L.nve_table_get_lookup_counter(t, ctx, ctypes.byref(cnt)))
    assert cnt.value == 0
    keys = np.array([1, 2, 3], np.int64)
    out = np.zeros(3, np.int64)
    mask = np.zeros(1, np.uint64)
    _lib.check(L.nve_table_find(t, ctx, 3, p(keys), p(mask), 8, p(out), None))
    _lib.check(L.nve_table_get_lookup_counter(t, ctx, ctypes.byref(cnt)))
    assert cnt.value == 3 and int(mask[0]) & 7 == 7
    missing = np.array([100, 200], np.int64)
    mask[0] = 0
    _lib.check(L.nve_table_find(t, ctx, 2, p(missing), p(mask), 8, p(out), None))
    _lib.check(L.nve_table_get_lookup_counter(t, ctx, ctypes.byref(cnt)))
    assert cnt.value == 3 and int(mask[0]) & 3 == 0


# ---------------------------------------------------------------------------
# GpuTable
# ---------------------------------------------------------------------------
@pytest.fixture
def gpu_table():
    torch = pytest.importorskip("torch")
    L = _lib.load()
    cfg = L.nve_gpu_table_config_default()
    cfg.cache_size = 1 << 20
    cfg.row_size_in_bytes = 8
    cfg.value_dtype = _lib.DT_F32
    t, ctx = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("nve_gpu_table_create", ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(cfg), None)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.call("nve_table_create_execution_context", t, ctypes.byref(ctx), s, s, None, None)
    yield t, ctx
    _lib.call("nve_context_wait", ctx)
    _lib.call("nve_context_destroy", ctx)
    _lib.call("nve_table_destroy", t)


@pytest.mark.gpu
def test_gpu_table_null_keys_and_null_outs(gpu_table):
    t, ctx = gpu_table
    check_null_keys(t, ctx)
    check_null_outs(t, ctx)


@pytest.mark.gpu
def test_gpu_table_zero_keys_are_no_ops(gpu_table):
    """c_api_boundary_test.cpp:139-154 on a GPU table: n = 0 with NULL buffers
    succeeds and changes nothing."""
    t, ctx = gpu_table
    L = _lib.load()
    assert L.nve_table_find(t, ctx, 0, None, None, 8, None, None) == _lib.SUCCESS
    assert L.nve_table_insert(t, ctx, 0, None, 8, 8, None) == _lib.SUCCESS
    assert L.nve_table_update(t, ctx, 0, None, 8, 8, None) == _lib.SUCCESS
    assert L.nve_table_update_accumulate(t, ctx, 0, None, 8, 8, None, _lib.DT_F32) == _lib.SUCCESS
    assert L.nve_table_erase(t, ctx, 0, None) == _lib.SUCCESS
    _lib.check(L.nve_context_wait(ctx))


@pytest.mark.gpu
def test_gpu_table_find_optional_arguments(gpu_table):
    """hit_mask and values each optional on a GPU table (values NULL: an
    existence check through the hit mask)."""
    t, ctx = gpu_table
    L = _lib.load()
    key = np.array([7], np.int64)
    val = np.array([700.0])
    _lib.check(L.nve_table_insert(t, ctx, 1, p(key), 8, 8, p(val)))
    _lib.check(L.nve_context_wait(ctx))
    out = np.full(1, -1.0)
    sizes = np.full(1, -1, np.int64)
    mask = np.zeros(1, np.uint64)
    # a GPU table has no per-row sizes to report (gpu_table.cu:380)
    assert L.nve_table_find(t, ctx, 1, p(key), None, 8, p(out), p(sizes)) == _lib.RUNTIME
    assert "value_sizes must be nullptr for GPU table" in _lib.last_error()
    _lib.check(L.nve_table_find(t, ctx, 1, p(key), None, 8, p(out), None))
    assert out[0] == 700.0
    _lib.check(L.nve_table_find(t, ctx, 1, p(key), p(mask), 8, None, None))
    assert int(mask[0]) & 1 == 1
    out[0], mask[0] = -1.0, 0
    _lib.check(L.nve_table_find(t, ctx, 1, p(key), p(mask), 8, p(out), None))
    assert out[0] == 700.0 and int(mask[0]) & 1 == 1


@pytest.mark.gpu
def test_hip_failure_is_reported_as_cuda_error():
    """c_api_boundary_test.cpp:81-101: a table on a device that does not exist
    fails with NVE_ERROR_CUDA (the HIP error) wherever the first HIP call is."""
    L = _lib.load()
    cfg = L.nve_gpu_table_config_default()
    cfg.device_id = 1000
    cfg.cache_size = 1 << 20
    cfg.row_size_in_bytes = 64
    cfg.value_dtype = _lib.DT_F32
    t, ctx = ctypes.c_void_p(), ctypes.c_void_p()
    st = L.nve_gpu_table_create(ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(cfg), None)
    if st == _lib.SUCCESS:
        st = L.nve_table_create_execution_context(t, ctypes.byref(ctx), None, None, None, None)
    if st == _lib.SUCCESS:
        st = L.nve_table_clear(t, ctx)
    assert st == _lib.HIP_ERROR, _lib.last_error()
    if ctx.value:
        L.nve_context_destroy(ctx)
    if t.value:
        L.nve_table_destroy(t)
    # the failed call leaves nothing behind for the next table's launches
    cfg.device_id = 0
    _lib.call("nve_gpu_table_create", ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(cfg), None)
    _lib.call("nve_table_destroy", t)

"""The C ABI's basic, thread-pool and handle-lifecycle conventions, after the
reference's tests/c_api/c_api_basic_test.cpp, c_api_threadpool_test.cpp and
c_api_handle_lifecycle_test.cpp: version calls reject NULL outs with a
message, the last error is always a valid string, a malformed thread-pool
JSON is an error status (not a crash) and the JSON is read as JSON, NULL
pools / outs / tables are invalid arguments, the default pool cannot be
reconfigured once used, and a failed factory create leaves its out handle
NULL.  Everything here runs on the CPU."""
import ctypes

import numpy as np
import pytest

from pynve import _lib


def last_error_is_set():
    msg = ctypes.c_char_p()
    assert _lib.load().nve_get_last_error(ctypes.byref(msg)) == _lib.SUCCESS
    return msg.value is not None and msg.value != b""


def test_version_and_abi_version_reject_null_outs():
    L = _lib.load()
    a, b, c = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    assert L.nve_version(None, None, None) == _lib.INVALID_ARGUMENT
    assert last_error_is_set()
    assert L.nve_abi_version(None, None) == _lib.INVALID_ARGUMENT
    assert L.nve_abi_version(ctypes.byref(a), None) == _lib.INVALID_ARGUMENT
    assert L.nve_abi_version(None, ctypes.byref(b)) == _lib.INVALID_ARGUMENT
    assert last_error_is_set()
    assert L.nve_version(ctypes.byref(a), ctypes.byref(b), ctypes.byref(c)) == _lib.SUCCESS


def test_last_error_is_a_valid_string_on_a_fresh_thread():
    """c_api_basic_test.cpp:57-61: a thread that made no failing call still
    gets a non-NULL (empty) message."""
    import threading
    got = {}

    def run():
        msg = ctypes.c_char_p()
        got["st"] = _lib.load().nve_get_last_error(ctypes.byref(msg))
        got["msg"] = msg.value

    t = threading.Thread(target=run)
    t.start()
    t.join()
    assert got["st"] == _lib.SUCCESS and got["msg"] == b""


def test_thread_pool_malformed_json_and_null_arguments():
    L = _lib.load()
    pool = ctypes.c_void_p()
    assert L.nve_thread_pool_create(ctypes.byref(pool), b"{not valid json") != _lib.SUCCESS
    n = ctypes.c_int64(-1)
    assert L.nve_thread_pool_num_workers(None, ctypes.byref(n)) == _lib.INVALID_ARGUMENT
    _lib.call("nve_thread_pool_create", ctypes.byref(pool), b'{"name": "simple", "num_workers": 1}')
    assert L.nve_thread_pool_num_workers(pool, None) == _lib.INVALID_ARGUMENT
    _lib.call("nve_thread_pool_destroy", pool)


def test_default_pool_cannot_be_reconfigured_once_used():
    """c_api_threadpool_test.cpp:87-106: a context made with thread_pool NULL
    materializes the process-wide default pool; configuring it afterwards
    fails."""
    L = _lib.load()
    data = np.zeros((4, 2), np.float32)
    tc = L.nve_host_table_config_default()
    tc.key_size, tc.max_value_size, tc.value_dtype = 8, 8, _lib.DT_F32
    t, ctx = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("nve_amd_linear_host_table_create", ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(tc),
              ctypes.c_void_p(data.ctypes.data), 4, 0)
    _lib.call("nve_table_create_execution_context", t, ctypes.byref(ctx), None, None, None, None)
    assert L.nve_configure_default_thread_pool(b'{"name": "simple", "num_workers": 2}') != _lib.SUCCESS
    assert last_error_is_set()
    _lib.call("nve_context_destroy", ctx)
    _lib.call("nve_table_destroy", t)


def test_null_table_is_rejected_by_every_table_call():
    """c_api_handle_lifecycle_test.cpp:57-88,134-147."""
    L = _lib.load()
    ctx = ctypes.c_void_p()
    k = np.zeros(1, np.int64)
    kp = ctypes.c_void_p(k.ctypes.data)
    assert L.nve_table_find(None, None, 1, kp, None, 8, kp, None) == _lib.INVALID_ARGUMENT
    assert L.nve_table_insert(None, None, 1, kp, 8, 8, kp) == _lib.INVALID_ARGUMENT
    assert L.nve_table_update(None, None, 1, kp, 8, 8, kp) == _lib.INVALID_ARGUMENT
    assert L.nve_table_update_accumulate(None, None, 1, kp, 8, 8, kp, _lib.DT_F32) == _lib.INVALID_ARGUMENT
    assert L.nve_table_clear(None, None) == _lib.INVALID_ARGUMENT
    assert L.nve_table_erase(None, None, 1, kp) == _lib.INVALID_ARGUMENT
    assert L.nve_table_create_execution_context(None, ctypes.byref(ctx), None, None, None,
                                                None) == _lib.INVALID_ARGUMENT
    data = np.zeros((4, 2), np.float32)
    tc = L.nve_host_table_config_default()
    tc.key_size, tc.max_value_size, tc.value_dtype = 8, 8, _lib.DT_F32
    t = ctypes.c_void_p()
    _lib.call("nve_amd_linear_host_table_create", ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(tc),
              ctypes.c_void_p(data.ctypes.data), 4, 0)
    assert L.nve_table_create_execution_context(t, None, None, None, None, None) == _lib.INVALID_ARGUMENT
    _lib.call("nve_table_destroy", t)


def test_failed_factory_create_leaves_its_out_handle_null():
    """c_api_handle_lifecycle_test.cpp:153-159 (nve_c_api_tables.cpp:313): *out
    is reset before a failure returns, so a caller never sees a stale handle."""
    L = _lib.load()
    out = ctypes.c_void_p(1)
    assert L.nve_create_table_factory(ctypes.byref(out), b"nonexistent_plugin_xyz.so", b"{}") != _lib.SUCCESS
    assert out.value is None


def test_thread_pool_json_is_parsed_as_json():
    """thread_pool.cpp:57-109: the configuration is parsed as JSON (a parse
    error fails the call, NULL is an invalid argument), fields come from the
    top-level object only, "implementation" names "simple" or "numa"."""
    L = _lib.load()
    pool = ctypes.c_void_p()
    n = ctypes.c_int64()
    assert L.nve_thread_pool_create(ctypes.byref(pool), None) == _lib.INVALID_ARGUMENT
    for bad in (b"", b"{", b'{"num_workers": 2,}', b'{"num_workers": 02}', b'{"a": "\\x"}', b"{} {}",
                b'{"num_workers": 2', b"[1, 2", b'{"a": tru}'):
        assert L.nve_thread_pool_create(ctypes.byref(pool), bad) == _lib.RUNTIME, bad
        assert "Malformed JSON" in _lib.last_error(), bad
    for good, want in ((b'{"num_workers": 2}', 2), (b' {"name": "x", "num_workers": 3} ', 3),
                       (b'{"cfg": {"num_workers": 9}, "num_workers": 1}', 1),
                       (b'{"name": "num_workers \\" 7", "num_workers": 4}', 4),
                       (b'{"implementation": "numa", "num_workers": 2, "x": [1, -2.5e3, null, true]}', 2)):
        _lib.call("nve_thread_pool_create", ctypes.byref(pool), good)
        _lib.call("nve_thread_pool_num_workers", pool, ctypes.byref(n))
        assert n.value == want, good
        _lib.call("nve_thread_pool_destroy", pool)
    assert L.nve_thread_pool_create(ctypes.byref(pool), b'{"implementation": "other"}') == _lib.RUNTIME
    assert "Thread pool implementation 'other' not found!" in _lib.last_error()
    assert L.nve_thread_pool_create(ctypes.byref(pool), b'{"num_workers": 1.5}') == _lib.INVALID_ARGUMENT
    assert L.nve_thread_pool_create(ctypes.byref(pool), b'{"num_workers": -1}') == _lib.INVALID_ARGUMENT

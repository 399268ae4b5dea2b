"""CPU tests of the C-ABI library: it loads without a GPU, exports every symbol
the headers declare, and keeps the reference's defaults, versions and
argument-error behaviour (tests/c_api/c_api_basic_test.cpp,
c_api_boundary_test.cpp).  No compute call is made here."""
import ctypes
import os
import re

import pytest

from pynve import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in ("nve_c_api.h", "nve_amd_ext.h")]


def declared_symbols():
    names = []
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"NVE_C_API\s+[\w\s\*]+?\b(nve_\w+)\s*\(", text)
    return names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 58
    for n in names:
        assert hasattr(lib, n), n
    # the ctypes table covers the header exactly
    assert set(names) == set(_lib.SIGNATURES)


def test_reference_enum_values_are_kept():
    text = open(HEADERS[0]).read()
    for name, val in [("NVE_SUCCESS", 0), ("NVE_ERROR_INVALID_ARGUMENT", 1), ("NVE_ERROR_CUDA", 2),
                      ("NVE_ERROR_RUNTIME", 3), ("NVE_ERROR_NOT_IMPLEMENTED", 4),
                      ("NVE_ERROR_OUT_OF_MEMORY", 5), ("NVE_DTYPE_FLOAT16", 3),
                      ("NVE_DTYPE_QUINT8_ROWWISE_F16", 10)]:
        assert re.search(rf"{name}\s*=\s*{val}\b", text), name


def test_versions():
    a, b, c = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    _lib.call("nve_abi_version", ctypes.byref(a), ctypes.byref(b))
    assert (a.value, b.value) == (1, 0)
    _lib.call("nve_version", ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    assert (a.value, b.value, c.value) == (26, 9, 0)
    assert _lib.load().nve_version(None, None, None) == _lib.INVALID_ARGUMENT


def test_config_defaults_match_reference():
    L = _lib.load()
    t = L.nve_gpu_table_config_default()  # nve_c_api_util.cpp:49-68
    assert (t.device_id, t.cache_size, t.row_size_in_bytes, t.uvm_table, t.uvm_num_rows) == (0, 0, 0, None, 0)
    assert (t.count_misses, t.max_modify_size, t.value_dtype) == (1, 1 << 20, 0)
    assert (t.disable_uvm_update, t.uvm_cpu_accumulate, t.data_storage_on_host, t.modify_on_gpu) == (0, 1, 0, 1)
    assert (t.kernel_mode_type, t.kernel_mode_value, t.invalid_key) == (0, 0, -1)
    g = L.nve_gpu_embedding_layer_config_default()
    assert (g.embedding_table, g.num_embeddings, g.value_dtype, g.default_row_index) == (None, 0, 0, -1)
    u = L.nve_linear_uvm_layer_config_default()
    assert (u.insert_heuristic, u.min_insert_freq_gpu, u.min_insert_size_gpu, u.default_row_index) == (None, 0, 65536, -1)
    h = L.nve_hierarchical_layer_config_default()
    assert (h.min_insert_size_gpu, h.min_insert_size_host, h.default_embedding_size) == (65536, 0, 0)
    o = L.nve_overflow_policy_config_default()
    assert (o.overflow_margin, o.handler, o.resolution_margin) == (2**63 - 1 - 1023, 0, 0.8)
    ht = L.nve_host_table_config_default()
    assert (ht.key_size, ht.max_value_size, ht.value_dtype, ht.invalid_key) == (8, 8, 0, -1)


def test_null_handles_are_invalid_argument_with_message():
    L = _lib.load()
    assert L.nve_layer_lookup(None, None, 0, None, None, 0, None, None) == _lib.INVALID_ARGUMENT
    assert "must not be NULL" in _lib.last_error()
    assert L.nve_layer_lookup_pooled(None, None, 0, None, None, 0, None, 1, 0, None, 0, 1, None, 0, 1,
                                     None) == _lib.INVALID_ARGUMENT
    assert L.nve_table_find(None, None, 0, None, None, 0, None, None) == _lib.INVALID_ARGUMENT
    assert L.nve_context_wait(None) == _lib.INVALID_ARGUMENT
    assert L.nve_gpu_table_create(None, 1, None, None) == _lib.INVALID_ARGUMENT
    assert L.nve_layer_destroy(None) == _lib.INVALID_ARGUMENT
    assert L.nve_table_destroy(None) == _lib.INVALID_ARGUMENT


def test_out_of_scope_entries_link_and_report_not_implemented():
    L = _lib.load()
    out = ctypes.c_void_p()
    assert L.nve_create_table_factory(ctypes.byref(out), b"libx.so", b"{}") == _lib.NOT_IMPLEMENTED
    assert out.value is None
    cfg = L.nve_hierarchical_layer_config_default()
    assert L.nve_hierarchical_layer_create(ctypes.byref(out), 1, ctypes.byref(cfg), None, 0,
                                           None) == _lib.NOT_IMPLEMENTED


def test_thread_pool_and_heuristics_lifecycle():
    L = _lib.load()
    pool = ctypes.c_void_p()
    _lib.call("nve_thread_pool_create", ctypes.byref(pool), b'{"name": "t", "num_workers": 3}')
    n = ctypes.c_int64()
    _lib.call("nve_thread_pool_num_workers", pool, ctypes.byref(n))
    assert n.value == 3
    _lib.call("nve_thread_pool_destroy", pool)
    _lib.call("nve_thread_pool_create", ctypes.byref(pool), b"{}")
    _lib.call("nve_thread_pool_num_workers", pool, ctypes.byref(n))
    assert n.value == max((os.cpu_count() or 1) - 2, 1)  # thread_pool.cpp:112-116
    _lib.call("nve_thread_pool_destroy", pool)
    h = ctypes.c_void_p()
    _lib.call("nve_heuristic_create_never", ctypes.byref(h))
    _lib.call("nve_heuristic_destroy", h)
    th = (ctypes.c_float * 2)(0.5, 0.9)
    _lib.call("nve_heuristic_create_default", ctypes.byref(h), th, 2)
    _lib.call("nve_heuristic_destroy", h)
    bad = (ctypes.c_float * 1)(1.5)
    assert L.nve_heuristic_create_default(ctypes.byref(h), bad, 1) == _lib.INVALID_ARGUMENT
    with pytest.raises(_lib.InvalidArgument):
        _lib.call("nve_heuristic_create_default", ctypes.byref(h), None, 3)

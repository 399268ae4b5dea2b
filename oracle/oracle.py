"""ctypes view of the CPU oracle (oracle/nve_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker / CPU baseline.  The product
library never loads it.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")

F32, F16, QI8_F32, QI8_F16, QU8_F32, QU8_F16, XI8A_F32, XE4M3_F32 = 1, 3, 7, 8, 9, 10, 32, 33
CONCAT, SUM, MEAN, WSUM, WMEAN = 0, 1, 2, 3, 4
FIXED, CSR = 0, 1

_lib = None


def build():
    subprocess.check_call(["make", "-s", "-C", _HERE])


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


P = ctypes.c_void_p
I64 = ctypes.c_int64
U64 = ctypes.c_uint64
I32 = ctypes.c_int


class OrcCache(ctypes.Structure):
    _fields_ = [
        ("num_sets", ctypes.c_uint64),
        ("row_bytes", ctypes.c_int64),
        ("key_bytes", ctypes.c_int),
        ("sentinel", ctypes.c_int64),
        ("decay_rate", ctypes.c_float),
        ("global_ts", ctypes.c_int64),
        ("data", ctypes.c_void_p),
        ("tags", ctypes.c_void_p),
        ("counters", ctypes.c_void_p),
        ("set_ts", ctypes.c_void_p),
        ("host_modify", ctypes.c_int),
    ]


def _declare(L):
    L.orc_f16_to_f32.restype = ctypes.c_float
    L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_f32_to_f16.restype = ctypes.c_uint16
    L.orc_f32_to_f16.argtypes = [ctypes.c_float]
    L.orc_e4m3_to_f32.restype = ctypes.c_float
    L.orc_e4m3_to_f32.argtypes = [ctypes.c_uint8]
    L.orc_f16_to_f32_n.argtypes = [P, P, I64]
    L.orc_f32_to_f16_n.argtypes = [P, P, I64]
    L.orc_sanitize_keys.argtypes = [P, P, I64, I32, U64, I64]
    L.orc_gather.restype = I64
    L.orc_gather.argtypes = [P, I32, I64, P, P, U64, I64, P, I64]
    L.orc_dequant_row.argtypes = [P, I32, I64, I32, P]
    L.orc_pool.argtypes = [P, I32, I64, I32, I32, I64, P, I32, I64, I64, P, I32, I32, P, I64]
    L.orc_pool_host.argtypes = L.orc_pool.argtypes
    L.orc_convert_host.argtypes = [P, I32, I64, I32, P]
    L.orc_linear_rows.argtypes = [P, I32, I64, P, I64, P]
    L.orc_host_layer_lookup.argtypes = [P, I32, I64, P, U64, I64, I32, I32, I32, P, I64, I64, P,
                                        I32, I32, P, P, I64, I32]
    L.orc_cache_num_sets.restype = U64
    L.orc_cache_num_sets.argtypes = [U64, I64, I32]
    L.orc_cache_init.restype = I32
    L.orc_cache_init.argtypes = [ctypes.POINTER(OrcCache), U64, I64, I32, I64]
    L.orc_cache_free.argtypes = [ctypes.POINTER(OrcCache)]
    L.orc_cache_num_sets_host.restype = U64
    L.orc_cache_num_sets_host.argtypes = [U64, I64, I32]
    L.orc_cache_init_ex.restype = I32
    L.orc_cache_init_ex.argtypes = [ctypes.POINTER(OrcCache), U64, I64, I32, I64, I32]
    L.orc_cache_clear.argtypes = [ctypes.POINTER(OrcCache)]
    L.orc_histogram_host.restype = I64
    L.orc_histogram_host.argtypes = [P, I32, I64, P, P, P]
    L.orc_cache_insert_host.restype = I64
    L.orc_cache_insert_host.argtypes = [ctypes.POINTER(OrcCache), P, P, P, I64, I64, P, P]
    L.orc_pooling_backprop.restype = I64
    L.orc_pooling_backprop.argtypes = [P, I32, I64, I32, I32, P, I64, I64, P, I32, P, I32, I64, I64, P, P]
    L.orc_cache_insert_keys_host.restype = I64
    L.orc_cache_insert_keys_host.argtypes = [ctypes.POINTER(OrcCache), P, I64, P, U64, P, I64, I64]
    L.orc_cache_set.restype = ctypes.c_uint32
    L.orc_cache_set.argtypes = [ctypes.POINTER(OrcCache), I64]
    L.orc_cache_tag.restype = I64
    L.orc_cache_tag.argtypes = [ctypes.POINTER(OrcCache), I64]
    L.orc_cache_key_of.restype = I64
    L.orc_cache_key_of.argtypes = [ctypes.POINTER(OrcCache), I64, ctypes.c_uint32]
    L.orc_cache_find_way.restype = I32
    L.orc_cache_find_way.argtypes = [ctypes.POINTER(OrcCache), I64]
    L.orc_cache_resolve.restype = I64
    L.orc_cache_resolve.argtypes = [ctypes.POINTER(OrcCache), P, I64, P, P, P]
    L.orc_histogram.restype = I64
    L.orc_histogram.argtypes = [P, I32, I64, P, P, P]
    L.orc_cache_insert_hist.restype = I64
    L.orc_cache_insert_hist.argtypes = [ctypes.POINTER(OrcCache), P, P, P, I64, P, P]
    L.orc_cache_insert_keys.restype = I64
    L.orc_cache_insert_keys.argtypes = [ctypes.POINTER(OrcCache), P, I64, P, U64, P, I64, I64]
    L.orc_cache_erase.restype = I64
    L.orc_cache_erase.argtypes = [ctypes.POINTER(OrcCache), P, I64]
    L.orc_dedup.restype = I64
    L.orc_dedup.argtypes = [P, I32, I64, P, P, P, P]
    L.orc_power_law.argtypes = [P, I64, ctypes.c_double, ctypes.c_double, ctypes.c_double, P]


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def f16_to_f32(bits):
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, np.float32)
    lib().orc_f16_to_f32_n(_p(bits), _p(out), bits.size)
    return out


def f32_to_f16(vals):
    vals = np.ascontiguousarray(vals, dtype=np.float32)
    out = np.empty(vals.shape, np.uint16)
    lib().orc_f32_to_f16_n(_p(vals), _p(out), vals.size)
    return out


def e4m3_to_f32(code):
    return lib().orc_e4m3_to_f32(int(code))


def meta_bytes(dtype):
    return {QI8_F32: 4, QI8_F16: 2, QU8_F32: 8, QU8_F16: 4, XI8A_F32: 8, XE4M3_F32: 4}.get(dtype, 0)


def value_bytes(dtype):
    return {F32: 4, F16: 2}.get(dtype, 1)


def native_out(dtype):
    return F16 if dtype in (F16, QI8_F16, QU8_F16) else F32


def out_np_dtype(out_dtype):
    return np.uint16 if out_dtype == F16 else np.float32


def sanitize(keys, num_rows, default_row):
    keys = np.ascontiguousarray(keys)
    out = np.empty_like(keys)
    lib().orc_sanitize_keys(_p(keys), _p(out), keys.size, keys.itemsize, num_rows, default_row)
    return out


def gather(keys, table_bytes, row_bytes, num_rows, hit_mask=None, out=None):
    """table_bytes: uint8 array (num_rows*row_bytes). Returns (out, hits)."""
    keys = np.ascontiguousarray(keys)
    n = keys.size
    if out is None:
        out = np.zeros((n, row_bytes), np.uint8)
    hits = lib().orc_gather(_p(keys), keys.itemsize, n, _p(hit_mask), _p(table_bytes), num_rows,
                            row_bytes, _p(out), row_bytes)
    return out, hits


def dequant_rows(rows_bytes, dtype, count, out_dtype):
    """rows_bytes: (n, row_bytes) uint8. Returns (n, count) in out dtype (f16 as uint16 bits)."""
    rows_bytes = np.ascontiguousarray(rows_bytes, dtype=np.uint8)
    n = rows_bytes.shape[0]
    out = np.empty((n, count), out_np_dtype(out_dtype))
    L = lib()
    for i in range(n):
        L.orc_dequant_row(_p(rows_bytes[i]), dtype, count, out_dtype, _p(out[i]))
    return out


def convert_rows_host(rows_bytes, dtype, count, out_dtype):
    """CPU HostLayer Concatenate to out_dtype of (n, row_bytes) stored rows."""
    rows_bytes = np.ascontiguousarray(rows_bytes, dtype=np.uint8)
    n = rows_bytes.shape[0]
    out = np.empty((n, count), out_np_dtype(out_dtype))
    L = lib()
    for i in range(n):
        L.orc_convert_host(_p(rows_bytes[i]), dtype, count, out_dtype, _p(out[i]))
    return out


def _row_ptrs(base_arr, idx_rows, row_bytes):
    base = base_arr.ctypes.data
    ptrs = (np.asarray(idx_rows, np.uint64) * np.uint64(row_bytes) + np.uint64(base)).astype(np.uint64)
    return ptrs


def pool(row_ptrs, dtype, count, sparse, pooling, num_keys, offsets, num_bags, hotness, weights,
         weight_dtype, out_dtype, host_order=False, key_bytes=8):
    """row_ptrs: uint64 array of absolute addresses (keep the backing arrays alive)."""
    row_ptrs = np.ascontiguousarray(row_ptrs, np.uint64)
    out = np.zeros((num_bags, count), out_np_dtype(out_dtype))
    if offsets is not None:
        offsets = np.ascontiguousarray(offsets)
        key_bytes = offsets.itemsize
    if weights is not None:
        weights = np.ascontiguousarray(weights)
    fn = lib().orc_pool_host if host_order else lib().orc_pool
    fn(_p(row_ptrs), dtype, count, sparse, pooling, num_keys, _p(offsets), key_bytes, num_bags,
       hotness, _p(weights), weight_dtype, out_dtype, _p(out), out.strides[0] if num_bags else 0)
    return out


def linear_row_ptrs(keys, table_bytes, row_bytes):
    keys = np.ascontiguousarray(keys).astype(np.int64)
    return (keys.astype(np.uint64) * np.uint64(row_bytes) + np.uint64(table_bytes.ctypes.data)).astype(np.uint64)


def host_layer_lookup(keys, table_bytes, num_rows, row_bytes, dtype, pooling, sparse, offsets,
                      num_bags, hotness, weights, weight_dtype, out_dtype, threads):
    keys = np.ascontiguousarray(keys)
    n = keys.size
    meta = meta_bytes(dtype)
    count = (row_bytes - meta) // value_bytes(dtype)
    if pooling == CONCAT:
        out = np.zeros((n, row_bytes), np.uint8)
        gbuf = None
        stride = row_bytes
    else:
        out = np.zeros((num_bags, count), out_np_dtype(out_dtype))
        gbuf = np.empty((n, row_bytes), np.uint8)
        stride = out.strides[0]
    if offsets is not None:
        offsets = np.ascontiguousarray(offsets)
    if weights is not None:
        weights = np.ascontiguousarray(weights)
    lib().orc_host_layer_lookup(_p(keys), keys.itemsize, n, _p(table_bytes), num_rows, row_bytes,
                                dtype, pooling, sparse, _p(offsets), num_bags, hotness,
                                _p(weights), weight_dtype, out_dtype, _p(gbuf), _p(out), stride,
                                threads)
    return out


class Cache:
    """Model of the 8-way set-associative GPU cache: EmbedCacheSA<K,K> with the
    device-modify policy, or with the host-metadata policy (modify_on_gpu =
    false) when host_modify is set."""

    def __init__(self, cache_bytes, row_bytes, key_bytes=8, sentinel=-1, host_modify=False):
        self.c = OrcCache()
        self.host_modify = bool(host_modify)
        rc = lib().orc_cache_init_ex(ctypes.byref(self.c), cache_bytes, row_bytes, key_bytes, sentinel,
                                     1 if host_modify else 0)
        if rc != 0:
            raise ValueError("cache too small")
        self.row_bytes = row_bytes
        self.key_bytes = key_bytes
        self.kdt = np.int32 if key_bytes == 4 else np.int64

    def __del__(self):
        try:
            lib().orc_cache_free(ctypes.byref(self.c))
        except Exception:
            pass

    @property
    def num_sets(self):
        return self.c.num_sets

    def tags(self):
        n = self.c.num_sets * 8
        return np.ctypeslib.as_array(ctypes.cast(self.c.tags, ctypes.POINTER(ctypes.c_int64)), (n,)).copy()

    def counters(self):
        n = self.c.num_sets * 8
        return np.ctypeslib.as_array(ctypes.cast(self.c.counters, ctypes.POINTER(ctypes.c_float)), (n,)).copy()

    def set_ts(self):
        n = self.c.num_sets
        return np.ctypeslib.as_array(ctypes.cast(self.c.set_ts, ctypes.POINTER(ctypes.c_int64)), (n,)).copy()

    def data(self):
        n = self.c.num_sets * 8 * self.row_bytes
        return np.ctypeslib.as_array(ctypes.cast(self.c.data, ctypes.POINTER(ctypes.c_uint8)), (n,))

    def set_of(self, key):
        return lib().orc_cache_set(ctypes.byref(self.c), int(key))

    def tag_of(self, key):
        return lib().orc_cache_tag(ctypes.byref(self.c), int(key))

    def key_of(self, tag, s):
        return lib().orc_cache_key_of(ctypes.byref(self.c), int(tag), int(s))

    def find_way(self, key):
        return lib().orc_cache_find_way(ctypes.byref(self.c), int(key))

    def resolve(self, keys, uvm):
        keys = np.ascontiguousarray(keys, self.kdt)
        n = keys.size
        rows = np.zeros(n, np.uint64)
        hits = np.zeros((n + 63) // 64, np.uint64)
        misses = lib().orc_cache_resolve(ctypes.byref(self.c), _p(keys), n, _p(uvm), _p(rows), _p(hits))
        return rows, hits, misses

    def insert_keys(self, keys, uvm=None, values=None, value_stride=0, max_modify_size=1 << 20):
        """GpuTable::insert / insert_from_uvm with this cache's policy; uvm is
        the backing table's bytes (its row count = uvm.size / row_bytes)."""
        keys = np.ascontiguousarray(keys, self.kdt)
        uvm_rows = 0 if uvm is None else np.asarray(uvm).nbytes // self.row_bytes
        fn = lib().orc_cache_insert_keys_host if self.host_modify else lib().orc_cache_insert_keys
        return fn(ctypes.byref(self.c), _p(keys), keys.size, _p(uvm), uvm_rows, _p(values), value_stride,
                  max_modify_size)

    def insert_hist_host(self, ukeys, priority, src_ptrs=None, max_update=1 << 20):
        """The host-metadata policy over an already-built histogram; returns
        the (set, way) records."""
        ukeys = np.ascontiguousarray(ukeys, np.int64)
        priority = np.ascontiguousarray(priority, np.float32)
        m = ukeys.size
        if src_ptrs is not None:
            src_ptrs = np.ascontiguousarray(src_ptrs, np.uint64)
        s = np.zeros(max(m, 1), np.int64)
        w = np.zeros(max(m, 1), np.int64)
        n = lib().orc_cache_insert_host(ctypes.byref(self.c), _p(ukeys), _p(priority), _p(src_ptrs), m,
                                        max_update, _p(s), _p(w))
        return s[:n], w[:n]

    def clear(self):
        lib().orc_cache_clear(ctypes.byref(self.c))

    def insert_hist(self, ukeys, priority, src_ptrs):
        ukeys = np.ascontiguousarray(ukeys, np.int64)
        priority = np.ascontiguousarray(priority, np.float32)
        src_ptrs = np.ascontiguousarray(src_ptrs, np.uint64)
        m = ukeys.size
        s = np.zeros(2 * m + 8, np.int64)
        w = np.zeros(2 * m + 8, np.int64)
        n = lib().orc_cache_insert_hist(ctypes.byref(self.c), _p(ukeys), _p(priority), _p(src_ptrs), m,
                                        _p(s), _p(w))
        return s[:n], w[:n]

    def erase(self, keys):
        keys = np.ascontiguousarray(keys, self.kdt)
        return lib().orc_cache_erase(ctypes.byref(self.c), _p(keys), keys.size)


def cache_num_sets(cache_bytes, row_bytes, key_bytes=8, host_modify=False):
    if host_modify:
        return lib().orc_cache_num_sets_host(cache_bytes, row_bytes, key_bytes)
    return lib().orc_cache_num_sets(cache_bytes, row_bytes, key_bytes)


def histogram_host(keys):
    """CPU DefaultHistogram order (first occurrence, stable by count desc)."""
    keys = np.ascontiguousarray(keys)
    n = keys.size
    uk = np.zeros(max(n, 1), np.int64)
    pr = np.zeros(max(n, 1), np.float32)
    fi = np.zeros(max(n, 1), np.int64)
    u = lib().orc_histogram_host(_p(keys), keys.itemsize, n, _p(uk), _p(pr), _p(fi))
    return uk[:u], pr[:u], fi[:u]


def histogram(keys):
    keys = np.ascontiguousarray(keys)
    n = keys.size
    uk = np.zeros(max(n, 1), np.int64)
    pr = np.zeros(max(n, 1), np.float32)
    fi = np.zeros(max(n, 1), np.int64)
    u = lib().orc_histogram(_p(keys), keys.itemsize, n, _p(uk), _p(pr), _p(fi))
    return uk[:u], pr[:u], fi[:u]


def dedup(keys):
    keys = np.ascontiguousarray(keys)
    n = keys.size
    uq = np.zeros(max(n, 1), np.int64)
    ct = np.zeros(max(n, 1), np.int64)
    inv = np.zeros(max(n, 1), np.int64)
    off = np.zeros(max(n, 1), np.int64)
    u = lib().orc_dedup(_p(keys), keys.itemsize, n, _p(uq), _p(ct), _p(inv), _p(off))
    return uq[:u], ct[:u], inv[:n], off[:u]


def power_law(x, min_v, max_v, alpha):
    x = np.ascontiguousarray(x, np.float64)
    out = np.empty(x.size, np.int64)
    lib().orc_power_law(_p(x), x.size, float(min_v), float(max_v), float(alpha), _p(out))
    return out


def pooling_backprop(keys, pooling, sparse, offsets, num_bags, hotness, weights, weight_dtype,
                     grads_in, grad_dtype, dim, block=32):
    """Sparse gradient (unique keys ascending, rows of grad_dtype bits) of a
    lookup, in the summation order documented in nve_oracle.h (pieces of
    `block`-aligned position blocks, eight sub-sequences per key)."""
    keys = np.ascontiguousarray(keys)
    n = keys.size
    if offsets is not None:
        offsets = np.ascontiguousarray(offsets, keys.dtype)
    if weights is not None:
        weights = np.ascontiguousarray(weights)
    grads_in = np.ascontiguousarray(grads_in)
    uq = np.zeros(max(n, 1), keys.dtype)
    out = np.zeros((max(n, 1), dim), np.uint16 if grad_dtype == F16 else np.float32)
    u = lib().orc_pooling_backprop(_p(keys), keys.itemsize, n, pooling, sparse, _p(offsets), num_bags,
                                   hotness, _p(weights), weight_dtype, _p(grads_in), grad_dtype, dim,
                                   block, _p(uq), _p(out))
    return uq[:u], out[:u]

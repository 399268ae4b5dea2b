"""The CPU HostLayer of libnve_amd.so (LinearHostTable + HostEmbeddingLayer)
through the C ABI, on host memory, without a GPU.

Checked against the oracle's restatement of the reference HostLayer
(host_embedding_layer.cpp:55-247, cpu_gather.hpp:28-80,
cpu_pooling.hpp:68-341), bit for bit: gathers, every pooling mode and row
format in the CPU order, Concatenate conversions, the default embedding for
missed keys, hit masks and counters, CSR contract errors, updates and
accumulates with repeated keys, and results that do not depend on the
number of worker threads.  Reference tests followed:
tests/embedding_layer/host_layer_test.cpp, cpu_ops tests
cpu_kernel_unit_tests.cpp:125-161 and cpu_pooling_unit_tests.cpp:268-518."""
import ctypes

import numpy as np
import pytest

from nve_helpers import csr_offsets, dyadic, quant_table
from oracle import oracle as O
from pynve import _lib

CDT = {O.F32: _lib.DT_F32, O.F16: _lib.DT_F16, O.QI8_F32: _lib.DT_QI8_F32, O.QI8_F16: 8,
       O.QU8_F32: 9, O.QU8_F16: _lib.DT_QU8_F16, O.XI8A_F32: _lib.DT_XI8A_F32,
       O.XE4M3_F32: _lib.DT_XE4M3_F32}


def p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


class HostLayer:
    """A LinearHostTable over `table_bytes` (rows x row_bytes uint8) and a
    host layer with one context."""

    def __init__(self, table_bytes, dtype, key_type=_lib.KEY_INT64, default_row=None, pool=None,
                 max_threads=0):
        L = _lib.load()
        self.table = np.ascontiguousarray(table_bytes)
        rows, width = self.table.shape
        tc = L.nve_host_table_config_default()
        tc.key_size = 4 if key_type == _lib.KEY_INT32 else 8
        tc.max_value_size = width
        tc.value_dtype = CDT[dtype]
        self.t, self.layer, self.ctx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        _lib.call("nve_amd_linear_host_table_create", ctypes.byref(self.t), key_type, ctypes.byref(tc),
                  p(self.table), rows, max_threads)
        lc = L.nve_host_embedding_layer_config_default()
        self._def = None
        if default_row is not None:
            self._def = np.ascontiguousarray(default_row, np.uint8)
            lc.default_embedding = self._def.ctypes.data
            lc.default_embedding_size = self._def.size
        _lib.call("nve_host_embedding_layer_create", ctypes.byref(self.layer), key_type, ctypes.byref(lc),
                  self.t, None)
        _lib.call("nve_layer_create_execution_context", self.layer, ctypes.byref(self.ctx), None, None, pool,
                  None)

    def lookup(self, keys, out, hitmask=None):
        hr = (ctypes.c_float * 1)()
        _lib.check(_lib.load().nve_layer_lookup(self.layer, self.ctx, keys.size, p(keys), p(out),
                                                out.strides[0] if out.ndim > 1 else out.itemsize,
                                                p(hitmask), hr))
        return hr[0]

    def pooled(self, keys, out, pooling, sparse, off=None, hot=0, w=None, wdt=0, odt=_lib.DT_F32):
        hr = (ctypes.c_float * 1)()
        _lib.check(_lib.load().nve_layer_lookup_pooled(
            self.layer, self.ctx, keys.size, p(keys), p(out), out.strides[0], None, pooling, sparse, p(off),
            0 if off is None else off.size, hot, p(w), wdt, odt, hr))
        return hr[0]

    def close(self):
        _lib.call("nve_context_destroy", self.ctx)
        _lib.call("nve_layer_destroy", self.layer)
        _lib.call("nve_table_destroy", self.t)


@pytest.fixture
def layers():
    made = []
    yield made
    for h in made:
        h.close()


def test_c1_workload_gather_and_fixed8_sum(layers):
    """BASELINE C1: 1,000,000 x 64 fp32 N(0, 0.01), 4,096 bags x 8 uniform keys."""
    rows, dim, bags, hot = 1_000_000, 64, 4096, 8
    rng = np.random.default_rng(0)
    table = rng.normal(0.0, 0.01, size=(rows, dim)).astype(np.float32)
    keys = np.random.default_rng(1).integers(0, rows, size=bags * hot).astype(np.int64)
    h = HostLayer(table.view(np.uint8), O.F32)
    layers.append(h)
    out = np.full((keys.size, dim), -1, np.float32)
    assert h.lookup(keys, out) == 1.0
    assert np.array_equal(out, table[keys])
    pooled = np.full((bags, dim), -1, np.float32)
    h.pooled(keys, pooled, _lib.POOL_SUM, _lib.SPARSE_FIXED, hot=hot)
    tb = table.view(np.uint8).reshape(-1)
    ref = O.pool(O.linear_row_ptrs(keys, tb, dim * 4), O.F32, dim, O.FIXED, O.SUM, keys.size, None, bags, hot,
                 None, 0, O.F32, host_order=True)
    assert np.array_equal(pooled.view(np.uint32), ref.view(np.uint32))
    # the oracle's threaded HostLayer restatement agrees too
    ref2 = O.host_layer_lookup(keys, tb, rows, dim * 4, O.F32, O.SUM, O.FIXED, None, bags, hot, None, 0,
                               O.F32, 4)
    assert np.array_equal(pooled.view(np.uint32), ref2.view(np.uint32))


FORMATS = [O.F32, O.F16, O.QI8_F32, O.QI8_F16, O.QU8_F32, O.QU8_F16, O.XI8A_F32, O.XE4M3_F32]


def table_of(rng, dtype, rows, count):
    if dtype == O.F32:
        return rng.normal(0, 1, size=(rows, count)).astype(np.float32).view(np.uint8)
    if dtype == O.F16:
        return rng.normal(0, 1, size=(rows, count)).astype(np.float16).view(np.uint8)
    return quant_table(rng, rows, count, dtype)


@pytest.mark.parametrize("dtype", FORMATS)
@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_MEAN, _lib.POOL_WSUM, _lib.POOL_WMEAN])
def test_pooling_every_format_matches_the_cpu_order(layers, dtype, pooling):
    rng = np.random.default_rng(100 * dtype + pooling)
    rows, count, bags = 3000, 56, 300
    tb = table_of(rng, dtype, rows, count)
    off = csr_offsets(rng, bags, 20)  # includes empty bags
    keys = rng.integers(0, rows, size=int(off[-1])).astype(np.int64)
    weighted = pooling in (_lib.POOL_WSUM, _lib.POOL_WMEAN)
    w = rng.uniform(0, 1, size=keys.size).astype(np.float32) if weighted else None
    h = HostLayer(tb, dtype)
    layers.append(h)
    for odt in (O.F32, O.F16):
        out = np.full((bags, count), 7, O.out_np_dtype(odt))
        h.pooled(keys, out, pooling, _lib.SPARSE_CSR, off=off, w=w, wdt=_lib.DT_F32 if weighted else 0,
                 odt=CDT[odt])
        flat = np.ascontiguousarray(tb).reshape(-1)
        ref = O.pool(O.linear_row_ptrs(keys, flat, tb.shape[1]), dtype, count, O.CSR, pooling, keys.size, off,
                     bags, 0, w, O.F32 if weighted else 0, odt, host_order=True)
        assert np.array_equal(out.view(np.uint8), ref.view(np.uint8)), f"out {odt}"


@pytest.mark.parametrize("dtype", FORMATS)
@pytest.mark.parametrize("odt", [O.F32, O.F16])
def test_concatenate_converts_or_dequantizes(layers, dtype, odt):
    rng = np.random.default_rng(7 * dtype + odt)
    rows, count = 500, 40
    tb = table_of(rng, dtype, rows, count)
    keys = rng.integers(0, rows, size=700).astype(np.int64)
    h = HostLayer(tb, dtype)
    layers.append(h)
    out = np.zeros((keys.size, count), O.out_np_dtype(odt))
    h.pooled(keys, out, _lib.POOL_CONCAT, 0, odt=CDT[odt])
    if CDT[odt] == CDT[dtype]:  # same-type Concatenate is the raw gather
        assert np.array_equal(out.view(np.uint8), tb[keys])
    else:
        assert np.array_equal(out, O.convert_rows_host(tb[keys], dtype, count, odt))


def test_fp16_fixed_and_weights_in_fp16(layers):
    rng = np.random.default_rng(5)
    rows, dim, bags, hot = 2000, 128, 64, 33
    tb = rng.normal(0, 0.02, size=(rows, dim)).astype(np.float16).view(np.uint8)
    keys = rng.integers(0, rows, size=bags * hot).astype(np.int64)
    w = rng.uniform(0, 2, size=keys.size).astype(np.float16)
    h = HostLayer(tb, O.F16)
    layers.append(h)
    out = np.zeros((bags, dim), np.uint16)
    h.pooled(keys, out, _lib.POOL_WMEAN, _lib.SPARSE_FIXED, hot=hot, w=w.view(np.uint16), wdt=_lib.DT_F16,
             odt=_lib.DT_F16)
    flat = np.ascontiguousarray(tb).reshape(-1)
    ref = O.pool(O.linear_row_ptrs(keys, flat, dim * 2), O.F16, dim, O.FIXED, O.WMEAN, keys.size, None, bags,
                 hot, w.view(np.uint16), O.F16, O.F16, host_order=True)
    assert np.array_equal(out, ref)


def test_int32_keys_and_offsets(layers):
    rng = np.random.default_rng(9)
    rows, dim, bags = 1000, 16, 90
    tb = dyadic(rng, (rows, dim)).astype(np.float32).view(np.uint8)
    off = csr_offsets(rng, bags, 9, np.int32)
    keys = rng.integers(0, rows, size=int(off[-1])).astype(np.int32)
    h = HostLayer(tb, O.F32, key_type=_lib.KEY_INT32)
    layers.append(h)
    out = np.zeros((bags, dim), np.float32)
    h.pooled(keys, out, _lib.POOL_SUM, _lib.SPARSE_CSR, off=off)
    flat = np.ascontiguousarray(tb).reshape(-1)
    ref = O.pool(O.linear_row_ptrs(keys, flat, dim * 4), O.F32, dim, O.CSR, O.SUM, keys.size, off, bags, 0,
                 None, 0, O.F32, host_order=True)
    assert np.array_equal(out, ref)
    # dyadic values: the sum is exact in any order
    want = np.zeros((bags, dim))
    tf = tb.view(np.float32)
    for b in range(bags):
        want[b] = tf[keys[off[b]:off[b + 1]]].astype(np.float64).sum(0)
    assert np.array_equal(out, want.astype(np.float32))


def test_missed_keys_default_row_hitmask_and_rate(layers):
    rng = np.random.default_rng(11)
    rows, dim = 100, 8
    table = rng.normal(0, 1, size=(rows, dim)).astype(np.float32)
    default = np.arange(dim, dtype=np.float32) + 0.5
    keys = np.array([3, -1, 99, 100, 7, 1 << 40, 0] * 20, np.int64)
    h = HostLayer(table.view(np.uint8), O.F32, default_row=default.view(np.uint8))
    layers.append(h)
    out = np.full((keys.size, dim), -9, np.float32)
    mask = np.full((keys.size + 63) // 64, 0xFFFF, np.uint64)  # the layer clears it first
    rate = h.lookup(keys, out, mask)
    hit = (keys >= 0) & (keys < rows)
    assert rate == pytest.approx(hit.mean())
    bits = np.array([(int(mask[i // 64]) >> (i % 64)) & 1 for i in range(keys.size)], bool)
    assert np.array_equal(bits, hit)
    assert np.array_equal(out[hit], table[keys[hit]])
    assert np.all(out[~hit] == default)
    # a pooled bag counts a missed key as the default row
    pooled = np.zeros((20, dim), np.float32)
    h.pooled(keys, pooled, _lib.POOL_SUM, _lib.SPARSE_FIXED, hot=7)
    want = (table[3] + default + table[99] + default + table[7] + default + table[0])
    assert np.allclose(pooled, want, rtol=1e-6)


def test_without_default_row_missed_rows_are_left_alone(layers):
    table = np.ones((10, 4), np.float32)
    keys = np.array([1, 50, 2], np.int64)
    h = HostLayer(table.view(np.uint8), O.F32)
    layers.append(h)
    out = np.full((3, 4), -3, np.float32)
    assert h.lookup(keys, out) == pytest.approx(2 / 3)
    assert np.all(out[1] == -3) and np.all(out[[0, 2]] == 1)


def test_empty_batch_zeroes_csr_bags(layers):
    table = np.ones((10, 4), np.float32)
    h = HostLayer(table.view(np.uint8), O.F32)
    layers.append(h)
    out = np.full((3, 4), 5, np.float32)
    off = np.zeros(4, np.int64)
    keys = np.zeros(0, np.int64)
    assert h.pooled(keys, out, _lib.POOL_MEAN, _lib.SPARSE_CSR, off=off) == 1.0
    assert np.all(out == 0)


def test_csr_contract_errors(layers):
    table = np.ones((10, 4), np.float32)
    h = HostLayer(table.view(np.uint8), O.F32)
    layers.append(h)
    keys = np.arange(6, dtype=np.int64)
    out = np.zeros((3, 4), np.float32)
    for off in ([1, 2, 4, 6], [0, 4, 2, 6], [0, 2, 4, 5]):
        with pytest.raises(_lib.InvalidArgument):
            h.pooled(keys, out, _lib.POOL_SUM, _lib.SPARSE_CSR, off=np.array(off, np.int64))
    with pytest.raises(_lib.InvalidArgument):  # 6 keys do not divide into bags of 4
        h.pooled(keys, out, _lib.POOL_SUM, _lib.SPARSE_FIXED, hot=4)
    with pytest.raises(_lib.InvalidArgument):  # weighted pooling without weights
        h.pooled(keys, out, _lib.POOL_WSUM, _lib.SPARSE_FIXED, hot=2)
    narrow = np.zeros((6, 3), np.float32)
    with pytest.raises(_lib.InvalidArgument):  # output rows narrower than a table row
        h.lookup(keys, narrow)


def test_results_do_not_depend_on_the_thread_count(layers):
    rng = np.random.default_rng(13)
    rows, dim, bags = 5000, 72, 700
    tb = rng.normal(0, 1, size=(rows, dim)).astype(np.float16).view(np.uint8)
    off = csr_offsets(rng, bags, 40)
    keys = rng.integers(0, rows, size=int(off[-1])).astype(np.int64)
    outs = []
    for workers in (1, 3, 8):
        pool = ctypes.c_void_p()
        _lib.call("nve_thread_pool_create", ctypes.byref(pool), f'{{"num_workers": {workers}}}'.encode())
        h = HostLayer(tb, O.F16, pool=pool)
        out = np.zeros((bags, dim), np.float32)
        h.pooled(keys, out, _lib.POOL_MEAN, _lib.SPARSE_CSR, off=off)
        g = np.zeros((keys.size, dim), np.uint16)
        h.lookup(keys, g)
        h.close()
        _lib.call("nve_thread_pool_destroy", pool)
        outs.append((out, g))
    for out, g in outs[1:]:
        assert np.array_equal(out, outs[0][0]) and np.array_equal(g, outs[0][1])


def test_table_api_find_counter_update_accumulate(layers):
    L = _lib.load()
    rows, dim = 64, 4
    table = np.zeros((rows, dim), np.float32)
    h = HostLayer(table.view(np.uint8), O.F32)
    layers.append(h)
    dev = ctypes.c_int32()
    _lib.call("nve_table_get_device_id", h.t, ctypes.byref(dev))
    assert dev.value == -1
    ctx = ctypes.c_void_p()
    _lib.call("nve_table_create_execution_context", h.t, ctypes.byref(ctx), None, None, None, None)
    try:
        # update: a repeated key takes its last value
        keys = np.array([5, 9, 5, 70], np.int64)
        vals = np.arange(16, dtype=np.float32).reshape(4, 4)
        _lib.call("nve_table_update", h.t, ctx, 4, p(keys), 16, 16, p(vals))
        assert np.array_equal(table[5], vals[2]) and np.array_equal(table[9], vals[1])
        # accumulate: every occurrence is added, in position order
        keys = np.array([1, 2, 1, 1] * 300, np.int64)
        ups = np.tile(np.array([[0.25] * 4, [1.0] * 4, [0.5] * 4, [0.125] * 4], np.float32), (300, 1))
        _lib.call("nve_table_update_accumulate", h.t, ctx, keys.size, p(keys), 16, 16, p(ups), _lib.DT_F32)
        assert np.all(table[1] == 300 * (0.25 + 0.5 + 0.125)) and np.all(table[2] == 300.0)
        # find skips keys whose hit bit is set; the counter counts found keys
        _lib.call("nve_table_reset_lookup_counter", h.t, ctx)
        keys = np.array([1, 2, 3, 99], np.int64)
        mask = np.array([0b0010], np.uint64)
        out = np.full((4, 4), -1, np.float32)
        _lib.call("nve_table_find", h.t, ctx, 4, p(keys), p(mask), 16, p(out), None)
        assert np.array_equal(out[0], table[1]) and np.all(out[1] == -1) and np.array_equal(out[2], table[3])
        assert int(mask[0]) == 0b0111
        cnt = ctypes.c_int64()
        _lib.call("nve_table_get_lookup_counter", h.t, ctx, ctypes.byref(cnt))
        assert cnt.value == 2
        # insert / erase / clear have no effect on a linear host table
        before = table.copy()
        _lib.call("nve_table_erase", h.t, ctx, 2, p(keys))
        _lib.call("nve_table_clear", h.t, ctx)
        assert np.array_equal(table, before)
    finally:
        _lib.call("nve_context_destroy", ctx)


def test_host_layer_needs_a_host_table():
    L = _lib.load()
    lc = L.nve_host_embedding_layer_config_default()
    out = ctypes.c_void_p()
    with pytest.raises(_lib.InvalidArgument):
        _lib.call("nve_host_embedding_layer_create", ctypes.byref(out), _lib.KEY_INT64, ctypes.byref(lc), None,
                  None)
    tc = L.nve_host_table_config_default()
    tc.key_size = 4  # does not match an int64 key type
    tc.max_value_size = 16
    tc.value_dtype = _lib.DT_F32
    buf = np.zeros(64, np.float32)
    t = ctypes.c_void_p()
    with pytest.raises(_lib.InvalidArgument):
        _lib.call("nve_amd_linear_host_table_create", ctypes.byref(t), _lib.KEY_INT64, ctypes.byref(tc), p(buf),
                  4, 0)

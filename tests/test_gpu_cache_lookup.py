"""GPU parity of the set-associative cache lookups (tag compare, set/tag math,
row layout, misses served from the host-linear backing table, miss counts)
against the oracle's cache model.

The cache content is produced by the oracle (its insert model) and loaded into
the GPU table with nve_amd_gpu_table_import_state plus a row copy, so these
tests pin the lookup side independently of the GPU insert.  Cases follow
tests/ecache/api_test.cu (lookup, UVM lookup, negative keys) and
tests/gpu_table/gpu_table_test.cpp (find with hit mask, find_uvm, combine)."""
import ctypes

import numpy as np
import pytest

from nve_helpers import (csr_offsets, float_table, hip_memcpy, pooled_f16_close, quant_table, rel_close,
                         stream_ptr, to_dev, vp)
from oracle import oracle as O
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


class CachedTable:
    """GPU table (+ optional pinned backing table) whose cache state is copied
    from an oracle cache model."""

    def __init__(self, uvm_bytes, cache_bytes, key_bytes=8, with_uvm=True, value_dtype=_lib.DT_F32,
                 kernel_mode_type=0, kernel_mode_value=0, modify_on_gpu=True, max_modify_size=None):
        self.rows, self.width = uvm_bytes.shape
        self.key_bytes = key_bytes
        self.uvm_np = np.ascontiguousarray(uvm_bytes)
        self.h_uvm = torch.from_numpy(self.uvm_np.reshape(-1).copy()).pin_memory() if with_uvm else None
        L = _lib.load()
        cfg = L.nve_gpu_table_config_default()
        cfg.cache_size = cache_bytes
        cfg.row_size_in_bytes = self.width
        cfg.value_dtype = value_dtype
        cfg.kernel_mode_type = kernel_mode_type
        cfg.kernel_mode_value = kernel_mode_value
        cfg.modify_on_gpu = 1 if modify_on_gpu else 0
        if max_modify_size is not None:
            cfg.max_modify_size = max_modify_size
        if with_uvm:
            cfg.uvm_table = self.h_uvm.data_ptr()
            cfg.uvm_num_rows = self.rows
        self.table = ctypes.c_void_p()
        kt = _lib.KEY_INT32 if key_bytes == 4 else _lib.KEY_INT64
        _lib.call("nve_gpu_table_create", ctypes.byref(self.table), kt, ctypes.byref(cfg), None)
        self.ctx = ctypes.c_void_p()
        s = stream_ptr()
        _lib.call("nve_table_create_execution_context", self.table, ctypes.byref(self.ctx), s, s, None, None)
        ns = ctypes.c_int64()
        _lib.call("nve_amd_gpu_table_num_sets", self.table, ctypes.byref(ns))
        self.num_sets = ns.value
        self.model = O.Cache(cache_bytes, self.width, key_bytes, host_modify=not modify_on_gpu)
        assert self.model.num_sets == self.num_sets

    def load_model(self):
        """Copy the oracle cache's tags and rows into the GPU table."""
        tags = self.model.tags()
        if self.key_bytes == 4:
            tags = tags.astype(np.int32)
        _lib.call("nve_amd_gpu_table_import_state", self.table, tags.ctypes.data_as(ctypes.c_void_p),
                  None, None, 0)
        data = ctypes.c_void_p()
        _lib.call("nve_amd_gpu_table_data", self.table, ctypes.byref(data))
        d = self.model.data()
        hip_memcpy(data.value, d.ctypes.data, d.nbytes)

    def close(self):
        _lib.call("nve_context_wait", self.ctx)
        _lib.call("nve_context_destroy", self.ctx)
        _lib.call("nve_table_destroy", self.table)


def warm(ct, rng, n_insert, hot_rows, elem_bytes=4):
    """Insert with the oracle's policy, then negate every cached value (sign
    bit flip) so that a cache row and its backing row differ: a wrong hit/miss
    decision then changes the output."""
    keys = rng.choice(hot_rows, size=n_insert).astype(np.int64 if ct.key_bytes == 8 else np.int32)
    ct.model.insert_keys(keys, uvm=ct.uvm_np.reshape(-1))
    d = ct.model.data()
    d.reshape(-1, elem_bytes)[:, elem_bytes - 1] ^= np.uint8(0x80)
    ct.load_model()


def test_num_sets_matches_reference_formula():
    # ec_set_associative.h:667-685 + device-modify counters: per set
    # align16(8*8) + align16(8*256) + align16(8*4) = 2144 bytes for int64 keys
    ct = CachedTable(np.zeros((10, 256), np.uint8), 2144 * 1000 + 2143)
    assert ct.num_sets == 1000
    ct.close()


@pytest.mark.parametrize("key_bytes", [8, 4])
def test_find_uvm_resolves_hits_from_cache_and_misses_from_host(key_bytes):
    rng = np.random.default_rng(5 + key_bytes)
    rows, dim = 20000, 64
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 300 * 1024, key_bytes)
    warm(ct, rng, 4000, np.arange(0, 3000))
    kdt = np.int64 if key_bytes == 8 else np.int32
    keys = rng.integers(0, rows, size=5000).astype(kdt)
    keys[:2500] = rng.integers(0, 3000, size=2500)
    rows_ptr, hits, misses = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
    out = torch.zeros((keys.size, dim * 4), dtype=torch.uint8, device="cuda")
    _lib.call("nve_table_reset_lookup_counter", ct.table, ct.ctx)
    d_keys = to_dev(keys)  # keep device inputs referenced until the call has run
    _lib.call("nve_table_find", ct.table, ct.ctx, keys.size, vp(d_keys), None, dim * 4, vp(out), None)
    cnt = ctypes.c_int64()
    _lib.call("nve_table_get_lookup_counter", ct.table, ct.ctx, ctypes.byref(cnt))
    got = out.cpu().numpy()
    # expected rows: cache slot or backing row, as the model resolves them
    data = ct.model.data()
    base_d, base_u = data.ctypes.data, ct.uvm_np.ctypes.data
    for i in range(keys.size):
        p = int(rows_ptr[i])
        if base_d <= p < base_d + data.nbytes:
            exp = data[p - base_d:p - base_d + dim * 4]
        else:
            exp = ct.uvm_np.reshape(-1)[p - base_u:p - base_u + dim * 4]
        assert np.array_equal(got[i], exp), i
    assert cnt.value == misses
    assert 0 < misses < keys.size
    ct.close()


def test_find_without_backing_sets_hit_mask_and_keeps_missed_rows():
    rng = np.random.default_rng(17)
    rows, dim = 5000, 32
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, 64 * 1024, 8, with_uvm=False)
    warm(ct, rng, 800, np.arange(0, 600))
    keys = rng.integers(0, 1200, size=1000).astype(np.int64)
    mask_in = np.zeros((1000 + 63) // 64, np.uint64)
    mask_in[0] = np.uint64(0xFF)  # first 8 keys already resolved: skipped
    d_mask = to_dev(mask_in)
    out = torch.full((1000, dim * 4), 0xAB, dtype=torch.uint8, device="cuda")
    d_keys = to_dev(keys)
    _lib.call("nve_table_find", ct.table, ct.ctx, 1000, vp(d_keys), vp(d_mask), dim * 4, vp(out), None)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    data = ct.model.data()
    mask = d_mask.cpu().numpy().view(np.uint64)
    for i, k in enumerate(keys.tolist()):
        bit = (int(mask[i // 64]) >> (i % 64)) & 1
        if i < 8:
            assert bit == 1 and np.all(got[i] == 0xAB)
            continue
        way = ct.model.find_way(k)
        if way < 0:
            assert bit == 0 and np.all(got[i] == 0xAB)
        else:
            slot = ct.model.set_of(k) * 8 + way
            assert bit == 1 and np.array_equal(got[i], data[slot * dim * 4:(slot + 1) * dim * 4])
    ct.close()


@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_WMEAN, _lib.POOL_CONCAT])
def test_uvm_layer_pooled_and_hitrate(pooling):
    rng = np.random.default_rng(23 + pooling)
    rows, dim, bags = 30000, 128, 400
    uvm = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    ct = CachedTable(uvm, 2 * 1024 * 1024, 8, value_dtype=_lib.DT_F16)
    warm(ct, rng, 20000, np.arange(0, 8000), elem_bytes=2)
    off = csr_offsets(rng, bags, 30)
    n = int(off[-1])
    keys = np.where(rng.uniform(size=n) < 0.8, rng.integers(0, 8000, size=n),
                    rng.integers(0, rows, size=n)).astype(np.int64)
    w = rng.uniform(0, 1, size=n).astype(np.float32)
    L = _lib.load()
    never = ctypes.c_void_p()
    _lib.call("nve_heuristic_create_never", ctypes.byref(never))
    lc = L.nve_linear_uvm_layer_config_default()
    lc.insert_heuristic = never.value
    layer = ctypes.c_void_p()
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), ct.table, None)
    _lib.call("nve_heuristic_destroy", never)
    lctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(lctx), s, s, None, None)
    hr = (ctypes.c_float * 1)()
    rows_ptr, _, misses = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
    d_keys, d_off, d_w = to_dev(keys), to_dev(off), to_dev(w)
    if pooling == _lib.POOL_CONCAT:
        out = torch.zeros((n, dim), dtype=torch.float16, device="cuda")
        _lib.call("nve_layer_lookup_pooled", layer, lctx, n, vp(d_keys), vp(out), dim * 2, None, pooling,
                  0, None, 0, 0, None, 0, _lib.DT_F16, hr)
        got = out.cpu().numpy().view(np.uint16)
        ref = np.stack([np.frombuffer(ctypes.string_at(int(p), dim * 2), np.uint16) for p in rows_ptr])
        assert np.array_equal(got, ref)
    else:
        out = torch.zeros((bags, dim), dtype=torch.float16, device="cuda")
        _lib.call("nve_layer_lookup_pooled", layer, lctx, n, vp(d_keys), vp(out), dim * 2, None, pooling,
                  _lib.SPARSE_CSR, vp(d_off), bags + 1, 0, vp(d_w), _lib.DT_F32, _lib.DT_F16, hr)
        got = out.cpu().numpy().view(np.uint16)
        ref = O.pool(rows_ptr, O.F16, dim, O.CSR, pooling, n, off, bags, 0, w, O.F32, O.F16)
        assert np.array_equal(got, ref)
    assert abs(hr[0] - (1.0 - misses / n)) < 1e-6
    _lib.call("nve_context_wait", lctx)
    _lib.call("nve_context_destroy", lctx)
    _lib.call("nve_layer_destroy", layer)
    ct.close()


def test_erase_and_clear():
    rng = np.random.default_rng(41)
    rows, dim = 4000, 16
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, 32 * 1024, 8)
    warm(ct, rng, 600, np.arange(0, 500))
    cached = [k for k in range(500) if ct.model.find_way(k) >= 0]
    assert len(cached) > 20
    erase = np.array(cached[:10], np.int64)
    d_erase = to_dev(erase)
    _lib.call("nve_table_erase", ct.table, ct.ctx, erase.size, vp(d_erase))
    ct.model.erase(erase)
    tags = np.zeros(ct.num_sets * 8, np.int64)
    _lib.call("nve_amd_gpu_table_export_state", ct.table, tags.ctypes.data_as(ctypes.c_void_p), None, None, None)
    assert np.array_equal(tags, ct.model.tags())
    _lib.call("nve_table_clear", ct.table, ct.ctx)
    _lib.call("nve_amd_gpu_table_export_state", ct.table, tags.ctypes.data_as(ctypes.c_void_p), None, None, None)
    assert np.all(tags == -1)
    ct.close()


def test_uvm_layer_hit_rates_of_consecutive_lookups_on_every_path():
    """The LinearUVM layer's hit rate after each of a run of lookups on one
    context: long pooled bags (the split kernel), short pooled bags and plain
    lookups, in an order that alternates them, including a batch that all
    hits and one that all misses: the counter is read and zeroed after each
    lookup, and every rate equals the oracle's count."""
    rng = np.random.default_rng(31)
    rows, dim = 30000, 128
    uvm = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    ct = CachedTable(uvm, 2 * 1024 * 1024, 8, value_dtype=_lib.DT_F16)
    warm(ct, rng, 20000, np.arange(0, 8000), elem_bytes=2)
    L = _lib.load()
    never = ctypes.c_void_p()
    _lib.call("nve_heuristic_create_never", ctypes.byref(never))
    lc = L.nve_linear_uvm_layer_config_default()
    lc.insert_heuristic = never.value
    layer = ctypes.c_void_p()
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), ct.table, None)
    _lib.call("nve_heuristic_destroy", never)
    lctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(lctx), s, s, None, None)
    tags = ct.model.tags()
    ways = np.nonzero(tags != -1)[0]
    resident = tags[ways] * ct.num_sets + ways // 8
    absent = np.setdiff1d(np.arange(rows), resident)
    hr = (ctypes.c_float * 1)()
    kinds = ["long", "long", "short", "long", "plain", "long", "long_all_hit", "long_all_miss", "plain", "long"]
    for step, kind in enumerate(kinds):
        bags, hot = (64, 1024) if kind.startswith("long") else (400, 8)
        n = bags * hot if kind != "plain" else 5000
        if kind == "long_all_hit":
            keys = rng.choice(resident, size=n)
        elif kind == "long_all_miss":
            keys = rng.choice(absent, size=n)
        else:
            keys = np.where(rng.uniform(size=n) < 0.8, rng.integers(0, 8000, size=n),
                            rng.integers(0, rows, size=n))
        keys = keys.astype(np.int64)
        rows_ptr, _, misses = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
        d_keys = to_dev(keys)
        if kind == "plain":
            out = torch.zeros((n, dim), dtype=torch.float16, device="cuda")
            _lib.call("nve_layer_lookup", layer, lctx, n, vp(d_keys), vp(out), dim * 2, None, hr)
        else:
            out = torch.zeros((bags, dim), dtype=torch.float16, device="cuda")
            _lib.call("nve_layer_lookup_pooled", layer, lctx, n, vp(d_keys), vp(out), dim * 2, None, _lib.POOL_SUM,
                      _lib.SPARSE_FIXED, None, 0, hot, None, 0, _lib.DT_F16, hr)
            ref = O.pool(rows_ptr, O.F16, dim, O.FIXED, O.SUM, n, None, bags, hot, None, 0, O.F16)
            got = out.cpu().numpy().view(np.uint16)
            if kind == "short":
                assert np.array_equal(got, ref), step
            else:  # split bags: fp32 partial sums combined in wave order
                assert pooled_f16_close(got, ref), step
        want = 1.0 - misses / n
        assert abs(hr[0] - want) < 1e-6, (step, kind, hr[0], want)
        if kind == "long_all_hit":
            assert misses == 0
        if kind == "long_all_miss":
            assert misses == n
    _lib.call("nve_context_wait", lctx)
    _lib.call("nve_context_destroy", lctx)
    _lib.call("nve_layer_destroy", layer)
    ct.close()


@pytest.mark.parametrize("dtype,dim", [(O.F32, 132), (O.F32, 30), (O.F16, 63), (O.F16, 30)])
@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_MEAN, _lib.POOL_WSUM, _lib.POOL_WMEAN])
@pytest.mark.parametrize("bags,hot", [(17, 59), (2048, 5)])
def test_uvm_layer_pooling_of_odd_row_widths(dtype, dim, pooling, bags, hot):
    """find_and_combine_lookup_tests.cu's shapes (dims 132, 30 and 63, batches
    of 17 bags of 59 keys and 2,048 bags) through a cache-backed LinearUVM
    layer, half the rows resident with negated values so that every hit and
    miss decision shows: rows whose width is not a multiple of 16 bytes, bit
    for bit against the oracle's cache model and pooling order."""
    rng = np.random.default_rng(dim * 7 + pooling * 3 + bags)
    rows = 6000
    esz = 4 if dtype == O.F32 else 2
    uvm = float_table(rng, rows, dim, dtype)
    ct = CachedTable(uvm, 1 << 20, 8, value_dtype=_lib.DT_F32 if dtype == O.F32 else _lib.DT_F16)
    warm(ct, rng, 4000, np.arange(0, 3000), elem_bytes=esz)
    L = _lib.load()
    never = ctypes.c_void_p()
    _lib.call("nve_heuristic_create_never", ctypes.byref(never))
    lc = L.nve_linear_uvm_layer_config_default()
    lc.insert_heuristic = never.value
    layer = ctypes.c_void_p()
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), ct.table, None)
    _lib.call("nve_heuristic_destroy", never)
    lctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(lctx), s, s, None, None)
    n = bags * hot
    keys = rng.integers(0, rows, size=n).astype(np.int64)
    weighted = pooling in (_lib.POOL_WSUM, _lib.POOL_WMEAN)
    w = rng.uniform(0.0, 1.0, size=n).astype(np.float32) if weighted else None
    rows_ptr, _, misses = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
    out = torch.zeros((bags, dim), dtype=torch.float32 if dtype == O.F32 else torch.float16, device="cuda")
    hr = (ctypes.c_float * 1)()
    d_keys = to_dev(keys)
    d_w = to_dev(w) if weighted else None
    _lib.call("nve_layer_lookup_pooled", layer, lctx, n, vp(d_keys), vp(out), dim * esz, None, pooling,
              _lib.SPARSE_FIXED, None, 0, hot, vp(d_w), _lib.DT_F32 if weighted else 0,
              _lib.DT_F32 if dtype == O.F32 else _lib.DT_F16, hr)
    torch.cuda.synchronize()
    ref = O.pool(rows_ptr, dtype, dim, O.FIXED, pooling, n, None, bags, hot, w, O.F32 if weighted else 0, dtype)
    got = out.cpu().numpy()
    # 2,048 bags: one lane group per bag, the oracle's key order, bit for bit.
    # 17 bags: each bag is split over lane groups whose fp32 partial sums are
    # added in wave order -- exact for the dyadic rows unweighted, within the
    # pooling tolerance with real weights.
    exact = bags > 17 or not weighted
    if dtype == O.F32:
        if exact:
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
        else:
            assert rel_close(got, ref)
    else:
        if exact:
            assert np.array_equal(got.view(np.uint16), ref)
        else:
            assert pooled_f16_close(got.view(np.uint16), ref)
    assert abs(hr[0] - (1.0 - misses / n)) < 1e-6
    _lib.call("nve_context_wait", lctx)
    _lib.call("nve_context_destroy", lctx)
    _lib.call("nve_layer_destroy", layer)
    ct.close()


@pytest.mark.parametrize("qt", [O.QI8_F32, O.QU8_F32, O.QI8_F16, O.QU8_F16])
@pytest.mark.parametrize("count", [132, 30, 63])
@pytest.mark.parametrize("n", [1000, 4099])
def test_uvm_layer_dequant_of_odd_row_widths(qt, count, n):
    """find_and_dequant_tests.cu's shapes (4 quantized formats, 132 / 30 / 63
    values, 1,000 and 4,099 keys) through a cache-backed LinearUVM layer:
    Concatenate to the scale's precision, hits from resident rows whose bytes
    differ from the backing rows, misses over the host link; bit for bit
    against the oracle's dequantization of the rows the cache model names."""
    rng = np.random.default_rng(count * 5 + qt + n)
    rows = 5000
    q = quant_table(rng, rows, count, qt)
    # stored rows padded to 4 bytes, as the reference's test lays them out
    # (find_and_dequant_tests.cu:104-107); the metadata follows the values
    width = (q.shape[1] + 3) & ~3
    tb = np.zeros((rows, width), np.uint8)
    tb[:, :q.shape[1]] = q
    ct = CachedTable(tb, 1 << 20, 8, value_dtype=qt)
    warm(ct, rng, 3000, np.arange(0, 2500), elem_bytes=1)
    L = _lib.load()
    never = ctypes.c_void_p()
    _lib.call("nve_heuristic_create_never", ctypes.byref(never))
    lc = L.nve_linear_uvm_layer_config_default()
    lc.insert_heuristic = never.value
    layer = ctypes.c_void_p()
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), ct.table, None)
    _lib.call("nve_heuristic_destroy", never)
    lctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(lctx), s, s, None, None)
    keys = np.where(rng.uniform(size=n) < 0.7, rng.integers(0, 2500, size=n),
                    rng.integers(0, rows, size=n)).astype(np.int64)
    rows_ptr, _, misses = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
    stored = np.stack([np.frombuffer(ctypes.string_at(int(p), width), np.uint8) for p in rows_ptr])
    nat = O.native_out(qt)
    oes = 2 if nat == O.F16 else 4
    out = torch.zeros((n, count * oes), dtype=torch.uint8, device="cuda")
    hr = (ctypes.c_float * 1)()
    d_keys = to_dev(keys)
    _lib.call("nve_layer_lookup_pooled", layer, lctx, n, vp(d_keys), vp(out), count * oes, None, _lib.POOL_CONCAT,
              0, None, 0, 0, None, 0, nat, hr)
    torch.cuda.synchronize()
    ref = O.dequant_rows(stored, qt, count, nat)
    got = out.cpu().numpy().view(np.uint16 if nat == O.F16 else np.float32).reshape(n, count)
    assert np.array_equal(got.view(np.uint16 if nat == O.F16 else np.uint32),
                          ref.view(np.uint16 if nat == O.F16 else np.uint32))
    assert abs(hr[0] - (1.0 - misses / n)) < 1e-6
    # the raw rows of the same keys (Concatenate to the stored type is the plain lookup)
    raw = torch.zeros((n, width), dtype=torch.uint8, device="cuda")
    _lib.call("nve_layer_lookup", layer, lctx, n, vp(d_keys), vp(raw), width, None, hr)
    assert np.array_equal(raw.cpu().numpy(), stored)
    _lib.call("nve_context_wait", lctx)
    _lib.call("nve_context_destroy", lctx)
    _lib.call("nve_layer_destroy", layer)
    ct.close()


@pytest.mark.parametrize("qt", [O.QI8_F32, O.QU8_F32, O.QI8_F16, O.QU8_F16])
@pytest.mark.parametrize("count", [132, 30, 63])
@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_WMEAN])
def test_uvm_layer_quantized_pooling_of_odd_row_widths(qt, count, pooling):
    """quant_lookup_tests.cu's case through a cache-backed LinearUVM layer:
    quantized rows of 132 / 30 / 63 values (padded to 4 bytes) pooled over
    CSR bags of up to 40 keys (one lane group per bag: the oracle's order),
    hits from resident rows that differ from the backing rows, bit for bit."""
    rng = np.random.default_rng(count * 11 + qt + pooling)
    rows, bags = 5000, 300
    q = quant_table(rng, rows, count, qt)
    width = (q.shape[1] + 3) & ~3
    tb = np.zeros((rows, width), np.uint8)
    tb[:, :q.shape[1]] = q
    ct = CachedTable(tb, 1 << 20, 8, value_dtype=qt)
    warm(ct, rng, 3000, np.arange(0, 2500), elem_bytes=1)
    L = _lib.load()
    never = ctypes.c_void_p()
    _lib.call("nve_heuristic_create_never", ctypes.byref(never))
    lc = L.nve_linear_uvm_layer_config_default()
    lc.insert_heuristic = never.value
    layer = ctypes.c_void_p()
    _lib.call("nve_linear_uvm_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), ct.table, None)
    _lib.call("nve_heuristic_destroy", never)
    lctx = ctypes.c_void_p()
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(lctx), s, s, None, None)
    off = csr_offsets(rng, bags, 40)
    n = int(off[-1])
    keys = np.where(rng.uniform(size=n) < 0.7, rng.integers(0, 2500, size=n),
                    rng.integers(0, rows, size=n)).astype(np.int64)
    weighted = pooling == _lib.POOL_WMEAN
    w = rng.uniform(0.0, 1.0, size=n).astype(np.float32) if weighted else None
    rows_ptr, _, misses = ct.model.resolve(keys, ct.uvm_np.reshape(-1))
    nat = O.native_out(qt)
    oes = 2 if nat == O.F16 else 4
    out = torch.zeros((bags, count * oes), dtype=torch.uint8, device="cuda")
    hr = (ctypes.c_float * 1)()
    d_keys, d_off = to_dev(keys), to_dev(off)
    d_w = to_dev(w) if weighted else None
    _lib.call("nve_layer_lookup_pooled", layer, lctx, n, vp(d_keys), vp(out), count * oes, None, pooling,
              _lib.SPARSE_CSR, vp(d_off), bags + 1, 0, vp(d_w), _lib.DT_F32 if weighted else 0, nat, hr)
    torch.cuda.synchronize()
    ref = O.pool(rows_ptr, qt, count, O.CSR, pooling, n, off, bags, 0, w, O.F32 if weighted else 0, nat)
    got = out.cpu().numpy().view(np.uint16 if nat == O.F16 else np.float32).reshape(bags, count)
    assert np.array_equal(got.view(np.uint16 if nat == O.F16 else np.uint32),
                          ref.view(np.uint16 if nat == O.F16 else np.uint32))
    assert abs(hr[0] - (1.0 - misses / n)) < 1e-6
    _lib.call("nve_context_wait", lctx)
    _lib.call("nve_context_destroy", lctx)
    _lib.call("nve_layer_destroy", layer)
    ct.close()

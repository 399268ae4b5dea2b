"""The capability matrix on the CPU: its totals against the reference's, and
the HostLayer's 336 cases (every pooling mode, layout, stored and output
dtype, weight dtype and key type; all enabled, as in the reference), plus the
HostLayer's side of the reference suite's standalone checks: empty CSR bags
and zero-sum weights give zero rows, a padded output stride is honoured, and
Concatenate ignores every bag and weight field
(tests/layer_pooling/layer_pooling_test.cu:70-219)."""
import ctypes
import zlib

import numpy as np
import pytest

import pooling_matrix as M
from oracle import oracle as O
from pynve import _lib

CASES = M.cases()
HOST_CASES = [(lab, c) for lab, c in CASES if c["layer"] == M.HOST]


def p(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def test_matrix_totals_match_the_reference_suite():
    got = {layer: [0, 0] for layer in M.LAYERS}
    for _, c in CASES:
        got[c["layer"]][0 if c["status"] == "enabled" else 1] += 1
    assert {k: tuple(v) for k, v in got.items()} == M.REFERENCE_TOTALS


class HostLayers:
    """One LinearHostTable + HostLayer + context per (stored dtype, key type)."""

    def __init__(self):
        self.made = {}

    def get(self, din, k64, tb=None):
        key = (din, k64, None if tb is None else id(tb))
        if key not in self.made:
            L = _lib.load()
            tb = M.table(din) if tb is None else tb
            kt = _lib.KEY_INT64 if k64 else _lib.KEY_INT32
            tc = L.nve_host_table_config_default()
            tc.key_size = 8 if k64 else 4
            tc.max_value_size = tb.shape[1]
            tc.value_dtype = din
            t, lay, ctx = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
            _lib.call("nve_amd_linear_host_table_create", ctypes.byref(t), kt, ctypes.byref(tc), p(tb),
                      tb.shape[0], 0)
            lc = L.nve_host_embedding_layer_config_default()
            _lib.call("nve_host_embedding_layer_create", ctypes.byref(lay), kt, ctypes.byref(lc), t, None)
            _lib.call("nve_layer_create_execution_context", lay, ctypes.byref(ctx), None, None, None, None)
            self.made[key] = (t, lay, ctx, tb)
        return self.made[key][1:3]

    def close(self):
        for t, lay, ctx, _ in self.made.values():
            _lib.call("nve_context_destroy", ctx)
            _lib.call("nve_layer_destroy", lay)
            _lib.call("nve_table_destroy", t)


@pytest.fixture(scope="module")
def hosts():
    h = HostLayers()
    yield h
    h.close()


def pooled_call(layer, ctx, case, keys, off, w, out, stride=None):
    """nve_layer_lookup_pooled for the case; Concatenate gets poisoned bag and
    weight fields (layer_pooling_harness.hpp:446-455).  Returns (status, hit rate)."""
    hr = (ctypes.c_float * 1)()
    stride = out.strides[0] if stride is None else stride
    if case["pool"] == O.CONCAT:
        poison = np.zeros(1, np.float64)
        st = _lib.load().nve_layer_lookup_pooled(layer, ctx, keys.size, p(keys), p(out), stride, None,
                                                 _lib.POOL_CONCAT, 2, None, -1, -1, p(poison), _lib.DT_F64,
                                                 case["dout"], hr)
    else:
        wv = None if w is None else (w.view(np.uint16) if w.dtype == np.float16 else w)
        st = _lib.load().nve_layer_lookup_pooled(
            layer, ctx, keys.size, p(keys), p(out), stride, None, case["pool"], case["sparse"], p(off),
            0 if off is None else off.size, M.HOTNESS if off is None else 0, p(wv),
            case["wdt"] if w is not None else 0, case["dout"], hr)
    return st, hr[0]


@pytest.mark.parametrize("label,case", HOST_CASES, ids=[lab for lab, _ in HOST_CASES])
def test_host_layer_case(hosts, label, case):
    layer, ctx = hosts.get(case["din"], case["k64"])
    keys, off, bags, w = M.inputs(case, seed=zlib.crc32(label.encode()))
    out = M.out_array(case, bags)
    st, hr = pooled_call(layer, ctx, case, keys, off, w, out)
    _lib.check(st)
    assert hr == 1.0
    ref = M.oracle_out(case, keys, off, bags, w, host_order=True)
    assert np.array_equal(out.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8)), label
    r64, mag = M.reduce64(case, keys, off, bags, w)
    M.assert_close64(case, out, r64, mag)


def small_table(din, count=16, rows=256, seed=3):
    rng = np.random.default_rng(seed + din)
    if din in M.QUANT:
        from nve_helpers import quant_table
        return quant_table(rng, rows, count, din)
    return rng.normal(0, 0.5, size=(rows, count)).astype(np.float32).view(np.uint8)


@pytest.mark.parametrize("din", [O.F32, O.QI8_F32])
@pytest.mark.parametrize("pool", [O.MEAN, O.WMEAN])
def test_host_empty_csr_bags_and_zero_weight_sum_give_zero_rows(hosts, din, pool):
    """layer_pooling_test.cu:149-186 / harness :639-700: bags {3,0,3,0,0,3,3,0},
    the last non-empty bag's weights summing to zero; the output is poisoned
    first so that zero rows are proven written."""
    tb = small_table(din)
    layer, ctx = hosts.get(din, True, tb)
    rng = np.random.default_rng(1)
    keys = rng.integers(0, 256, size=12).astype(np.int64)
    off = np.array([0, 3, 3, 6, 6, 6, 9, 12, 12], np.int64)
    w = np.ones(12, np.float32)
    w[9:12] = [1.0, -2.0, 1.0]
    out = np.full((8, 16), np.frombuffer(b"\x5a\x5a\x5a\x5a", np.float32)[0], np.float32)
    hr = (ctypes.c_float * 1)()
    _lib.check(_lib.load().nve_layer_lookup_pooled(layer, ctx, 12, p(keys), p(out), 64, None, pool,
                                                   _lib.SPARSE_CSR, p(off), off.size, 0,
                                                   p(w) if pool == O.WMEAN else None,
                                                   _lib.DT_F32 if pool == O.WMEAN else 0, _lib.DT_F32, hr))
    assert not np.isnan(out).any()
    zero = [1, 3, 4, 7] + ([6] if pool == O.WMEAN else [])
    assert np.all(out[zero] == 0.0)
    v = M.values64(tb[keys], din, 16)
    for b in range(8):
        if b in zero:
            continue
        s, e = off[b], off[b + 1]
        ww = w[s:e] if pool == O.WMEAN else np.ones(e - s)
        ref = (v[s:e] * ww[:, None]).sum(0) / ww.sum()
        assert np.allclose(out[b], ref, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("din", [O.F32, O.QI8_F32])
def test_host_padded_output_stride_is_honoured(hosts, din):
    """layer_pooling_test.cu:188-219: the CPU pooling path takes the width from
    the stored row, so a stride two elements wider pools into the padded rows."""
    tb = small_table(din)
    layer, ctx = hosts.get(din, True, tb)
    keys = np.random.default_rng(2).integers(0, 256, size=64).astype(np.int64)
    out = np.full((16, 18), -7.0, np.float32)
    hr = (ctypes.c_float * 1)()
    _lib.check(_lib.load().nve_layer_lookup_pooled(layer, ctx, 64, p(keys), p(out), 72, None, _lib.POOL_SUM,
                                                   _lib.SPARSE_FIXED, None, 0, 4, None, 0, _lib.DT_F32, hr))
    v = M.values64(tb[keys], din, 16)
    ref = v.reshape(16, 4, 16).sum(1)
    assert np.allclose(out[:, :16], ref, rtol=1e-5, atol=1e-6)
    assert np.all(out[:, 16:] == -7.0)  # the padding is left alone


def test_host_malformed_pool_params_are_invalid_arguments(hosts):
    """layer_pooling_test.cu:70-96,113-146 through the C ABI: unknown output
    type, hotness 0, keys not a multiple of the hotness, weighted pooling
    without weights, CSR without offsets; Fixed needs no offsets."""
    tb = small_table(O.F32)
    layer, ctx = hosts.get(O.F32, True, tb)
    keys = np.arange(12, dtype=np.int64)
    out = np.zeros((12, 16), np.float32)
    L = _lib.load()

    def call(n, pool, sparse, off, n_off, hot, w, wdt, odt):
        return L.nve_layer_lookup_pooled(layer, ctx, n, p(keys), p(out), 64, None, pool, sparse, p(off), n_off,
                                         hot, p(w), wdt, odt, None)

    w = np.ones(12, np.float32)
    assert call(12, _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, 3, None, 0, 0) == _lib.INVALID_ARGUMENT
    assert call(12, _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, 0, None, 0, _lib.DT_F32) == _lib.INVALID_ARGUMENT
    assert call(11, _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, 3, None, 0, _lib.DT_F32) == _lib.INVALID_ARGUMENT
    assert call(12, _lib.POOL_WSUM, _lib.SPARSE_FIXED, None, 0, 3, None, _lib.DT_F32,
                _lib.DT_F32) == _lib.INVALID_ARGUMENT
    assert call(12, _lib.POOL_SUM, _lib.SPARSE_CSR, None, 5, 0, None, 0, _lib.DT_F32) == _lib.INVALID_ARGUMENT
    assert call(12, _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, 3, None, 0, _lib.DT_F32) == _lib.SUCCESS
    off = np.array([0, 3, 6, 9, 12], np.int64)
    assert call(12, _lib.POOL_SUM, _lib.SPARSE_CSR, off, 5, 0, None, 0, _lib.DT_F32) == _lib.SUCCESS
    assert call(12, _lib.POOL_WSUM, _lib.SPARSE_FIXED, None, 0, 3, w, _lib.DT_F32, _lib.DT_F32) == _lib.SUCCESS

"""The capability matrix on the GPU-backed layers: the GPU layer's 152 enabled
and 112 refused cases and the LinearUVM layer's 168 and 112
(tests/layer_pooling/layer_pooling_harness.hpp:131-190 restated in
tests/pooling_matrix.py), plus the GPU-backed side of the reference suite's
standalone checks: empty CSR bags and zero-sum weights give zero rows, and a
padded output stride is refused (layer_pooling_test.cu:149-219).

Every enabled case passes host-resident keys, offsets, weights and output,
as the reference's harness does (the layer stages them); its result must
equal the oracle bit for bit (the kernels' reduction order) and an
independent float64 reduction within the stated tolerance.  The LinearUVM
layer's cache holds part of the table (inserted from the backing table
first), so its cases mix hits from HBM and misses over the host link; with
the reference's never-insert heuristic the cache then stays as it is."""
import ctypes
import zlib

import numpy as np
import pytest

import pooling_matrix as M
from nve_helpers import quant_table, stream_ptr, to_dev
from oracle import oracle as O
from pynve import _lib
from test_pooling_matrix_cpu import p, pooled_call

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

CASES = [(lab, c) for lab, c in M.cases() if c["layer"] != M.HOST]


class Layers:
    """One layer + context per (layer kind, stored dtype, key type, table)."""

    def __init__(self):
        self.made = {}
        self.keep = []

    def get(self, kind, din, k64, tb=None):
        key = (kind, din, k64, None if tb is None else id(tb))
        if key in self.made:
            return self.made[key]
        L = _lib.load()
        tb = M.table(din) if tb is None else tb
        self.keep.append(tb)
        rows, width = tb.shape
        kt = _lib.KEY_INT64 if k64 else _lib.KEY_INT32
        lay, ctx, table = ctypes.c_void_p(), ctypes.c_void_p(), None
        s = stream_ptr()
        if kind == M.GPU:
            d = to_dev(tb.reshape(-1))
            self.keep.append(d)
            cfg = L.nve_gpu_embedding_layer_config_default()
            cfg.layer_name = b"matrix"
            cfg.embedding_table = d.data_ptr()
            cfg.num_embeddings = rows
            cfg.embedding_width_in_bytes = width
            cfg.value_dtype = din
            _lib.call("nve_gpu_embedding_layer_create", ctypes.byref(lay), kt, ctypes.byref(cfg), None)
        else:
            h = torch.from_numpy(np.ascontiguousarray(tb).reshape(-1).copy()).pin_memory()
            self.keep.append(h)
            tc = L.nve_gpu_table_config_default()
            tc.cache_size = 4 << 20
            tc.row_size_in_bytes = width
            tc.value_dtype = din
            tc.uvm_table = h.data_ptr()
            tc.uvm_num_rows = rows
            table = ctypes.c_void_p()
            _lib.call("nve_gpu_table_create", ctypes.byref(table), kt, ctypes.byref(tc), None)
            # part of the table resident: lookups mix cache hits and host misses
            tctx = ctypes.c_void_p()
            _lib.call("nve_table_create_execution_context", table, ctypes.byref(tctx), s, s, None, None)
            kdt = np.int64 if k64 else np.int32
            warm = to_dev(np.random.default_rng(din).integers(0, rows, size=rows // 2).astype(kdt))
            _lib.call("nve_amd_table_insert_from_uvm", table, tctx, warm.numel(), ctypes.c_void_p(warm.data_ptr()))
            _lib.call("nve_context_wait", tctx)
            _lib.call("nve_context_destroy", tctx)
            never = ctypes.c_void_p()
            _lib.call("nve_heuristic_create_never", ctypes.byref(never))
            lc = L.nve_linear_uvm_layer_config_default()
            lc.insert_heuristic = never
            _lib.call("nve_linear_uvm_layer_create", ctypes.byref(lay), kt, ctypes.byref(lc), table, None)
            _lib.call("nve_heuristic_destroy", never)
        _lib.call("nve_layer_create_execution_context", lay, ctypes.byref(ctx), s, s, None, None)
        self.made[key] = (lay, ctx, table)
        return self.made[key]

    def close(self):
        for lay, ctx, table in self.made.values():
            _lib.call("nve_context_wait", ctx)
            _lib.call("nve_context_destroy", ctx)
            _lib.call("nve_layer_destroy", lay)
            if table is not None:
                _lib.call("nve_table_destroy", table)


@pytest.fixture(scope="module")
def layers():
    lays = Layers()
    yield lays
    lays.close()


@pytest.mark.parametrize("label,case", CASES, ids=[lab for lab, _ in CASES])
def test_gpu_backed_layer_case(layers, label, case):
    lay, ctx, _ = layers.get(case["layer"], case["din"], case["k64"])
    keys, off, bags, w = M.inputs(case, seed=zlib.crc32(label.encode()))
    out = M.out_array(case, bags)
    st, hr = pooled_call(lay, ctx, case, keys, off, w, out)
    if case["status"] == "rejected":
        # a well-formed request whose dtype combination is not implemented
        assert st == _lib.INVALID_ARGUMENT, (label, st, _lib.last_error())
        assert "output type" in _lib.last_error()
        return
    _lib.check(st)
    _lib.call("nve_context_wait", ctx)
    torch.cuda.synchronize()
    if case["layer"] == M.GPU:
        assert hr == 1.0
    ref = M.oracle_out(case, keys, off, bags, w, host_order=False)
    assert np.array_equal(out.view(np.uint8), np.ascontiguousarray(ref).view(np.uint8)), label
    r64, mag = M.reduce64(case, keys, off, bags, w)
    M.assert_close64(case, out, r64, mag)


def small_table(din, count=16, rows=256, seed=3):
    rng = np.random.default_rng(seed + din)
    if din in M.QUANT:
        return quant_table(rng, rows, count, din)
    return rng.normal(0, 0.5, size=(rows, count)).astype(np.float32).view(np.uint8)


@pytest.mark.parametrize("kind", [M.GPU, M.UVM])
@pytest.mark.parametrize("din", [O.F32, O.QI8_F32])
@pytest.mark.parametrize("pool", [O.MEAN, O.WMEAN])
def test_empty_csr_bags_and_zero_weight_sum_give_zero_rows(layers, kind, din, pool):
    """layer_pooling_test.cu:149-186: bags {3,0,3,0,0,3,3,0}, the last
    non-empty bag's weights summing to zero; the output is poisoned first so
    that zero rows are proven written, and nothing may be NaN."""
    tb = small_table(din)
    lay, ctx, _ = layers.get(kind, din, True, tb)
    keys = np.random.default_rng(1).integers(0, 256, size=12).astype(np.int64)
    off = np.array([0, 3, 3, 6, 6, 6, 9, 12, 12], np.int64)
    w = np.ones(12, np.float32)
    w[9:12] = [1.0, -2.0, 1.0]
    out = np.full((8, 16), np.frombuffer(b"\x5a\x5a\x5a\x5a", np.float32)[0], np.float32)
    _lib.check(_lib.load().nve_layer_lookup_pooled(lay, ctx, 12, p(keys), p(out), 64, None, pool,
                                                   _lib.SPARSE_CSR, p(off), off.size, 0,
                                                   p(w) if pool == O.WMEAN else None,
                                                   _lib.DT_F32 if pool == O.WMEAN else 0, _lib.DT_F32, None))
    _lib.call("nve_context_wait", ctx)
    torch.cuda.synchronize()
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


@pytest.mark.parametrize("kind", [M.GPU, M.UVM])
@pytest.mark.parametrize("din", [O.F32, O.QI8_F32])
def test_padded_output_stride_is_refused(layers, kind, din):
    """layer_pooling_test.cu:188-219: the GPU pool kernels take the width from
    the output stride, so a stride two elements wider than the stored row
    holds is refused before any work."""
    tb = small_table(din)
    lay, ctx, _ = layers.get(kind, din, True, tb)
    keys = np.random.default_rng(2).integers(0, 256, size=64).astype(np.int64)
    out = np.full((16, 18), -7.0, np.float32)
    st = _lib.load().nve_layer_lookup_pooled(lay, ctx, 64, p(keys), p(out), 72, None, _lib.POOL_SUM,
                                             _lib.SPARSE_FIXED, None, 0, 4, None, 0, _lib.DT_F32, None)
    assert st == _lib.INVALID_ARGUMENT
    assert "stride" in _lib.last_error()
    _lib.call("nve_context_wait", ctx)
    assert np.all(out == -7.0)

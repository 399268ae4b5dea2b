"""GPU parity of GPUEmbeddingLayer through the C ABI against the CPU oracle.

Cases follow the reference's own tests: plain gathers are compared bytewise
(tests/embedding_layer/gpu_layer_test.cpp:353,692), pooled results against the
per-bag fp32 reduction (MockHostTable::combine, mock_host_table.hpp:273-402;
find_and_combine_lookup_tests.cu:176-194) with dyadic-fraction tables so that
Sum is exact, dims {132, 30, 63} and batches {17, 2048}, and sanitize of
out-of-range keys (gpu_layer_test.cpp:619-624)."""
import ctypes

import numpy as np
import pytest

from nve_helpers import (csr_offsets, f16_ulp_close, float_table, from_dev, oracle_dequant,
                         oracle_pool, quant_table, rel_close, stream_ptr, to_dev, vp)
from oracle import oracle as O
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

DT = {O.F32: _lib.DT_F32, O.F16: _lib.DT_F16}


class GpuLayer:
    """GPUEmbeddingLayer + one execution context on torch's current stream."""

    def __init__(self, table_bytes, dtype, key_bytes=8, default_row=-1):
        self.rows, self.width = table_bytes.shape
        self.d_table = to_dev(table_bytes.reshape(-1))
        L = _lib.load()
        cfg = L.nve_gpu_embedding_layer_config_default()
        cfg.layer_name = b"t"
        cfg.embedding_table = self.d_table.data_ptr()
        cfg.num_embeddings = self.rows
        cfg.embedding_width_in_bytes = self.width
        cfg.value_dtype = dtype
        cfg.default_row_index = default_row
        self.kt = _lib.KEY_INT32 if key_bytes == 4 else _lib.KEY_INT64
        self.layer = ctypes.c_void_p()
        _lib.call("nve_gpu_embedding_layer_create", ctypes.byref(self.layer), self.kt, ctypes.byref(cfg), None)
        self.ctx = ctypes.c_void_p()
        s = stream_ptr()
        _lib.call("nve_layer_create_execution_context", self.layer, ctypes.byref(self.ctx), s, s, None, None)

    def close(self):
        _lib.call("nve_context_wait", self.ctx)
        _lib.call("nve_context_destroy", self.ctx)
        _lib.call("nve_layer_destroy", self.layer)

    def lookup(self, d_keys, n, d_out, stride):
        _lib.call("nve_layer_lookup", self.layer, self.ctx, n, vp(d_keys), vp(d_out), stride, None, None)

    def pooled(self, d_keys, n, d_out, stride, pooling, sparse, d_off, n_off, hot, d_w, wt, ot):
        hr = (ctypes.c_float * 1)()
        _lib.call("nve_layer_lookup_pooled", self.layer, self.ctx, n, vp(d_keys), vp(d_out), stride, None,
                  pooling, sparse, vp(d_off), n_off, hot, vp(d_w), wt, ot, hr)
        assert hr[0] == 1.0


@pytest.mark.parametrize("dtype,dim", [(O.F32, 132), (O.F32, 30), (O.F16, 63), (O.F16, 128),
                                       (O.F32, 1), (O.F16, 1)])
@pytest.mark.parametrize("n", [17, 2048])
@pytest.mark.parametrize("key_bytes", [4, 8])
def test_plain_gather_bit_exact(dtype, dim, n, key_bytes):
    rng = np.random.default_rng(dim * 1000 + n + key_bytes)
    rows = 5000
    tb = float_table(rng, rows, dim, dtype, dyadic_values=False)
    kdt = np.int32 if key_bytes == 4 else np.int64
    keys = rng.integers(0, rows, size=n).astype(kdt)
    lay = GpuLayer(tb, DT[dtype], key_bytes)
    out = torch.zeros((n, tb.shape[1]), dtype=torch.uint8, device="cuda")
    lay.lookup(to_dev(keys), n, out, tb.shape[1])
    torch.cuda.synchronize()
    ref, hits = O.gather(keys, np.ascontiguousarray(tb).reshape(-1), tb.shape[1], rows)
    assert hits == n
    assert np.array_equal(out.cpu().numpy(), ref)
    lay.close()


def test_gather_host_buffers_and_empty_batch():
    rng = np.random.default_rng(3)
    tb = float_table(rng, 100, 16, O.F32)
    lay = GpuLayer(tb, _lib.DT_F32)
    keys = rng.integers(0, 100, size=77).astype(np.int64)
    out = np.zeros((77, 64), np.uint8)
    _lib.call("nve_layer_lookup", lay.layer, lay.ctx, 77, keys.ctypes.data_as(ctypes.c_void_p),
              out.ctypes.data_as(ctypes.c_void_p), 64, None, None)
    _lib.call("nve_context_wait", lay.ctx)
    assert np.array_equal(out, tb[keys])
    dummy = torch.zeros(1, dtype=torch.int64, device="cuda")
    lay.lookup(dummy, 0, dummy, 64)  # zero keys: nothing happens
    lay.close()


def test_sanitize_default_row():
    rng = np.random.default_rng(4)
    rows = 64
    tb = float_table(rng, rows, 8, O.F32)
    keys = np.array([0, 5, 63, 64, -1, 1 << 40, 7, -(1 << 40)], np.int64)
    lay = GpuLayer(tb, _lib.DT_F32, default_row=7)
    out = torch.zeros((keys.size, 32), dtype=torch.uint8, device="cuda")
    lay.lookup(to_dev(keys), keys.size, out, 32)
    torch.cuda.synchronize()
    exp = tb[O.sanitize(keys, rows, 7)]
    assert np.array_equal(out.cpu().numpy(), exp)
    lay.close()


def test_out_of_range_keys_without_default_row():
    """No default row: keys outside [0, rows) read nothing (the reference reads
    past the table).  Their gathered rows keep the output's content; a bag
    counts them as zero rows (the oracle on the table plus one zero row)."""
    rng = np.random.default_rng(14)
    rows, dim = 100, 16
    tb = float_table(rng, rows, dim, O.F32)
    keys = np.array([3, -1, 99, 100, 1 << 40, 42, -(1 << 40), 7], np.int64)
    lay = GpuLayer(tb, _lib.DT_F32)
    out = torch.full((keys.size, dim * 4), 0xAB, dtype=torch.uint8, device="cuda")
    d_keys = to_dev(keys)
    lay.lookup(d_keys, keys.size, out, dim * 4)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    inside = (keys >= 0) & (keys < rows)
    assert np.array_equal(got[inside], tb[keys[inside]])
    assert np.all(got[~inside] == 0xAB)
    # pooled: 2 bags of 4, Sum and Mean
    padded = np.concatenate([tb, np.zeros((1, tb.shape[1]), np.uint8)])
    mapped = np.where(inside, keys, rows)
    for pooling in (_lib.POOL_SUM, _lib.POOL_MEAN):
        pout = torch.zeros((2, dim * 4), dtype=torch.uint8, device="cuda")
        lay.pooled(d_keys, keys.size, pout, dim * 4, pooling, _lib.SPARSE_FIXED, None, 0, 4, None,
                   _lib.DT_F32, _lib.DT_F32)
        torch.cuda.synchronize()
        ref = oracle_pool(padded, mapped, O.F32, dim, O.FIXED, pooling, None, 2, 4, None, O.F32, O.F32)
        assert np.array_equal(pout.cpu().numpy().view(np.uint32).reshape(2, dim), ref.view(np.uint32))
    lay.close()


def test_invalid_arguments_raise_before_work():
    rng = np.random.default_rng(5)
    tb = float_table(rng, 16, 4, O.F32)
    lay = GpuLayer(tb, _lib.DT_F32)
    k = to_dev(np.zeros(4, np.int64))
    out = torch.zeros(64, dtype=torch.uint8, device="cuda")
    with pytest.raises(_lib.InvalidArgument, match="Output stride"):
        lay.lookup(k, 4, out, 8)
    with pytest.raises(_lib.InvalidArgument, match="Hitmask"):
        _lib.call("nve_layer_lookup", lay.layer, lay.ctx, 4, vp(k), vp(out), 16, vp(out), None)
    with pytest.raises(_lib.InvalidArgument, match="divide"):  # fixed hotness must divide
        lay.pooled(k, 4, out, 16, _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, 3, None, 0, _lib.DT_F32)
    with pytest.raises(_lib.InvalidArgument, match="output type"):
        lay.pooled(k, 4, out, 16, _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, 2, None, 0, _lib.DT_F16)
    with pytest.raises(_lib.InvalidArgument, match="weights are required"):
        lay.pooled(k, 4, out, 16, _lib.POOL_WSUM, _lib.SPARSE_FIXED, None, 0, 2, None, 0, _lib.DT_F32)
    lay.close()


POOLS = [_lib.POOL_SUM, _lib.POOL_MEAN, _lib.POOL_WSUM, _lib.POOL_WMEAN]


@pytest.mark.parametrize("dtype,dim", [(O.F32, 132), (O.F32, 30), (O.F16, 63), (O.F16, 128)])
@pytest.mark.parametrize("pooling", POOLS)
@pytest.mark.parametrize("sparse", [_lib.SPARSE_FIXED, _lib.SPARSE_CSR])
@pytest.mark.parametrize("bags", [17, 2048])
def test_pooled_matches_oracle(dtype, dim, pooling, sparse, bags):
    """Default geometry: bags reduced in key order -> bit-exact with the oracle."""
    rng = np.random.default_rng(bags * 7 + dim + pooling * 3 + sparse)
    rows = 4000
    tb = float_table(rng, rows, dim, dtype)
    hot = 59 if bags == 17 else 5
    if sparse == _lib.SPARSE_FIXED:
        off = None
        n = bags * hot
    else:
        off = csr_offsets(rng, bags, 2 * hot)
        n = int(off[-1])
    keys = rng.integers(0, rows, size=n).astype(np.int64)
    weighted = pooling in (_lib.POOL_WSUM, _lib.POOL_WMEAN)
    w = (np.exp2(-rng.integers(0, 4, size=n)) * rng.choice([-1, 1], size=n)) if weighted else None
    if w is not None:
        w = w.astype(np.float32 if dtype == O.F32 else np.float16)
    lay = GpuLayer(tb, DT[dtype])
    out_np = np.float32 if dtype == O.F32 else np.uint16
    out = torch.zeros((bags, dim), dtype=torch.float32 if dtype == O.F32 else torch.float16, device="cuda")
    lay.pooled(to_dev(keys), n, out, tb.shape[1], pooling, sparse, None if off is None else to_dev(off),
               0 if off is None else bags + 1, hot if off is None else 0,
               None if w is None else to_dev(w.view(np.uint16) if dtype == O.F16 else w),
               DT[dtype] if weighted else 0, DT[dtype])
    torch.cuda.synchronize()
    got = from_dev(out, out_np)
    ref = oracle_pool(tb, keys, dtype, dim, O.CSR if off is not None else O.FIXED, pooling, off, bags,
                      hot, None if w is None else (w.view(np.uint16) if dtype == O.F16 else w),
                      dtype, dtype)
    if dtype == O.F32:
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    else:
        assert np.array_equal(got, ref)
    lay.close()


QTYPES = [(O.QI8_F32, _lib.DT_QI8_F32), (O.QI8_F16, _lib.DT_QI8_F16), (O.QU8_F32, _lib.DT_QU8_F32),
          (O.QU8_F16, _lib.DT_QU8_F16)]


@pytest.mark.parametrize("qt", QTYPES)
@pytest.mark.parametrize("count", [132, 30, 64])
def test_quant_raw_concat_and_dequant(qt, count):
    odt, cdt = qt
    rng = np.random.default_rng(count + odt)
    rows, n = 3000, 1000
    tb = quant_table(rng, rows, count, odt)
    keys = rng.integers(0, rows, size=n).astype(np.int64)
    lay = GpuLayer(tb, cdt)
    width = tb.shape[1]
    # plain lookup: raw stored rows incl. metadata
    raw = torch.zeros((n, width), dtype=torch.uint8, device="cuda")
    lay.lookup(to_dev(keys), n, raw, width)
    # Concatenate to the metadata precision: dequantized rows
    nat = O.native_out(odt)
    oes = 2 if nat == O.F16 else 4
    deq = torch.zeros((n, count * oes), dtype=torch.uint8, device="cuda")
    lay.pooled(to_dev(keys), n, deq, count * oes, _lib.POOL_CONCAT, 0, None, 0, 0, None, 0, DT[nat])
    torch.cuda.synchronize()
    assert np.array_equal(raw.cpu().numpy(), tb[keys])
    ref = oracle_dequant(tb, keys, odt, count, nat)
    got = deq.cpu().numpy().view(np.uint16 if nat == O.F16 else np.float32).reshape(n, count)
    assert np.array_equal(got.view(np.uint16 if nat == O.F16 else np.uint32),
                          ref.view(np.uint16 if nat == O.F16 else np.uint32))
    lay.close()


@pytest.mark.parametrize("qt", QTYPES)
@pytest.mark.parametrize("pooling", POOLS)
def test_quant_pooled(qt, pooling):
    odt, cdt = qt
    count = 64
    rng = np.random.default_rng(odt * 10 + pooling)
    rows, bags = 2000, 300
    tb = quant_table(rng, rows, count, odt)
    off = csr_offsets(rng, bags, 20)
    n = int(off[-1])
    keys = rng.integers(0, rows, size=n).astype(np.int64)
    weighted = pooling in (_lib.POOL_WSUM, _lib.POOL_WMEAN)
    w = rng.uniform(0, 1, size=n).astype(np.float32) if weighted else None
    nat = O.native_out(odt)
    oes = 2 if nat == O.F16 else 4
    lay = GpuLayer(tb, cdt)
    out = torch.zeros((bags, count * oes), dtype=torch.uint8, device="cuda")
    lay.pooled(to_dev(keys), n, out, count * oes, pooling, _lib.SPARSE_CSR, to_dev(off), bags + 1, 0,
               None if w is None else to_dev(w), _lib.DT_F32 if weighted else 0, DT[nat])
    torch.cuda.synchronize()
    ref = oracle_pool(tb, keys, odt, count, O.CSR, pooling, off, bags, 0, w, O.F32, nat)
    got = out.cpu().numpy().view(np.uint16 if nat == O.F16 else np.float32).reshape(bags, count)
    assert np.array_equal(got.view(np.uint16 if nat == O.F16 else np.uint32),
                          ref.view(np.uint16 if nat == O.F16 else np.uint32))
    lay.close()


def test_layer_creation_validation():
    """gpu_layer_test.cpp:371-400,562-581,974-986: an unsupported value type,
    a NULL table, zero rows, a default row outside the table, more rows than
    int32 keys can address, and quantized widths without values are refused
    at creation."""
    L = _lib.load()
    buf = torch.zeros(64, dtype=torch.uint8, device="cuda")

    def create(kt=_lib.KEY_INT64, **fields):
        cfg = L.nve_gpu_embedding_layer_config_default()
        cfg.layer_name = b"v"
        cfg.embedding_table = buf.data_ptr()
        cfg.num_embeddings = 1
        cfg.embedding_width_in_bytes = 4
        cfg.value_dtype = _lib.DT_F32
        for k, v in fields.items():
            setattr(cfg, k, v)
        lay = ctypes.c_void_p()
        st = L.nve_gpu_embedding_layer_create(ctypes.byref(lay), kt, ctypes.byref(cfg), None)
        if st == _lib.SUCCESS:
            _lib.call("nve_layer_destroy", lay)
        return st

    assert create() == _lib.SUCCESS
    assert create(value_dtype=_lib.DT_F64, embedding_width_in_bytes=8) != _lib.SUCCESS
    assert create(embedding_table=None) != _lib.SUCCESS
    assert create(num_embeddings=0) != _lib.SUCCESS
    assert create(num_embeddings=16, default_row_index=16) != _lib.SUCCESS
    assert create(_lib.KEY_INT32, num_embeddings=1 << 31) != _lib.SUCCESS
    assert "cannot be represented" in _lib.last_error()
    for width in (3, 2, 0):
        assert create(value_dtype=_lib.DT_QI8_F16, embedding_width_in_bytes=width) != _lib.SUCCESS, width


def test_lookup_validation_of_output_and_weight_types():
    """gpu_layer_test.cpp:583-607 and 987-1010: a float32 table refuses pooled
    fp16 output and fp16 weights; a quantized table refuses a plain lookup
    narrower than its rows and Concatenate to Unknown or to the other
    precision."""
    rng = np.random.default_rng(5)
    tb = float_table(rng, 4, 16, O.F32)
    lay = GpuLayer(tb, _lib.DT_F32)
    keys = to_dev(np.arange(4, dtype=np.int64))
    out = torch.zeros((4, 64), dtype=torch.uint8, device="cuda")
    w = to_dev(np.ones(4, np.float16).view(np.uint16))
    L = _lib.load()
    assert L.nve_layer_lookup_pooled(lay.layer, lay.ctx, 4, vp(keys), vp(out), 32, None, _lib.POOL_SUM,
                                     _lib.SPARSE_FIXED, None, 0, 2, None, 0, _lib.DT_F16, None) == _lib.INVALID_ARGUMENT
    assert L.nve_layer_lookup_pooled(lay.layer, lay.ctx, 4, vp(keys), vp(out), 64, None, _lib.POOL_WSUM,
                                     _lib.SPARSE_FIXED, None, 0, 2, vp(w), _lib.DT_F16, _lib.DT_F32,
                                     None) == _lib.INVALID_ARGUMENT
    lay.close()
    qt = quant_table(rng, 4, 16, O.QI8_F32)
    lay = GpuLayer(qt, _lib.DT_QI8_F32)
    width = qt.shape[1]
    assert L.nve_layer_lookup(lay.layer, lay.ctx, 1, vp(keys), vp(out), width - 1, None,
                              None) == _lib.INVALID_ARGUMENT
    for odt in (0, _lib.DT_F16):
        assert L.nve_layer_lookup_pooled(lay.layer, lay.ctx, 1, vp(keys), vp(out), 64, None, _lib.POOL_CONCAT,
                                         0, None, 0, 0, None, 0, odt, None) == _lib.INVALID_ARGUMENT, odt
    assert L.nve_layer_lookup_pooled(lay.layer, lay.ctx, 1, vp(keys), vp(out), 64, None, _lib.POOL_CONCAT,
                                     0, None, 0, 0, None, 0, _lib.DT_F32, None) == _lib.SUCCESS
    lay.close()

"""GPU parity of multi-table jagged pooling (BASELINE config 5's shape:
several fp16 tables, Poisson bag lengths, fp32 per-key weights, weighted mean
to an fp32 [batch][table][dim] output) against the oracle run table by table
(the reference pools one table per call, gpu_table.cu:211)."""
import ctypes

import numpy as np
import pytest

from nve_helpers import float_table, quant_table, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

CDT = {O.F32: _lib.DT_F32, O.F16: _lib.DT_F16, O.QI8_F32: _lib.DT_QI8_F32, O.XI8A_F32: _lib.DT_XI8A_F32}


def make_inputs(rng, num_tables, batch, dim, dtype, card_lo=1000, card_hi=100000, max_len=100):
    cards = np.exp(rng.uniform(np.log(card_lo), np.log(card_hi), size=num_tables)).astype(np.int64)
    if dtype in (O.F32, O.F16):
        tabs = [float_table(rng, int(c), dim, dtype, dyadic_values=False) for c in cards]
    else:
        tabs = [quant_table(rng, int(c), dim, dtype) for c in cards]
    lens = np.clip(rng.poisson(20, size=(num_tables, batch)), 1, max_len)
    off = np.zeros(num_tables * batch + 1, np.int64)
    off[1:] = np.cumsum(lens.reshape(-1))
    keys = np.concatenate([
        (O.power_law(rng.random(int(lens[t].sum())), 1, int(cards[t]), 1.1)).astype(np.int64)
        for t in range(num_tables)])
    w = rng.uniform(0, 1, size=keys.size).astype(np.float32)
    return tabs, off, keys, w


def run_multi(tabs, off, keys, w, batch, dtype, pooling, out_dtype, bounded=True, wdt=_lib.DT_F32):
    T = len(tabs)
    width = tabs[0].shape[1]
    count = (width - O.meta_bytes(dtype)) // O.value_bytes(dtype)
    d_tabs = [to_dev(t.reshape(-1)) for t in tabs]
    ptrs = (ctypes.c_void_p * T)(*[d.data_ptr() for d in d_tabs])
    rows = (ctypes.c_int64 * T)(*[t.shape[0] for t in tabs]) if bounded else None
    d_keys, d_off, d_w = to_dev(keys), to_dev(off), to_dev(w)
    oes = 2 if out_dtype == O.F16 else 4
    out = torch.zeros((batch, T * count * oes), dtype=torch.uint8, device="cuda")
    _lib.call("nve_amd_find_and_pool_multi", _lib.KEY_INT64, T, ptrs, rows, width, CDT[dtype], batch,
              keys.size, vp(d_keys), vp(d_off), vp(d_w), wdt, pooling, CDT[out_dtype], vp(out), stream_ptr())
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16 if out_dtype == O.F16 else np.float32).reshape(batch, T, count)


def oracle_multi(tabs, off, keys, w, batch, dtype, pooling, out_dtype):
    T = len(tabs)
    count = (tabs[0].shape[1] - O.meta_bytes(dtype)) // O.value_bytes(dtype)
    res = []
    for t in range(T):
        lo, hi = off[t * batch], off[(t + 1) * batch]
        loc = off[t * batch:(t + 1) * batch + 1] - lo
        kt = keys[lo:hi]
        ptrs = O.linear_row_ptrs(kt, np.ascontiguousarray(tabs[t]).reshape(-1), tabs[t].shape[1])
        res.append(O.pool(ptrs, dtype, count, O.CSR, pooling, kt.size, loc, batch, 0, w[lo:hi], O.F32,
                          out_dtype))
    return np.stack(res, axis=1)


@pytest.mark.parametrize("pooling,out_dtype", [(_lib.POOL_WMEAN, O.F32), (_lib.POOL_SUM, O.F16),
                                               (_lib.POOL_WSUM, O.F32), (_lib.POOL_MEAN, O.F32)])
def test_multi_table_fp16_rows(pooling, out_dtype):
    rng = np.random.default_rng(pooling * 7 + out_dtype)
    batch, dim = 512, 128
    tabs, off, keys, w = make_inputs(rng, 6, batch, dim, O.F16)
    got = run_multi(tabs, off, keys, w, batch, O.F16, pooling, out_dtype)
    ref = oracle_multi(tabs, off, keys, w, batch, O.F16, pooling, out_dtype)
    bits = np.uint16 if out_dtype == O.F16 else np.uint32
    assert np.array_equal(got.view(bits), ref.view(bits))


def test_more_tables_than_one_launch_and_quantized_rows():
    rng = np.random.default_rng(77)
    batch, dim = 64, 32
    tabs, off, keys, w = make_inputs(rng, 70, batch, dim, O.XI8A_F32, card_lo=100, card_hi=2000,
                                     max_len=30)
    got = run_multi(tabs, off, keys, w, batch, O.XI8A_F32, _lib.POOL_WMEAN, O.F32)
    ref = oracle_multi(tabs, off, keys, w, batch, O.XI8A_F32, _lib.POOL_WMEAN, O.F32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("bounded", [True, False])
def test_unbounded_tables_take_the_general_kernel_with_the_same_bits(bounded):
    """Without row counts the launch keeps the general kernel (no bound check,
    64-bit row indices); with them the short-bag kernel runs.  Same sums."""
    rng = np.random.default_rng(91)
    batch, dim = 256, 128
    tabs, off, keys, w = make_inputs(rng, 5, batch, dim, O.F16)
    got = run_multi(tabs, off, keys, w, batch, O.F16, _lib.POOL_WMEAN, O.F32, bounded=bounded)
    ref = oracle_multi(tabs, off, keys, w, batch, O.F16, _lib.POOL_WMEAN, O.F32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_keys_outside_their_table_read_nothing():
    """With row counts, a key outside its own table adds nothing (the bag's
    Mean still counts it), checked against the oracle on tables padded with a
    zero row; fp32 tables, f16 weights."""
    rng = np.random.default_rng(93)
    batch, dim = 128, 64
    tabs, off, keys, w = make_inputs(rng, 4, batch, dim, O.F32)
    bad = rng.random(keys.size) < 0.05
    keys = keys.copy()
    keys[bad] = 10**9
    mapped = keys.copy()
    padded = []
    for t in range(len(tabs)):
        lo, hi = off[t * batch], off[(t + 1) * batch]
        rows = tabs[t].shape[0]
        mapped[lo:hi] = np.where(keys[lo:hi] < rows, keys[lo:hi], rows)
        padded.append(np.concatenate([tabs[t], np.zeros((1, tabs[t].shape[1]), np.uint8)]))
    w16 = w.astype(np.float16)
    for pooling in (_lib.POOL_SUM, _lib.POOL_MEAN, _lib.POOL_WSUM):
        got = run_multi(tabs, off, keys, w16, batch, O.F32, pooling, O.F32, wdt=_lib.DT_F16)
        res = []
        for t in range(len(tabs)):
            lo, hi = off[t * batch], off[(t + 1) * batch]
            loc = off[t * batch:(t + 1) * batch + 1] - lo
            ptrs = O.linear_row_ptrs(mapped[lo:hi], np.ascontiguousarray(padded[t]).reshape(-1),
                                     padded[t].shape[1])
            res.append(O.pool(ptrs, O.F32, dim, O.CSR, pooling, hi - lo, loc, batch, 0,
                              w16[lo:hi].view(np.uint16), O.F16, O.F32))
        ref = np.stack(res, axis=1)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))

"""GPU parity of the kernel-level find-and-pool router (nve_amd_find_and_pool,
restating cuda_ops/find_and_pool.cuh:103-132 over a linear table).

Covers the two reduction shapes (one lane group per bag in key order, which is
bit-exact with the oracle; bags split over lane groups and combined by a fixed
tree, within fp32 tolerance), the long-bag shape of the headline benchmark,
and the two row formats of this build (int8 affine, fp8 e4m3)."""
import ctypes

import numpy as np
import pytest

from nve_helpers import (csr_offsets, pooled_f16_close, float_table, from_dev, oracle_dequant,
                         oracle_pool, quant_table, rel_close, stream_ptr, to_dev, vp)
from oracle import oracle as O
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

CDT = {O.F32: _lib.DT_F32, O.F16: _lib.DT_F16, O.XI8A_F32: _lib.DT_XI8A_F32,
       O.XE4M3_F32: _lib.DT_XE4M3_F32, O.QI8_F32: _lib.DT_QI8_F32, O.QU8_F16: _lib.DT_QU8_F16}


def fap(d_keys, n, d_table, rows, width, vdt, pooling, sparse, d_off, n_off, hot, d_w, wdt, odt,
        d_out, stride, split=0, key_type=_lib.KEY_INT64, unroll=0):
    _lib.call("nve_amd_find_and_pool", key_type, n, vp(d_keys), vp(d_table), rows, width, vdt, pooling,
              sparse, vp(d_off), n_off, hot, vp(d_w), wdt, odt, vp(d_out), stride, split, unroll,
              stream_ptr())


def run_pool(tb, dtype, keys, pooling, sparse, off, bags, hot, w, wdt, out_dtype, split=0, unroll=0):
    rows, width = tb.shape
    count = (width - O.meta_bytes(dtype)) // O.value_bytes(dtype)
    oes = 2 if out_dtype == O.F16 else 4
    out = torch.zeros((bags, count * oes), dtype=torch.uint8, device="cuda")
    fap(to_dev(keys), keys.size, to_dev(tb.reshape(-1)), rows, width, CDT[dtype], pooling, sparse,
        None if off is None else to_dev(off), 0 if off is None else off.size, hot,
        None if w is None else to_dev(w), 0 if w is None else (_lib.DT_F16 if wdt == O.F16 else _lib.DT_F32),
        CDT[out_dtype], out, count * oes, split, unroll=unroll)
    torch.cuda.synchronize()
    return out.cpu().numpy().view(np.uint16 if out_dtype == O.F16 else np.float32).reshape(bags, count)


@pytest.mark.parametrize("split", [-1, 2, 4, 8, 16, 64])
@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_MEAN, _lib.POOL_WMEAN])
@pytest.mark.parametrize("unroll", [8, 16])
def test_split_shapes_on_random_data(split, pooling, unroll):
    rng = np.random.default_rng(11 + split)
    rows, dim, bags, hot = 20000, 128, 48, 300
    tb = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    keys = rng.integers(0, rows, size=bags * hot).astype(np.int64)
    w = rng.uniform(0, 1, size=keys.size).astype(np.float32) if pooling == _lib.POOL_WMEAN else None
    got = run_pool(tb, O.F32, keys, pooling, _lib.SPARSE_FIXED, None, bags, hot, w, O.F32, O.F32, split,
                   unroll)
    ref = oracle_pool(tb, keys, O.F32, dim, O.FIXED, pooling, None, bags, hot, w, O.F32, O.F32)
    if split == -1:
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))  # key order: bit-exact
    else:
        assert rel_close(got, ref, 1e-5)


def test_headline_shape_long_fixed_bags_fp16():
    """256 bags x 1024 keys of 128-dim fp16 rows (the benchmark's pooled shape)
    on a smaller table; fp32 accumulation, fp16 output within 1 ulp."""
    rng = np.random.default_rng(21)
    rows, dim, bags, hot = 200000, 128, 256, 1024
    tb = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    keys = rng.integers(0, rows, size=bags * hot).astype(np.int64)
    got = run_pool(tb, O.F16, keys, _lib.POOL_SUM, _lib.SPARSE_FIXED, None, bags, hot, None, 0, O.F16)
    ref = oracle_pool(tb, keys, O.F16, dim, O.FIXED, O.SUM, None, bags, hot, None, 0, O.F16)
    assert pooled_f16_close(got, ref)


def test_csr_with_empty_and_long_bags():
    rng = np.random.default_rng(31)
    rows, dim, bags = 5000, 64, 200
    tb = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    lens = rng.integers(0, 4, size=bags)
    lens[::17] = 0
    lens[5] = 3000  # one very long bag among short ones
    off = np.zeros(bags + 1, np.int64)
    off[1:] = np.cumsum(lens)
    keys = rng.integers(0, rows, size=int(off[-1])).astype(np.int64)
    w = rng.uniform(0, 1, size=keys.size).astype(np.float16)
    for pooling in (_lib.POOL_MEAN, _lib.POOL_WSUM):
        ww = w.view(np.uint16) if pooling == _lib.POOL_WSUM else None
        got = run_pool(tb, O.F16, keys, pooling, _lib.SPARSE_CSR, off, bags, 0, ww, O.F16, O.F16)
        ref = oracle_pool(tb, keys, O.F16, dim, O.CSR, pooling, off, bags, 0, ww, O.F16, O.F16)
        assert np.array_equal(got, ref)
        assert np.all(got[lens == 0] == 0)  # empty bag -> zero row


def test_int32_keys_and_offsets():
    rng = np.random.default_rng(41)
    rows, dim, bags = 3000, 32, 500
    tb = float_table(rng, rows, dim, O.F32)
    off = csr_offsets(rng, bags, 12, np.int32)
    keys = rng.integers(0, rows, size=int(off[-1])).astype(np.int32)
    out = torch.zeros((bags, dim), dtype=torch.float32, device="cuda")
    fap(to_dev(keys), keys.size, to_dev(tb.reshape(-1)), rows, dim * 4, _lib.DT_F32, _lib.POOL_SUM,
        _lib.SPARSE_CSR, to_dev(off), off.size, 0, None, 0, _lib.DT_F32, out, dim * 4, 0, _lib.KEY_INT32)
    torch.cuda.synchronize()
    ref = oracle_pool(tb, keys, O.F32, dim, O.CSR, O.SUM, off, bags, 0, None, 0, O.F32)
    assert np.array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("dtype,out_dtype", [(O.XI8A_F32, O.F16), (O.XI8A_F32, O.F32),
                                             (O.XE4M3_F32, O.F32), (O.XE4M3_F32, O.F16)])
def test_extension_row_formats_dequant_and_pool(dtype, out_dtype):
    rng = np.random.default_rng(dtype + out_dtype)
    rows, count, n = 4000, 256, 3000
    tb = quant_table(rng, rows, count, dtype)
    keys = rng.integers(0, rows, size=n).astype(np.int64)
    oes = 2 if out_dtype == O.F16 else 4
    out = torch.zeros((n, count * oes), dtype=torch.uint8, device="cuda")
    fap(to_dev(keys), n, to_dev(tb.reshape(-1)), rows, tb.shape[1], CDT[dtype], _lib.POOL_CONCAT, 0, None,
        0, 0, None, 0, CDT[out_dtype], out, count * oes)
    torch.cuda.synchronize()
    ref = oracle_dequant(tb, keys, dtype, count, out_dtype)
    bits = np.uint16 if out_dtype == O.F16 else np.uint32
    assert np.array_equal(out.cpu().numpy().view(bits).reshape(n, count), ref.view(bits))
    # pooled, key order
    bags = 300
    hot = n // bags
    got = run_pool(tb, dtype, keys[:bags * hot], _lib.POOL_SUM, _lib.SPARSE_FIXED, None, bags, hot, None,
                   0, out_dtype, split=-1)
    refp = oracle_pool(tb, keys[:bags * hot], dtype, count, O.FIXED, O.SUM, None, bags, hot, None, 0,
                       out_dtype)
    assert np.array_equal(got.view(bits), refp.view(bits))


def test_e4m3_every_code_decodes_exactly():
    """One row holding all 256 fp8 codes (NaN codes included), scale 1."""
    count = 256
    tb = np.zeros((1, count + 4), np.uint8)
    tb[0, :count] = np.arange(256, dtype=np.uint8)
    tb[0, count:] = np.float32(1.0).reshape(1).view(np.uint8)
    keys = np.zeros(1, np.int64)
    out = torch.zeros((1, count * 4), dtype=torch.uint8, device="cuda")
    fap(to_dev(keys), 1, to_dev(tb.reshape(-1)), 1, tb.shape[1], _lib.DT_XE4M3_F32, _lib.POOL_CONCAT, 0,
        None, 0, 0, None, 0, _lib.DT_F32, out, count * 4)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.float32).reshape(-1)
    ref = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # NaN codes included, bit for bit with the oracle: S.1111.111 decodes to
    # the quiet NaN with the code's sign (S = 0 and S = 1 both)
    orc = oracle_dequant(tb, keys, O.XE4M3_F32, count, O.F32).reshape(-1)
    assert np.array_equal(got.view(np.uint32), orc.view(np.uint32))
    assert got.view(np.uint32)[0x7F] == 0x7FC00000 and got.view(np.uint32)[0xFF] == 0xFFC00000


@pytest.mark.parametrize("dtype", [O.F16, O.XI8A_F32])
@pytest.mark.parametrize("split", [-1, 8])
def test_out_of_range_keys_read_as_zero_rows(dtype, split):
    """Keys outside [0, num_rows) add a zero row to their bag (and count in its
    Mean); checked against the oracle on the table plus one zero row."""
    rng = np.random.default_rng(21 + split)
    rows, count, bags, hot = 500, 64, 12, 40
    tb = (float_table(rng, rows, count, dtype, dyadic_values=False) if dtype == O.F16
          else quant_table(rng, rows, count, dtype))
    keys = rng.integers(0, rows, size=bags * hot).astype(np.int64)
    bad = rng.random(keys.size) < 0.2
    keys[bad] = rng.choice(np.array([-1, rows, rows + 7, 1 << 40, -(1 << 50)], np.int64), size=int(bad.sum()))
    padded = np.concatenate([tb, np.zeros((1, tb.shape[1]), np.uint8)])
    mapped = np.where((keys >= 0) & (keys < rows), keys, rows)
    out_dtype = O.F16 if dtype == O.F16 else O.F32  # fp16 rows pool to fp16 (find_and_pool.cuh:40-51)
    bits = np.uint16 if out_dtype == O.F16 else np.uint32
    for pooling in (_lib.POOL_SUM, _lib.POOL_MEAN):
        got = run_pool(tb, dtype, keys, pooling, _lib.SPARSE_FIXED, None, bags, hot, None, O.F32,
                       out_dtype, split)
        ref = oracle_pool(padded, mapped, dtype, count, O.FIXED, pooling, None, bags, hot, None, O.F32,
                          out_dtype)
        if split == -1:
            assert np.array_equal(got.view(bits), ref.view(bits))
        elif out_dtype == O.F16:
            assert pooled_f16_close(got.view(np.uint16), ref.view(np.uint16))
        else:
            assert rel_close(got, ref, 1e-5)


@pytest.mark.parametrize("dtype,dim", [(O.F16, 64), (O.F16, 128), (O.F32, 128), (O.F16, 512), (O.F32, 256)])
@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_MEAN, _lib.POOL_WSUM, _lib.POOL_WMEAN])
@pytest.mark.parametrize("split", [0, 8, 64])
def test_long_bag_kernel_matches_general_kernel_bitwise(dtype, dim, pooling, split):
    """Long bags over a linear f16/f32 table take the lean split-bag kernel
    (unroll hint 0); an unroll hint forces the general kernel.  Both cut a bag
    into the same chunks and add them in the same order, so their outputs must
    be identical bit for bit -- and within fp32 tolerance of the key-order
    oracle.  Keys outside the table (read as nothing) are mixed in."""
    rng = np.random.default_rng(1000 + dim + 7 * pooling + split)
    rows, bags, hot = 30000, 40, 700
    tb = float_table(rng, rows, dim, dtype, dyadic_values=False)
    keys = rng.integers(0, rows, size=bags * hot).astype(np.int64)
    keys[rng.uniform(size=keys.size) < 0.01] = rows + 5  # outside the table
    weighted = pooling in (_lib.POOL_WSUM, _lib.POOL_WMEAN)
    w = rng.uniform(0, 1, size=keys.size).astype(np.float32) if weighted else None
    got = [run_pool(tb, dtype, keys, pooling, _lib.SPARSE_FIXED, None, bags, hot, w, O.F32, dtype, split, unroll)
           for unroll in (0, 16, 8)]
    bits = np.uint16 if dtype == O.F16 else np.uint32
    assert np.array_equal(got[0].view(bits), got[1].view(bits))
    assert np.array_equal(got[0].view(bits), got[2].view(bits))
    padded = np.concatenate([tb, np.zeros((1, tb.shape[1]), np.uint8)])
    mapped = np.where(keys < rows, keys, rows)
    ref = oracle_pool(padded, mapped, dtype, dim, O.FIXED, pooling, None, bags, hot, w, O.F32, dtype)
    if dtype == O.F16:
        assert pooled_f16_close(got[0].view(np.uint16), ref.view(np.uint16))
    else:
        assert rel_close(got[0], ref, 1e-5)


def test_long_bag_kernel_csr_empty_and_int32():
    """CSR bags with empty and very long bags, int32 keys and offsets: the
    lean kernel equals the general one bitwise and the oracle within fp32
    tolerance (empty bags give zero rows)."""
    rng = np.random.default_rng(77)
    rows, dim, bags = 20000, 128, 64
    tb = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    lens = rng.integers(500, 1500, size=bags)
    lens[::9] = 0
    off = np.zeros(bags + 1, np.int32)
    off[1:] = np.cumsum(lens)
    keys = rng.integers(0, rows, size=int(off[-1])).astype(np.int32)
    res = []
    for unroll in (0, 16):
        out = torch.zeros((bags, dim), dtype=torch.float32, device="cuda")
        fap(to_dev(keys), keys.size, to_dev(tb.reshape(-1)), rows, dim * 4, _lib.DT_F32, _lib.POOL_MEAN,
            _lib.SPARSE_CSR, to_dev(off), off.size, 0, None, 0, _lib.DT_F32, out, dim * 4, 0, _lib.KEY_INT32,
            unroll)
        torch.cuda.synchronize()
        res.append(out.cpu().numpy())
    assert np.array_equal(res[0].view(np.uint32), res[1].view(np.uint32))
    ref = oracle_pool(tb, keys, O.F32, dim, O.CSR, O.MEAN, off, bags, 0, None, 0, O.F32)
    assert rel_close(res[0], ref, 1e-5)
    assert np.all(res[0][lens == 0] == 0)


@pytest.mark.parametrize("dtype,dim", [(O.F16, 64), (O.F16, 128), (O.F32, 128), (O.F16, 512), (O.F32, 256)])
@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_MEAN, _lib.POOL_WSUM, _lib.POOL_WMEAN])
def test_short_bag_kernel_matches_general_kernel_and_oracle(dtype, dim, pooling):
    """Short CSR bags over a linear f16/f32 table take the lean short-bag
    kernel (unroll hint 0); an unroll hint forces the general kernel.  One
    lane group per bag in key order, so both equal the key-order oracle bit
    for bit; empty bags and keys outside the table included."""
    rng = np.random.default_rng(2000 + dim + 11 * pooling)
    rows, bags = 20000, 700
    tb = float_table(rng, rows, dim, dtype, dyadic_values=False)
    off = csr_offsets(rng, bags, 45)
    keys = rng.integers(0, rows, size=int(off[-1])).astype(np.int64)
    keys[rng.uniform(size=keys.size) < 0.02] = rows + 3
    weighted = pooling in (_lib.POOL_WSUM, _lib.POOL_WMEAN)
    w = rng.uniform(0, 1, size=keys.size).astype(np.float32) if weighted else None
    got = [run_pool(tb, dtype, keys, pooling, _lib.SPARSE_CSR, off, bags, 0, w, O.F32, dtype, 0, unroll)
           for unroll in (0, 8)]
    bits = np.uint16 if dtype == O.F16 else np.uint32
    assert np.array_equal(got[0].view(bits), got[1].view(bits))
    padded = np.concatenate([tb, np.zeros((1, tb.shape[1]), np.uint8)])
    mapped = np.where(keys < rows, keys, rows)
    ref = oracle_pool(padded, mapped, dtype, dim, O.CSR, pooling, off, bags, 0, w, O.F32, dtype)
    assert np.array_equal(got[0].view(bits), ref.view(bits))


@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_WMEAN])
def test_short_bags_with_offsets_out_of_order(pooling):
    """CSR offsets that are not ascending (bags out of order, overlapping, and
    ends before starts, which make empty bags): the short-bag kernel stages
    each bag's keys on its own then, and still adds them in key order, bit for
    bit with the oracle; workgroups with ascending offsets beside them take the
    shared staging."""
    rng = np.random.default_rng(77 + pooling)
    rows, dim, bags = 5000, 128, 300
    tb = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    n = 4000
    keys = rng.integers(0, rows, size=n).astype(np.int64)
    keys[rng.uniform(size=n) < 0.03] = rows + 9
    off = np.sort(rng.integers(0, n + 1, size=bags + 1)).astype(np.int64)
    shuffled = rng.permutation(np.arange(40, 120))  # some workgroups out of order
    off[40:120] = off[shuffled]
    off[0], off[-1] = 0, n
    weighted = pooling == _lib.POOL_WMEAN
    w = rng.uniform(0, 1, size=n).astype(np.float32) if weighted else None
    got = run_pool(tb, O.F16, keys, pooling, _lib.SPARSE_CSR, off, bags, 0, w, O.F32, O.F16, 0, 0)
    padded = np.concatenate([tb, np.zeros((1, tb.shape[1]), np.uint8)])
    mapped = np.where(keys < rows, keys, rows)
    ref = oracle_pool(padded, mapped, O.F16, dim, O.CSR, pooling, off, bags, 0, w, O.F32, O.F16)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))

"""Pins of the oracle's CPU HostLayer arithmetic (orc_convert_host and the
element values orc_pool_host adds), independent of the oracle's own code.

cpu_pooling.hpp:166-259 and :302-341 widen a quantized element as
float(q) * scale + offset; the oracle takes that as one fused multiply-add.
Here the same value is computed in float64, where q * scale + offset is exact
for these inputs (q has 8 significant bits, scale and offset 24, and their
exponents lie within 30 of each other), then rounded to float32 once.  A
separate multiply and add (two roundings), a dropped offset or a wrong
metadata position fails these checks."""
import numpy as np
import pytest

from oracle import oracle as O


def quant_rows(rng, rows, count, dtype):
    meta = O.meta_bytes(dtype)
    out = np.zeros((rows, count + meta), np.uint8)
    out[:, :count] = rng.integers(0, 256, size=(rows, count), dtype=np.uint8)
    scale = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), size=rows))
    off = rng.normal(0, 0.01, size=rows)
    if dtype in (O.QI8_F32, O.QU8_F32, O.XI8A_F32, O.XE4M3_F32):
        s32 = scale.astype(np.float32)
        out[:, count:count + 4] = s32.view(np.uint8).reshape(rows, 4)
        s, o = s32.astype(np.float64), np.zeros(rows)
        if dtype in (O.QU8_F32, O.XI8A_F32):
            o32 = off.astype(np.float32)
            out[:, count + 4:count + 8] = o32.view(np.uint8).reshape(rows, 4)
            o = o32.astype(np.float64)
    else:
        s16 = scale.astype(np.float16)
        out[:, count:count + 2] = s16.view(np.uint8).reshape(rows, 2)
        s, o = s16.astype(np.float64), np.zeros(rows)
        if dtype == O.QU8_F16:
            o16 = off.astype(np.float16)
            out[:, count + 2:count + 4] = o16.view(np.uint8).reshape(rows, 2)
            o = o16.astype(np.float64)
    return out, s, o


def expected_values(rows, s, o, dtype, count):
    q = rows[:, :count]
    if dtype in (O.QI8_F32, O.QI8_F16, O.XI8A_F32):
        qv = q.view(np.int8).astype(np.float64)
    elif dtype == O.XE4M3_F32:
        import torch
        qv = torch.from_numpy(np.ascontiguousarray(q)).view(torch.float8_e4m3fn).double().numpy()
    else:
        qv = q.astype(np.float64)
    if dtype == O.XE4M3_F32:  # e4m3(q) * scale: one product, rounded once
        return (qv * s[:, None]).astype(np.float32)
    return (qv * s[:, None] + o[:, None]).astype(np.float32)


@pytest.mark.parametrize("dtype", [O.QI8_F32, O.QI8_F16, O.QU8_F32, O.QU8_F16, O.XI8A_F32, O.XE4M3_F32])
@pytest.mark.parametrize("out_dtype", [O.F32, O.F16])
def test_convert_host_closed_form(dtype, out_dtype):
    rng = np.random.default_rng(dtype * 10 + out_dtype)
    count = 48
    rows, s, o = quant_rows(rng, 200, count, dtype)
    if dtype == O.XE4M3_F32:
        q = rows[:, :count]
        q[(q & 0x7F) == 0x7F] = 0x3C  # no NaN codes
    want = expected_values(rows, s, o, dtype, count)
    got = O.convert_rows_host(rows, dtype, count, out_dtype)
    if out_dtype == O.F32:
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    else:
        assert np.array_equal(got, want.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("src,dst", [(O.F32, O.F16), (O.F16, O.F32), (O.F32, O.F32), (O.F16, O.F16)])
def test_convert_host_float_casts(src, dst):
    rng = np.random.default_rng(3)
    v = rng.normal(0, 4, size=(50, 33))
    rows = v.astype(np.float32 if src == O.F32 else np.float16)
    got = O.convert_rows_host(rows.view(np.uint8), src, 33, dst)
    want = rows.astype(np.float16 if dst == O.F16 else np.float32)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))


@pytest.mark.parametrize("dtype", [O.QI8_F16, O.QU8_F32, O.XE4M3_F32])
def test_pool_host_single_key_bags_are_the_element_values(dtype):
    """A Sum bag of one key is its row's element values (acc = 0 + v, times 1)."""
    rng = np.random.default_rng(7 + dtype)
    count = 40
    rows, s, o = quant_rows(rng, 64, count, dtype)
    if dtype == O.XE4M3_F32:
        q = rows[:, :count]
        q[(q & 0x7F) == 0x7F] = 0x3C
    want = expected_values(rows, s, o, dtype, count) + np.float32(0)  # 0 + (-0) is +0
    tb = np.ascontiguousarray(rows).reshape(-1)
    keys = np.arange(64, dtype=np.int64)
    got = O.pool(O.linear_row_ptrs(keys, tb, rows.shape[1]), dtype, count, O.FIXED, O.SUM, 64, None, 64, 1,
                 None, 0, O.F32, host_order=True)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_pool_host_weighted_product_is_rounded_before_the_add():
    """cpu_pooling.hpp:118-124: v *= w, then acc += v.  Key 0 adds 1; key 1 has
    x = 1 + 2^-23 and w = 1 + 2^-7, so x*w = 1 + 2^-7 + 2^-23 + 2^-30 rounds
    to 1 + 2^-7 + 2^-23, and 1 + that = 2 + 2^-7 + 2^-23 is a tie that rounds
    to even: 2 + 2^-7.  A fused x*w + 1 keeps 2^-30 and rounds up to
    2 + 2^-7 + 2^-22 (the GPU order, orc_pool, which fuses)."""
    x = np.float32(1 + 2.0 ** -23)
    rows = np.array([[1.0], [x]], np.float32)
    w = np.array([1.0, 1 + 2.0 ** -7], np.float32)
    tb = rows.view(np.uint8).reshape(-1)
    keys = np.array([0, 1], np.int64)
    args = (O.linear_row_ptrs(keys, tb, 4), O.F32, 1, O.FIXED, O.WSUM, 2, None, 1, 2, w, O.F32, O.F32)
    assert O.pool(*args, host_order=True)[0, 0] == np.float32(2 + 2.0 ** -7)
    assert O.pool(*args)[0, 0] == np.float32(2 + 2.0 ** -7 + 2.0 ** -22)

"""Pins for the oracle's scalar conversions, dequant and pooling.

Each check compares the oracle with something independent of it: numpy /
torch casts (library routines), closed forms evaluated in float64, or exact
arithmetic on dyadic fractions.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O


def test_f16_to_f32_all_codes_match_numpy():
    codes = np.arange(65536, dtype=np.uint16)
    ours = O.f16_to_f32(codes)
    ref = codes.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy():
    rng = np.random.default_rng(7)
    # random bit patterns cover every exponent incl. subnormal / overflow ranges
    bits = rng.integers(0, 2**32, size=1_000_000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[~np.isnan(vals)]
    # exact ties: halfway cases in the normal and subnormal half ranges
    ties = np.array([1.0 + 2.0**-11, 1.0 + 3 * 2.0**-11, 2.0**-24 * 0.5, 2.0**-24 * 1.5,
                     65504.0, 65519.0, 65520.0, -65520.0, 2.0**-25, 6.1035156e-05], np.float32)
    vals = np.concatenate([vals, ties])
    ours = O.f32_to_f16(vals)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_e4m3_all_codes_match_torch_ocp_fn():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).to(torch.float32).numpy()
    ours = np.array([O.e4m3_to_f32(c) for c in range(256)], np.float32)
    nan = np.isnan(ref)
    assert nan.sum() == 2  # 0x7F and 0xFF
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0**-9


def test_sanitize_closed_form():
    keys = np.array([0, 5, 9, 10, -1, -100, 2**40, 3], np.int64)
    out = O.sanitize(keys, 10, 7)
    assert out.tolist() == [0, 5, 9, 7, 7, 7, 7, 3]
    k32 = keys.astype(np.int32)
    out32 = O.sanitize(k32, 10, 2)
    exp = [k if 0 <= k < 10 else 2 for k in k32.tolist()]
    assert out32.tolist() == exp


def test_gather_brute_force_with_hitmask_and_out_of_range():
    rng = np.random.default_rng(1)
    rows, rb = 100, 24
    table = rng.integers(0, 256, size=rows * rb, dtype=np.uint8)
    keys = rng.integers(-20, rows + 20, size=200).astype(np.int64)
    mask = np.zeros(4, np.uint64)
    mask[0] = np.uint64(0xF0F0F0F0F0F0F0F0)
    before = mask.copy()
    out = np.full((200, rb), 0xAB, np.uint8)
    out, hits = O.gather(keys, table, rb, rows, hit_mask=mask, out=out)
    exp_hits = 0
    for i, k in enumerate(keys.tolist()):
        pre = (int(before[i // 64]) >> (i % 64)) & 1
        if pre or not (0 <= k < rows):
            assert (out[i] == 0xAB).all()
            assert ((int(mask[i // 64]) >> (i % 64)) & 1) == pre
        else:
            exp_hits += 1
            assert np.array_equal(out[i], table[k * rb:(k + 1) * rb])
            assert (int(mask[i // 64]) >> (i % 64)) & 1
    assert hits == exp_hits


def _quant_rows(rng, n, count, dtype):
    """Build stored rows [values][scale][offset?] and the float64 closed form."""
    meta = O.meta_bytes(dtype)
    rows = np.zeros((n, count + meta), np.uint8)
    if dtype in (O.QI8_F32, O.QI8_F16, O.XI8A_F32):
        q = rng.integers(-127, 128, size=(n, count)).astype(np.int8)
        rows[:, :count] = q.view(np.uint8)
        qf = q.astype(np.float64)
    elif dtype == O.XE4M3_F32:
        codes = rng.integers(0, 256, size=(n, count)).astype(np.uint8)
        codes[(codes & 0x7F) == 0x7F] = 0x10  # no NaN payloads
        rows[:, :count] = codes
        qf = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    else:
        q = rng.integers(0, 256, size=(n, count)).astype(np.uint8)
        rows[:, :count] = q
        qf = q.astype(np.float64)
    if dtype in (O.QI8_F32, O.QU8_F32, O.XI8A_F32, O.XE4M3_F32):
        s = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), n)).astype(np.float32)
        o = rng.normal(0, 0.01, n).astype(np.float32)
        rows[:, count:count + 4] = s.view(np.uint8).reshape(n, 4)
        if dtype in (O.QU8_F32, O.XI8A_F32):
            rows[:, count + 4:count + 8] = o.view(np.uint8).reshape(n, 4)
        else:
            o = np.zeros(n, np.float32)
    else:
        s = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), n)).astype(np.float16)
        o = rng.normal(0, 0.01, n).astype(np.float16)
        rows[:, count:count + 2] = s.view(np.uint8).reshape(n, 2)
        if dtype == O.QU8_F16:
            rows[:, count + 2:count + 4] = o.view(np.uint8).reshape(n, 2)
        else:
            o = np.zeros(n, np.float16)
    exact = qf * s.astype(np.float64)[:, None] + o.astype(np.float64)[:, None]
    return rows, exact


@pytest.mark.parametrize("dtype", [O.QI8_F32, O.QU8_F32, O.XI8A_F32, O.XE4M3_F32])
def test_dequant_f32_meta_closed_form(dtype):
    rng = np.random.default_rng(dtype)
    count = 64
    rows, exact = _quant_rows(rng, 200, count, dtype)
    got = O.dequant_rows(rows, dtype, count, O.F32)
    ref = exact.astype(np.float32)  # one rounding of the float64 value
    if dtype in (O.QI8_F32, O.XE4M3_F32):
        # product of two floats is exact in float64: single rounding, bit-exact
        assert np.array_equal(got, ref)
    else:
        # fma = single rounding of the exact value; float64 evaluation may round
        # twice, so allow a rare 1-ulp disagreement
        ulp = np.spacing(np.abs(ref))
        diff = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        assert (diff <= ulp).all()
        assert (diff > 0).mean() < 1e-3


@pytest.mark.parametrize("dtype", [O.QI8_F16, O.QU8_F16])
def test_dequant_f16_meta_closed_form(dtype):
    rng = np.random.default_rng(dtype + 100)
    count = 48
    rows, exact = _quant_rows(rng, 200, count, dtype)
    got = O.dequant_rows(rows, dtype, count, O.F16).view(np.float16)
    ref = exact.astype(np.float32).astype(np.float16)
    if dtype == O.QI8_F16:
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    else:
        ulp = np.spacing(np.abs(ref)).astype(np.float64)
        assert (np.abs(got.astype(np.float64) - ref.astype(np.float64)) <= ulp).all()
    # the F32 output of an F16-metadata row is the half value widened exactly
    got32 = O.dequant_rows(rows, dtype, count, O.F32)
    assert np.array_equal(got32, got.astype(np.float32))


def _dyadic_table(rng, rows, dim):
    # nom in [-8, 8] over 2^[3, 9]: sums of a few thousand stay exact in fp32
    nom = rng.integers(-8, 9, size=(rows, dim)).astype(np.float64)
    den = 2.0 ** rng.integers(3, 10, size=(rows, dim))
    return (nom / den)


@pytest.mark.parametrize("dtype", [O.F32, O.F16])
@pytest.mark.parametrize("sparse", [O.FIXED, O.CSR])
def test_pool_sum_is_exact_on_dyadic_table(dtype, sparse):
    rng = np.random.default_rng(3)
    rows, dim = 500, 33
    t = _dyadic_table(rng, rows, dim)
    table = (t.astype(np.float32) if dtype == O.F32 else t.astype(np.float16))
    tb = table.view(np.uint8).reshape(-1)
    rb = table.strides[0]
    if sparse == O.FIXED:
        hot = 7
        nb = 40
        keys = rng.integers(0, rows, size=nb * hot).astype(np.int64)
        offsets = None
        spans = [(b * hot, (b + 1) * hot) for b in range(nb)]
    else:
        lens = rng.integers(0, 30, size=50)
        offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
        keys = rng.integers(0, rows, size=int(offsets[-1])).astype(np.int64)
        nb, hot = 50, 0
        spans = [(int(offsets[b]), int(offsets[b + 1])) for b in range(nb)]
    ptrs = O.linear_row_ptrs(keys, tb, rb)
    for out_dtype in (O.F32, O.F16):
        got = O.pool(ptrs, dtype, dim, sparse, O.SUM, keys.size, offsets, nb, hot, None, O.F32, out_dtype)
        exp = np.stack([t[keys[s:e]].sum(axis=0) if e > s else np.zeros(dim) for s, e in spans])
        if out_dtype == O.F32:
            assert np.array_equal(got, exp.astype(np.float32))
        else:
            assert np.array_equal(got, exp.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("host_order", [False, True])
@pytest.mark.parametrize("mode", ["mean", "wsum", "wmean", "sum"])
def test_pool_matches_torch_embedding_bag(mode, host_order):
    rng = np.random.default_rng(11)
    rows, dim = 300, 40
    table = rng.normal(0, 0.5, size=(rows, dim)).astype(np.float32)
    tb = table.view(np.uint8).reshape(-1)
    lens = rng.integers(0, 25, size=64)
    lens[5] = 0
    offsets = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    keys = rng.integers(0, rows, size=int(offsets[-1])).astype(np.int64)
    w = rng.uniform(0, 1, size=keys.size).astype(np.float32)
    pooling = {"sum": O.SUM, "mean": O.MEAN, "wsum": O.WSUM, "wmean": O.WMEAN}[mode]
    weighted = mode in ("wsum", "wmean")
    ptrs = O.linear_row_ptrs(keys, tb, table.strides[0])
    got = O.pool(ptrs, O.F32, dim, O.CSR, pooling, keys.size, offsets, 64, 0,
                 w if weighted else None, O.F32, O.F32, host_order=host_order)
    t64 = torch.from_numpy(table.astype(np.float64))
    kk = torch.from_numpy(keys)
    oo = torch.from_numpy(offsets)
    ww = torch.from_numpy(w.astype(np.float64)) if weighted else None
    if mode == "wmean":
        num = torch.nn.functional.embedding_bag(kk, t64, oo, mode="sum", per_sample_weights=ww,
                                                include_last_offset=True)
        den = torch.tensor([w[offsets[b]:offsets[b + 1]].astype(np.float64).sum() for b in range(64)])
        ref = torch.where(den[:, None] != 0, num / den.clamp_min(1e-300)[:, None], torch.zeros_like(num))
    else:
        ref = torch.nn.functional.embedding_bag(kk, t64, oo, mode="mean" if mode == "mean" else "sum",
                                                per_sample_weights=ww, include_last_offset=True)
    ref = ref.numpy()
    assert np.all(got[5] == 0)
    scale = np.abs(table).max() * (lens.max() + 1)
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-6 * scale)


def test_pool_f16_metadata_rows_round_to_half_before_accumulating():
    # GPU order dequantizes QInt8RowwiseF16 to a half first (kernels_common.cuh:247);
    # the CPU order keeps the float product.  Build a row where that matters.
    count = 4
    row = np.zeros(count + 2, np.uint8)
    q = np.array([3, 5, 7, 1], np.int8)
    row[:count] = q.view(np.uint8)
    s = np.float16(0.0999)
    row[count:] = np.array([s]).view(np.uint8)
    rows = np.stack([row, row])
    ptrs = (np.arange(2, dtype=np.uint64) * np.uint64(row.size) + np.uint64(rows.ctypes.data))
    gpu = O.pool(ptrs, O.QI8_F16, count, O.FIXED, O.SUM, 2, None, 1, 2, None, O.F32, O.F32)
    cpu = O.pool(ptrs, O.QI8_F16, count, O.FIXED, O.SUM, 2, None, 1, 2, None, O.F32, O.F32, host_order=True)
    halfs = (q.astype(np.float32) * np.float32(s)).astype(np.float16).astype(np.float32)
    assert np.array_equal(gpu[0], halfs + halfs)
    assert np.array_equal(cpu[0], (q.astype(np.float32) * np.float32(s)) * 2)


def test_host_layer_lookup_threads_agree_and_match_torch():
    rng = np.random.default_rng(5)
    rows, dim = 10000, 64
    table = rng.normal(0, 0.01, size=(rows, dim)).astype(np.float32)
    tb = table.view(np.uint8).reshape(-1)
    keys = rng.integers(0, rows, size=4096 * 8).astype(np.int64)
    outs = [O.host_layer_lookup(keys, tb, rows, dim * 4, O.F32, O.SUM, O.FIXED, None, 4096, 8,
                                None, O.F32, O.F32, th) for th in (1, 3, 6)]
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])
    ref = table[keys].reshape(4096, 8, dim).astype(np.float64).sum(axis=1)
    assert np.allclose(outs[0], ref, rtol=1e-6, atol=1e-7)
    g = O.host_layer_lookup(keys, tb, rows, dim * 4, O.F32, O.CONCAT, O.FIXED, None, 0, 0, None,
                            O.F32, O.F32, 4)
    assert np.array_equal(g.view(np.float32).reshape(-1, dim), table[keys])

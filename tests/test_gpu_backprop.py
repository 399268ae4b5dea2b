"""GPU parity of the training backprop (nve_amd_pooling_backprop, restating
GradientCalculator::compute_gradients, cuda_ops/gradient_calculator.cuh:238-301)
against the oracle (orc_pooling_backprop, itself pinned to torch autograd).

Both add each unique key's positions in pieces (its positions inside one
32-position block of the dedup order, fp32, position order), then the pieces in
eight sub-sequences and their sums in order, rounding once, so unique keys and
gradient rows must match bit for bit.  Cases follow
tests/kernels/pooling_backprop_tests.cu: Concatenate / Sum / Mean / WeightedSum
/ WeightedMean, Fixed and CSR bags, int32 and int64 keys, plus fp16 gradients,
Zipf keys whose hottest key spans many blocks, empty bags and positions outside
every bag, row widths of every lane layout (odd widths, rows wider than one
pass of a lane group) and unaligned gradient buffers."""
import ctypes

import numpy as np
import pytest

from nve_helpers import stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

POOL = {O.CONCAT: _lib.POOL_CONCAT, O.SUM: _lib.POOL_SUM, O.MEAN: _lib.POOL_MEAN,
        O.WSUM: _lib.POOL_WSUM, O.WMEAN: _lib.POOL_WMEAN}


def gpu_backprop(keys, pooling, sparse, offsets, hot, w, wdt, g, gdt, dim):
    n = keys.size
    kt = _lib.KEY_INT32 if keys.dtype == np.int32 else _lib.KEY_INT64
    bags = 0 if pooling == O.CONCAT else (offsets.size - 1 if sparse == O.CSR else n // hot)
    wsb = ctypes.c_uint64()
    _lib.call("nve_amd_backprop_workspace_size", n, bags, dim, ctypes.byref(wsb))
    ws = torch.empty(max(int(wsb.value), 1), dtype=torch.uint8, device="cuda")
    uq = torch.zeros(max(n, 1), dtype=torch.int32 if kt == _lib.KEY_INT32 else torch.int64, device="cuda")
    ges = 2 if gdt == O.F16 else 4
    out = torch.zeros((max(n, 1), dim * ges), dtype=torch.uint8, device="cuda")
    nu = ctypes.c_int64(-1)
    # device copies kept alive until the call returns (a freed temporary's
    # block would be handed to the next allocation)
    d_keys = to_dev(keys) if n else None
    d_off = to_dev(offsets) if offsets is not None else None
    d_w = to_dev(w) if w is not None else None
    d_g = to_dev(g.reshape(-1))
    _lib.call("nve_amd_pooling_backprop", kt, n, vp(d_keys) if n else None, POOL[pooling],
              _lib.SPARSE_CSR if sparse == O.CSR else _lib.SPARSE_FIXED,
              vp(d_off) if d_off is not None else None, 0 if offsets is None else offsets.size, hot,
              vp(d_w) if d_w is not None else None,
              (_lib.DT_F16 if wdt == O.F16 else _lib.DT_F32) if w is not None else _lib.DT_UNKNOWN,
              vp(d_g), _lib.DT_F16 if gdt == O.F16 else _lib.DT_F32, dim, vp(uq), vp(out),
              ctypes.byref(nu), vp(ws), wsb.value, stream_ptr())
    torch.cuda.synchronize()
    u = nu.value
    bits = np.uint16 if gdt == O.F16 else np.uint32
    return uq.cpu().numpy()[:u], out.cpu().numpy()[:u].view(bits)


def make_case(rng, pooling, sparse, key_dtype, wdt, gdt, bags=150, hot=40, rows=5000, dim=64):
    if sparse == O.FIXED or pooling == O.CONCAT:
        offsets = None
        n = bags * hot
    else:
        lens = rng.integers(0, 2 * hot, size=bags)
        lens[::13] = 0
        offsets = np.zeros(bags + 1, key_dtype)
        offsets[1:] = np.cumsum(lens)
        n = int(offsets[-1])
    keys = (rng.zipf(1.15, size=n) % rows).astype(key_dtype)  # the hottest key spans many runs
    w = None
    if pooling in (O.WSUM, O.WMEAN):
        w = rng.uniform(0.1, 1.0, size=n).astype(np.float16 if wdt == O.F16 else np.float32)
    grows = n if pooling == O.CONCAT else bags
    g = rng.normal(0, 1, size=(grows, dim)).astype(np.float16 if gdt == O.F16 else np.float32)
    return keys, offsets, n, w, g


# Concatenate has no bags, so it takes no sparse layout
POOL_LAYOUTS = [(O.CONCAT, O.FIXED)] + [(p, s) for p in (O.SUM, O.MEAN, O.WSUM, O.WMEAN) for s in (O.FIXED, O.CSR)]


@pytest.mark.parametrize("pooling,sparse", POOL_LAYOUTS)
@pytest.mark.parametrize("key_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("gdt", [O.F32, O.F16])
def test_backprop_matches_oracle_bitwise(pooling, sparse, key_dtype, gdt):
    rng = np.random.default_rng(400 + 10 * pooling + sparse + (key_dtype == np.int32) * 3 + gdt)
    wdt = O.F16 if gdt == O.F16 else O.F32
    keys, offsets, n, w, g = make_case(rng, pooling, sparse, key_dtype, wdt, gdt)
    hot = 40
    counts = np.bincount(keys.astype(np.int64))
    assert counts.max() > 64  # several pieces for the hottest key
    uq, out = gpu_backprop(keys, pooling, sparse, offsets, hot, w, wdt, g, gdt, g.shape[1])
    bags = 0 if pooling == O.CONCAT else (offsets.size - 1 if offsets is not None else n // hot)
    ruq, rout = O.pooling_backprop(keys, pooling, sparse, offsets, bags, hot, w, wdt,
                                   g.view(np.uint16) if gdt == O.F16 else g, gdt, g.shape[1])
    assert np.array_equal(uq, ruq)
    bits = np.uint16 if gdt == O.F16 else np.uint32
    assert np.array_equal(out, rout.view(bits))


@pytest.mark.parametrize("case", ["high_common_bits", "bit_27_outlier", "negative_int32"])
def test_key_spans_beyond_the_assumed_sort_bits(case):
    """The dedup inside the backprop first sorts on the low 27 bits and reads
    the key span with the unique count; keys that differ higher up (an outlier
    with bit 27 set, negative int32 keys) are run again on their exact bits,
    keys that only share high bits are not.  Sum over Fixed bags, fp32."""
    rng = np.random.default_rng(127)
    bags, hot, dim = 96, 32, 64
    n = bags * hot
    keys = rng.zipf(1.2, size=n) % 3000
    if case == "high_common_bits":
        keys = (keys + 2**40).astype(np.int64)
    elif case == "bit_27_outlier":
        keys = keys.astype(np.int64)
        keys[n // 3] = 2**27 + 5
    else:
        keys = (keys - 1500).astype(np.int32)
    g = rng.normal(0, 1, size=(bags, dim)).astype(np.float32)
    uq, out = gpu_backprop(keys, O.SUM, O.FIXED, None, hot, None, O.F32, g, O.F32, dim)
    ruq, rout = O.pooling_backprop(keys, O.SUM, O.FIXED, None, bags, hot, None, O.F32, g, O.F32, dim)
    assert np.array_equal(uq, ruq)
    assert np.array_equal(out, rout.view(np.uint32))


def test_positions_outside_bags_and_empty_input():
    rng = np.random.default_rng(431)
    rows, dim, bags = 300, 32, 20
    lens = rng.integers(0, 10, size=bags)
    offsets = np.zeros(bags + 1, np.int64)
    offsets[1:] = np.cumsum(lens)
    n = int(offsets[-1]) + 17  # the last 17 keys belong to no bag
    keys = rng.integers(0, rows, size=n).astype(np.int64)
    g = rng.normal(size=(bags, dim)).astype(np.float32)
    uq, out = gpu_backprop(keys, O.SUM, O.CSR, offsets, 0, None, O.F32, g, O.F32, dim)
    ruq, rout = O.pooling_backprop(keys, O.SUM, O.CSR, offsets, bags, 0, None, O.F32, g, O.F32, dim)
    assert np.array_equal(uq, ruq) and np.array_equal(out, rout.view(np.uint32))
    empty = np.zeros(0, np.int64)
    uq, out = gpu_backprop(empty, O.SUM, O.FIXED, None, 4, None, O.F32, np.zeros((0, dim), np.float32),
                           O.F32, dim)
    assert uq.size == 0 and out.size == 0


def test_uniform_keys_one_run_each_large_batch():
    """262,144 keys over a large row range (mostly distinct keys): every run
    holds a handful of positions; gradient rows of 128 fp16 values."""
    rng = np.random.default_rng(433)
    rows, dim, bags, hot = 10_000_000, 128, 2048, 128
    keys = rng.integers(0, rows, size=bags * hot).astype(np.int64)
    g = rng.normal(0, 0.1, size=(bags, dim)).astype(np.float16)
    uq, out = gpu_backprop(keys, O.MEAN, O.FIXED, None, hot, None, O.F32, g, O.F16, dim)
    ruq, rout = O.pooling_backprop(keys, O.MEAN, O.FIXED, None, bags, hot, None, O.F32, g.view(np.uint16),
                                   O.F16, dim)
    assert np.array_equal(uq, ruq) and np.array_equal(out, rout)


@pytest.mark.parametrize("dim", [1, 3, 7, 8, 12, 100, 128, 200, 300, 520, 1030])
@pytest.mark.parametrize("gdt", [O.F32, O.F16])
def test_row_widths(dim, gdt):
    """Vector lanes (16-byte rows pieces) and scalar lanes, 8 to 64 lanes per
    block, and rows wider than one lane group's pass (column chunks)."""
    rng = np.random.default_rng(500 + dim + gdt)
    bags, hot, rows = 40, 30, 700
    keys = (rng.zipf(1.2, size=bags * hot) % rows).astype(np.int64)
    g = rng.normal(0, 1, size=(bags, dim)).astype(np.float16 if gdt == O.F16 else np.float32)
    w = rng.uniform(0.1, 1.0, size=bags * hot).astype(np.float32)
    for pooling in (O.SUM, O.WMEAN):
        ww = w if pooling == O.WMEAN else None
        uq, out = gpu_backprop(keys, pooling, O.FIXED, None, hot, ww, O.F32, g, gdt, dim)
        ruq, rout = O.pooling_backprop(keys, pooling, O.FIXED, None, bags, hot, ww, O.F32,
                                       g.view(np.uint16) if gdt == O.F16 else g, gdt, dim)
        bits = np.uint16 if gdt == O.F16 else np.uint32
        assert np.array_equal(uq, ruq) and np.array_equal(out, rout.view(bits))


@pytest.mark.parametrize("n", [1, 31, 32, 33, 63, 64, 65, 127, 128, 4097])
def test_block_edges(n):
    """Batches ending inside, at and just past a block; one key over all of
    them, and keys that start exactly on a block edge."""
    rng = np.random.default_rng(600 + n)
    dim = 16
    keys = np.sort(rng.integers(0, max(n // 20, 1), size=n)).astype(np.int64)
    keys[: min(n, 32)] = 0  # key 0 fills the first block exactly when n >= 32
    g = rng.normal(0, 1, size=(n, dim)).astype(np.float32)
    for ks in (keys, np.zeros(n, np.int64), rng.permutation(keys)):
        uq, out = gpu_backprop(ks, O.CONCAT, O.FIXED, None, 1, None, O.F32, g, O.F32, dim)
        ruq, rout = O.pooling_backprop(ks, O.CONCAT, O.FIXED, None, 0, 1, None, O.F32, g, O.F32, dim)
        assert np.array_equal(uq, ruq) and np.array_equal(out, rout.view(np.uint32))


def test_hot_keys_hundreds_of_blocks():
    """The c2bwd shape in miniature: 131,072 keys, the hottest over 7000
    positions (more than 200 pieces, all eight sub-sequences long)."""
    rng = np.random.default_rng(611)
    bags, hot, dim = 512, 256, 128
    x = rng.random(bags * hot)
    keys = (np.floor(x ** 6 * 5_000_000)).astype(np.int64)
    assert np.bincount(keys).max() > 7000
    g = rng.normal(0, 0.1, size=(bags, dim)).astype(np.float16)
    uq, out = gpu_backprop(keys, O.SUM, O.FIXED, None, hot, None, O.F32, g, O.F16, dim)
    ruq, rout = O.pooling_backprop(keys, O.SUM, O.FIXED, None, bags, hot, None, O.F32, g.view(np.uint16),
                                   O.F16, dim)
    assert np.array_equal(uq, ruq) and np.array_equal(out, rout)


def test_unaligned_gradient_buffers_take_scalar_lanes():
    rng = np.random.default_rng(613)
    bags, hot, dim = 30, 20, 64
    keys = (rng.zipf(1.3, size=bags * hot) % 200).astype(np.int64)
    g = rng.normal(0, 1, size=(bags, dim)).astype(np.float32)
    n = keys.size
    wsb = ctypes.c_uint64()
    _lib.call("nve_amd_backprop_workspace_size", n, bags, dim, ctypes.byref(wsb))
    ws = torch.empty(int(wsb.value), dtype=torch.uint8, device="cuda")
    d_keys = to_dev(keys)
    d_g = torch.empty(g.nbytes + 4, dtype=torch.uint8, device="cuda")
    d_g[4:].copy_(torch.from_numpy(g.reshape(-1).view(np.uint8)))  # 4-byte aligned, not 16
    uq = torch.zeros(n, dtype=torch.int64, device="cuda")
    out = torch.zeros(n * dim * 4 + 4, dtype=torch.uint8, device="cuda")
    nu = ctypes.c_int64(-1)
    _lib.call("nve_amd_pooling_backprop", _lib.KEY_INT64, n, vp(d_keys), _lib.POOL_SUM, _lib.SPARSE_FIXED,
              None, 0, hot, None, _lib.DT_UNKNOWN, ctypes.c_void_p(d_g.data_ptr() + 4), _lib.DT_F32, dim,
              vp(uq), ctypes.c_void_p(out.data_ptr() + 4), ctypes.byref(nu), vp(ws), wsb.value,
              stream_ptr())
    torch.cuda.synchronize()
    u = nu.value
    got = out[4:4 + u * dim * 4].cpu().numpy().view(np.uint32).reshape(u, dim)
    ruq, rout = O.pooling_backprop(keys, O.SUM, O.FIXED, None, bags, hot, None, O.F32, g, O.F32, dim)
    assert np.array_equal(uq.cpu().numpy()[:u], ruq) and np.array_equal(got, rout.view(np.uint32))

"""GPU parity of the training backprop (nve_amd_pooling_backprop, restating
GradientCalculator::compute_gradients, cuda_ops/gradient_calculator.cuh:238-301)
against the oracle (orc_pooling_backprop, itself pinned to torch autograd).

Both sum each unique key's positions in runs of 64 (fp32, position order) and
then the runs, rounding once, so unique keys and gradient rows must match bit
for bit.  Cases follow tests/kernels/pooling_backprop_tests.cu: Concatenate /
Sum / Mean / WeightedSum / WeightedMean, Fixed and CSR bags, int32 and int64
keys, plus fp16 gradients, Zipf keys whose hottest key spans many runs, empty
bags and positions outside every bag."""
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


@pytest.mark.parametrize("pooling", [O.CONCAT, O.SUM, O.MEAN, O.WSUM, O.WMEAN])
@pytest.mark.parametrize("sparse", [O.FIXED, O.CSR])
@pytest.mark.parametrize("key_dtype", [np.int32, np.int64])
@pytest.mark.parametrize("gdt", [O.F32, O.F16])
def test_backprop_matches_oracle_bitwise(pooling, sparse, key_dtype, gdt):
    if pooling == O.CONCAT and sparse == O.CSR:
        pytest.skip("Concatenate has no bags")
    rng = np.random.default_rng(400 + 10 * pooling + sparse + (key_dtype == np.int32) * 3 + gdt)
    wdt = O.F16 if gdt == O.F16 else O.F32
    keys, offsets, n, w, g = make_case(rng, pooling, sparse, key_dtype, wdt, gdt)
    hot = 40
    counts = np.bincount(keys.astype(np.int64))
    assert counts.max() > 64  # several runs for the hottest key
    uq, out = gpu_backprop(keys, pooling, sparse, offsets, hot, w, wdt, g, gdt, g.shape[1])
    bags = 0 if pooling == O.CONCAT else (offsets.size - 1 if offsets is not None else n // hot)
    ruq, rout = O.pooling_backprop(keys, pooling, sparse, offsets, bags, hot, w, wdt,
                                   g.view(np.uint16) if gdt == O.F16 else g, gdt, g.shape[1])
    assert np.array_equal(uq, ruq)
    bits = np.uint16 if gdt == O.F16 else np.uint32
    assert np.array_equal(out, rout.view(bits))


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

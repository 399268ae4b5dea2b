"""BASELINE configurations C1 and C2 at their real sizes, through the C ABI.

C1 (the reference HostLayer configuration, here on the GPU layer): a
1,000,000 x 64 fp32 table, 4,096 bags of exactly 8 keys drawn uniformly from
[0, 1e6); the plain gather (32,768 x 64) must equal the oracle's bit for bit,
and the Fixed-8 Sum (4,096 x 64) too: 8-key bags are reduced by one lane group
in key order, the oracle's order (tests/embedding_layer/gpu_layer_test.cpp:
163-210,353 hold the same shapes to the MockHostTable combine).

C2 / C2-pool at full size: a 50,000,000 x 128 fp16 table (12.8 GB, so row
offsets pass 2^32 bytes from row 16,777,216 on) and 262,144 keys drawn
Zipf(1.05) with the reference generator (samples/pytorch/
pytorch_samples_common.py:21-47).  The pooled lookup of the benchmark is
checked on sampled bags against the oracle over the rows those bags touch
(split bags: within 1 fp16 ulp or 1e-5 of the row's magnitude); the dedup
and both gathers are checked over the whole batch.
"""
import ctypes
import sys

import numpy as np
import pytest

from nve_helpers import pooled_f16_close, stream_ptr, vp
from oracle import oracle as O
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _bench():
    import bench  # the key generator of the benchmark (repo root)
    return bench


def gpu_layer(d_table, rows, width, dtype):
    L = _lib.load()
    lc = L.nve_gpu_embedding_layer_config_default()
    lc.layer_name = b"configs"
    lc.embedding_table = d_table.data_ptr()
    lc.num_embeddings = rows
    lc.embedding_width_in_bytes = width
    lc.value_dtype = dtype
    layer, ctx = ctypes.c_void_p(), ctypes.c_void_p()
    _lib.call("nve_gpu_embedding_layer_create", ctypes.byref(layer), _lib.KEY_INT64, ctypes.byref(lc), None)
    s = stream_ptr()
    _lib.call("nve_layer_create_execution_context", layer, ctypes.byref(ctx), s, s, None, None)
    return layer, ctx


def destroy(layer, ctx):
    _lib.call("nve_context_wait", ctx)
    _lib.call("nve_context_destroy", ctx)
    _lib.call("nve_layer_destroy", layer)


@pytest.mark.parametrize("values", ["dyadic", "normal"])
def test_c1_gather_and_fixed8_sum(values):
    rows, dim, bags, hot = 1_000_000, 64, 4096, 8
    rng = np.random.default_rng(0)
    if values == "dyadic":  # sums exact in any order
        table = (rng.integers(-8, 9, size=(rows, dim)) / np.exp2(rng.integers(3, 10, size=(rows, dim))))
        table = table.astype(np.float32)
    else:  # BASELINE's N(0, 0.01)
        table = rng.normal(0.0, 0.01, size=(rows, dim)).astype(np.float32)
    keys = np.random.default_rng(1).integers(0, rows, size=bags * hot).astype(np.int64)
    print(f"[c1] {values} table {rows}x{dim} f32, {keys.size} keys", flush=True)
    d_table = torch.from_numpy(table).cuda()
    d_keys = torch.from_numpy(keys).cuda()
    layer, ctx = gpu_layer(d_table, rows, dim * 4, _lib.DT_F32)
    try:
        L = _lib.load()
        gathered = torch.full((keys.size, dim), -1.0, dtype=torch.float32, device="cuda")
        _lib.check(L.nve_layer_lookup(layer, ctx, keys.size, vp(d_keys), vp(gathered), dim * 4, None, None))
        pooled = torch.full((bags, dim), -1.0, dtype=torch.float32, device="cuda")
        _lib.check(L.nve_layer_lookup_pooled(layer, ctx, keys.size, vp(d_keys), vp(pooled), dim * 4, None,
                                             _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, hot, None,
                                             _lib.DT_UNKNOWN, _lib.DT_F32, None))
        torch.cuda.synchronize()
    finally:
        destroy(layer, ctx)
    tb = table.view(np.uint8).reshape(-1)
    ref_rows, hits = O.gather(keys, tb, dim * 4, rows)
    assert hits == keys.size
    assert np.array_equal(gathered.cpu().numpy().view(np.uint8), ref_rows)
    ref = O.pool(O.linear_row_ptrs(keys, tb, dim * 4), O.F32, dim, O.FIXED, O.SUM, keys.size, None, bags,
                 hot, None, 0, O.F32)
    assert np.array_equal(pooled.cpu().numpy().view(np.uint32), ref.view(np.uint32))


@pytest.fixture(scope="module")
def c2_table():
    """The benchmark's C2 table and key batch, built on the GPU as bench.py builds them."""
    bench = _bench()
    rows, dim, nkeys = 50_000_000, 128, 262144
    print(f"[c2] building {rows}x{dim} f16 table (12.8 GB) and Zipf(1.05) keys", flush=True)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    table = torch.empty((rows, dim), dtype=torch.float16, device="cuda")
    for r0 in range(0, rows, 1 << 24):
        table[r0:min(rows, r0 + (1 << 24))].normal_(0.0, 0.02, generator=gen)
    pg = torch.Generator(device="cuda")
    pg.manual_seed(31337)
    perm = torch.randperm(rows, generator=pg, device="cuda", dtype=torch.int64)
    kg = torch.Generator(device="cuda")
    kg.manual_seed(1)
    keys = bench.power_law_keys(torch, nkeys, rows, 1.05, kg, perm)
    del perm
    # bag 0 holds the table's last 1024 rows: the highest row addresses
    keys[:1024] = torch.arange(rows - 1024, rows, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()
    yield table, keys, rows, dim
    del table
    torch.cuda.empty_cache()


def test_c2pool_full_size_every_bag(c2_table):
    table, keys, rows, dim = c2_table
    bags, hot = 256, 1024
    width = dim * 2
    k = keys.cpu().numpy()
    assert (k >= (1 << 32) // width).mean() > 0.5  # most rows lie past 4 GiB
    layer, ctx = gpu_layer(table, rows, width, _lib.DT_F16)
    out = torch.full((bags, dim), float("nan"), dtype=torch.float16, device="cuda")
    try:
        L = _lib.load()
        _lib.check(L.nve_layer_lookup_pooled(layer, ctx, keys.numel(), vp(keys), vp(out), width, None,
                                             _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, hot, None,
                                             _lib.DT_UNKNOWN, _lib.DT_F16, None))
        torch.cuda.synchronize()
    finally:
        destroy(layer, ctx)
    got = out.cpu().numpy().view(np.uint16)
    # every bag: the batch's rows by torch's own gather (row i = table[key i],
    # 67 MB), pooled by the oracle in key order
    rows_all = np.ascontiguousarray(table[keys].cpu().numpy().view(np.uint16)).view(np.uint8).reshape(-1)
    ref = O.pool(O.linear_row_ptrs(np.arange(keys.numel()), rows_all, width), O.F16, dim, O.FIXED, O.SUM,
                 keys.numel(), None, bags, hot, None, 0, O.F16)
    bad = [b for b in range(bags) if not pooled_f16_close(got[b:b + 1], ref[b:b + 1])]
    assert bad == [], f"bags off the oracle: {bad[:16]}"


def test_c2_full_size_dedup_and_gathers(c2_table):
    table, keys, rows, dim = c2_table
    n, width = keys.numel(), dim * 2
    s = stream_ptr()
    want = table[keys]  # torch's gather of the same rows
    # plain gather through the GPU layer
    layer, ctx = gpu_layer(table, rows, width, _lib.DT_F16)
    got = torch.empty((n, dim), dtype=torch.float16, device="cuda")
    try:
        _lib.check(_lib.load().nve_layer_lookup(layer, ctx, n, vp(keys), vp(got), width, None, None))
        torch.cuda.synchronize()
    finally:
        destroy(layer, ctx)
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # dedup then gather
    wsb = ctypes.c_uint64()
    _lib.call("nve_amd_dedup_workspace_size", n, ctypes.byref(wsb))
    ws = torch.empty(int(wsb.value), dtype=torch.uint8, device="cuda")
    got2 = torch.empty((n, dim), dtype=torch.float16, device="cuda")
    _lib.call("nve_amd_dedup_gather", _lib.KEY_INT64, n, vp(keys), vp(table), rows, width, vp(got2), width,
              vp(ws), wsb.value, s)
    torch.cuda.synchronize()
    assert torch.equal(got2.view(torch.int16), want.view(torch.int16))
    # the dedup itself against the oracle
    outs = [torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(4)]
    nu = ctypes.c_int64()
    _lib.call("nve_amd_dedup", _lib.KEY_INT64, n, vp(keys), *[vp(o) for o in outs], ctypes.byref(nu), vp(ws),
              wsb.value, s)
    torch.cuda.synchronize()
    u = nu.value
    ru, rc, rinv, roff = O.dedup(keys.cpu().numpy())
    assert u == ru.size and 0.3 < u / n < 0.45  # Zipf(1.05): about 38 % unique
    uq, ct, inv, off = [o.cpu().numpy() for o in outs]
    assert np.array_equal(uq[:u], ru) and np.array_equal(ct[:u], rc)
    assert np.array_equal(inv, rinv) and np.array_equal(off[:u], roff)

"""The CPU HostLayer on the GPU box's own host cores.

The bench's `cpu_baseline` times the product HostLayer (host_kernels.cpp,
whose row loops pick 8-wide AVX2/F16C code at run time) on the GPU box, whose
CPU can take a different loop than this build container's.  These tests are
marked `gpu` so that the GPU-box run executes them there: the C1 workload
(1,000,000 x 64 rows, 4,096 bags of 8 uniform keys) in fp32 and fp16 rows,
Sum and Mean, and the bench's long-bag fp16 shape (1,024-key bags, fp16
output), each bit for bit against the oracle's restatement of the reference
HostLayer (host_embedding_layer.cpp:55-247, cpu_gather.hpp:28-80,
cpu_pooling.hpp:68-150).  No GPU call is made."""
import numpy as np
import pytest

from oracle import oracle as O
from pynve import _lib
from test_host_layer_cpu import HostLayer

pytestmark = pytest.mark.gpu


def simd_path():
    try:
        flags = set(next(l for l in open("/proc/cpuinfo") if l.startswith("flags")).split(":")[1].split())
    except (OSError, StopIteration):
        return "unknown"
    return "avx2+f16c+fma" if {"avx2", "f16c", "fma"} <= flags else "scalar"


@pytest.fixture
def layers():
    made = []
    yield made
    for h in made:
        h.close()


@pytest.mark.parametrize("pooling", [_lib.POOL_SUM, _lib.POOL_MEAN])
@pytest.mark.parametrize("dtype", [O.F32, O.F16])
def test_c1_shape_on_this_host(layers, dtype, pooling):
    rows, dim, bags, hot = 1_000_000, 64, 4096, 8
    print(f"[host layer] C1 shape dtype={dtype} pooling={pooling} simd={simd_path()}", flush=True)
    rng = np.random.default_rng(0)
    npdt = np.float32 if dtype == O.F32 else np.float16
    table = rng.normal(0.0, 0.01, size=(rows, dim)).astype(npdt)
    keys = np.random.default_rng(1).integers(0, rows, size=bags * hot).astype(np.int64)
    width = dim * table.itemsize
    h = HostLayer(table.view(np.uint8), dtype)
    layers.append(h)
    gathered = np.full((keys.size, dim), -1, npdt)
    assert h.lookup(keys, gathered) == 1.0
    assert np.array_equal(gathered.view(np.uint8), table[keys].view(np.uint8))
    pooled = np.full((bags, dim), -1, np.float32)
    h.pooled(keys, pooled, pooling, _lib.SPARSE_FIXED, hot=hot)
    tb = table.view(np.uint8).reshape(-1)
    opool = O.SUM if pooling == _lib.POOL_SUM else O.MEAN
    ref = O.pool(O.linear_row_ptrs(keys, tb, width), dtype, dim, O.FIXED, opool, keys.size, None, bags, hot,
                 None, 0, O.F32, host_order=True)
    assert np.array_equal(pooled.view(np.uint32), ref.view(np.uint32))


def test_bench_long_bag_shape_on_this_host(layers):
    """The bench's CPU baseline shape: fp16 rows of 128, bags of 1,024 Zipf keys,
    Sum to fp16 (here 2,000,000 rows and 64 bags)."""
    rows, dim, bags, hot = 2_000_000, 128, 64, 1024
    print(f"[host layer] long bags simd={simd_path()}", flush=True)
    rng = np.random.default_rng(3)
    table = rng.normal(0.0, 0.02, size=(rows, dim)).astype(np.float16)
    # the reference generator's Zipf(1.05) ranks 1..rows, permuted
    ranks = O.power_law(rng.random(bags * hot), 1, rows, 1.05)
    keys = np.ascontiguousarray(rng.permutation(rows)[ranks - 1], np.int64)
    h = HostLayer(table.view(np.uint8), O.F16)
    layers.append(h)
    out = np.full((bags, dim), np.nan, np.float16)
    h.pooled(keys, out, _lib.POOL_SUM, _lib.SPARSE_FIXED, hot=hot, odt=_lib.DT_F16)
    tb = table.view(np.uint8).reshape(-1)
    ref = O.pool(O.linear_row_ptrs(keys, tb, dim * 2), O.F16, dim, O.FIXED, O.SUM, keys.size, None, bags, hot,
                 None, 0, O.F16, host_order=True)
    assert np.array_equal(out.view(np.uint16), ref)

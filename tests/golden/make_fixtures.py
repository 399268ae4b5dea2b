"""Writes tests/golden/fixtures.npz: small input/output vectors of the lookup
path (pooled find-and-pool over a linear table, key dedup, pooling backprop),
computed by the CPU oracle in oracle/.

The reference commits no vector files: its tests generate data from seeded
generators and compare with CPU references at run time
(tests/kernels/kernel_test_common.cuh AllocateTable, tests/kernels/*_test.cu,
tests/dedup_test.cu).  These fixtures are this build's own, and every value
they hold is fixed by arithmetic a reader can redo: tables and gradients are
dyadic fractions nom / 2^e (nom in [-8, 8], e in [3, 9], the reference's
kernel-test fixture), so every sum and weighted sum below is exact in fp32 in
any order, and dedup's outputs are what a stable sort defines.
tests/test_golden_cpu.py recomputes them with numpy and checks the oracle
against them; tests/test_gpu_golden.py checks the HIP library against them.

Run from the repository root:  python tests/golden/make_fixtures.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
sys.path.insert(0, os.path.dirname(HERE))

from nve_helpers import dyadic, float_table, oracle_pool  # noqa: E402
from oracle import oracle as O  # noqa: E402

POOL_SUM, POOL_MEAN, POOL_WSUM = 1, 2, 3  # nve_pooling_type_t values

# (name, value dtype, out dtype, sparse, pooling, key dtype, rows, dim, bags, hotness or max bag length)
POOL_CASES = [
    ("pool_f16_fixed_sum", O.F16, O.F16, O.FIXED, POOL_SUM, np.int64, 64, 32, 10, 6),
    ("pool_f32_csr_mean_i32", O.F32, O.F32, O.CSR, POOL_MEAN, np.int32, 80, 16, 12, 9),
    ("pool_f32_fixed_wsum", O.F32, O.F32, O.FIXED, POOL_WSUM, np.int64, 50, 64, 8, 4),
    ("pool_f16_csr_sum", O.F16, O.F16, O.CSR, POOL_SUM, np.int64, 40, 128, 9, 30),
]


def pool_case(rng, name, vdt, odt, sparse, pooling, kdt, rows, dim, bags, hot):
    tb = float_table(rng, rows, dim, vdt)
    off = None
    if sparse == O.CSR:
        lens = rng.integers(0, hot + 1, size=bags)
        lens[1] = 0  # an empty bag
        off = np.zeros(bags + 1, kdt)
        off[1:] = np.cumsum(lens)
        n = int(off[-1])
        hot_arg = 0
    else:
        n = bags * hot
        hot_arg = hot
    keys = rng.integers(0, rows, size=n).astype(kdt)
    keys[: min(n, 3)] = keys[0]  # a repeated key
    w = dyadic(rng, n).astype(np.float32) if pooling == POOL_WSUM else None
    out = oracle_pool(tb, keys, vdt, dim, sparse, pooling, off, bags, hot_arg, w, O.F32, odt)
    bits = np.uint16 if odt == O.F16 else np.uint32
    d = {
        "params": np.array([vdt, odt, sparse, pooling, rows, dim, bags, hot_arg], np.int64),
        "table": tb,
        "keys": keys,
        "out_bits": out.view(bits).reshape(bags, dim),
    }
    if off is not None:
        d["offsets"] = off
    if w is not None:
        d["weights"] = w
    return {f"{name}/{k}": v for k, v in d.items()}


def dedup_case(name, keys):
    uq, ct, inv, off = O.dedup(keys)
    return {f"{name}/keys": keys, f"{name}/unique": uq.astype(keys.dtype), f"{name}/counts": ct,
            f"{name}/inverse": inv, f"{name}/offsets": off}


def backprop_case(rng, name, sparse, kdt, gdt, bags, hot, rows, dim):
    if sparse == O.CSR:
        lens = rng.integers(0, hot + 1, size=bags)
        lens[0] = 0
        off = np.zeros(bags + 1, kdt)
        off[1:] = np.cumsum(lens)
        n = int(off[-1])
        hot_arg = 0
    else:
        off, n, hot_arg = None, bags * hot, hot
    keys = rng.integers(0, rows, size=n).astype(kdt)
    g = dyadic(rng, (bags, dim))
    g_bits = g.astype(np.float16).view(np.uint16) if gdt == O.F16 else g.astype(np.float32).view(np.uint32)
    uq, grad = O.pooling_backprop(keys, POOL_SUM, sparse, off, bags, hot_arg, None, O.F32, g_bits, gdt, dim)
    d = {"params": np.array([sparse, gdt, bags, hot_arg, dim], np.int64), "keys": keys,
         "grads_in_bits": g_bits, "unique": uq,
         "grad_bits": grad.view(np.uint16 if gdt == O.F16 else np.uint32)}
    if off is not None:
        d["offsets"] = off
    return {f"{name}/{k}": v for k, v in d.items()}


def main():
    rng = np.random.default_rng(0x600D)
    arrays = {}
    for case in POOL_CASES:
        arrays.update(pool_case(rng, *case))
    k64 = rng.integers(-40, 40, size=300).astype(np.int64)
    k64[:4] = [np.iinfo(np.int64).min, np.iinfo(np.int64).max, -1, 0]
    arrays.update(dedup_case("dedup_i64", k64))
    k32 = (rng.zipf(1.3, size=257) % 1000).astype(np.int32) - 500
    arrays.update(dedup_case("dedup_i32", k32))
    arrays.update(backprop_case(rng, "bwd_f32_fixed", O.FIXED, np.int64, O.F32, 20, 6, 40, 16))
    arrays.update(backprop_case(rng, "bwd_f16_csr_i32", O.CSR, np.int32, O.F16, 15, 12, 30, 64))
    path = os.path.join(HERE, "fixtures.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path}: {len(arrays)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()

"""The committed golden fixtures (tests/golden/fixtures.npz, written by
tests/golden/make_fixtures.py) recomputed two ways on the CPU:

* independently with numpy in float64 (dyadic tables, weights and gradients:
  sums are exact, so a dropped term, a wrong bag cut or a transposed index
  changes the bits), and with numpy's unique / stable argsort for dedup;
* by the oracle (a regression pin: the oracle keeps producing these bits).

Pooled lookup: find_and_pool, cuda_ops/find_and_pool.cuh:103-132 over a linear
table; dedup: Deduper::dedup, cuda_ops/deduper.cuh:136-221; backprop:
GradientCalculator::compute_gradients, cuda_ops/gradient_calculator.cuh:238-301."""
import os

import numpy as np
import pytest

from nve_helpers import oracle_pool
from oracle import oracle as O

FIXTURES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")
Z = np.load(FIXTURES)  # written by this repository; allow_pickle stays False


def cases(prefix):
    return sorted({k.split("/")[0] for k in Z.files if k.startswith(prefix)})


def get(name, key):
    k = f"{name}/{key}"
    return Z[k] if k in Z.files else None


def decode_rows(table, vdt, dim):
    if vdt == O.F16:
        return table.view(np.float16).reshape(-1, dim).astype(np.float64)
    return table.view(np.float32).reshape(-1, dim).astype(np.float64)


def bag_bounds(off, hot, bags):
    if off is not None:
        return [(int(off[b]), int(off[b + 1])) for b in range(bags)]
    return [(b * hot, (b + 1) * hot) for b in range(bags)]


@pytest.mark.parametrize("name", cases("pool_"))
def test_pool_fixture_numpy_and_oracle(name):
    vdt, odt, sparse, pooling, rows, dim, bags, hot = (int(x) for x in get(name, "params"))
    table, keys, off, w = get(name, "table"), get(name, "keys"), get(name, "offsets"), get(name, "weights")
    want = get(name, "out_bits")
    vals = decode_rows(table, vdt, dim)
    ref = np.zeros((bags, dim))
    for b, (s, e) in enumerate(bag_bounds(off, hot, bags)):
        rows_b = vals[keys[s:e].astype(np.int64)]
        if pooling == O.WSUM:
            rows_b = rows_b * w[s:e, None].astype(np.float64)
        ref[b] = rows_b.sum(axis=0)
        if pooling == O.MEAN and e > s:
            ref[b] /= e - s
    if odt == O.F16:
        np_bits = ref.astype(np.float16).view(np.uint16)
    else:
        np_bits = ref.astype(np.float32).view(np.uint32)
    if pooling == O.MEAN:
        # a quotient: within one fp32 ulp of the float64 one
        got = want.view(np.float32).astype(np.float64)
        assert np.all(np.abs(got - ref) <= np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64))
    else:
        assert np.array_equal(want, np_bits)
    again = oracle_pool(table, keys, vdt, dim, sparse, pooling, off, bags, hot, w, O.F32, odt)
    assert np.array_equal(again.view(want.dtype).reshape(want.shape), want)
    if off is not None:
        assert np.all(want[np.diff(off) == 0] == 0)


@pytest.mark.parametrize("name", cases("dedup_"))
def test_dedup_fixture_numpy_and_oracle(name):
    keys = get(name, "keys")
    uq, ct = np.unique(keys, return_counts=True)
    assert np.array_equal(get(name, "unique"), uq)
    assert np.array_equal(get(name, "counts"), ct)
    assert np.array_equal(get(name, "inverse"), np.argsort(keys, kind="stable"))
    assert np.array_equal(get(name, "offsets"), np.concatenate([[0], np.cumsum(ct)[:-1]]))
    again = O.dedup(keys)
    for got, key in zip(again, ("unique", "counts", "inverse", "offsets")):
        assert np.array_equal(got, get(name, key)), key


@pytest.mark.parametrize("name", cases("bwd_"))
def test_backprop_fixture_numpy_and_oracle(name):
    sparse, gdt, bags, hot, dim = (int(x) for x in get(name, "params"))
    keys, off, g_bits = get(name, "keys"), get(name, "offsets"), get(name, "grads_in_bits")
    g = (g_bits.view(np.float16) if gdt == O.F16 else g_bits.view(np.float32)).astype(np.float64)
    g = g.reshape(bags, dim)
    acc = {}
    for b, (s, e) in enumerate(bag_bounds(off, hot, bags)):
        for k in keys[s:e]:
            acc[int(k)] = acc.get(int(k), 0.0) + g[b]
    uq = np.array(sorted(acc), keys.dtype)
    rows = np.array([acc[int(k)] for k in uq]).reshape(len(uq), dim)
    bits = rows.astype(np.float16).view(np.uint16) if gdt == O.F16 else rows.astype(np.float32).view(np.uint32)
    assert np.array_equal(get(name, "unique"), uq)
    assert np.array_equal(get(name, "grad_bits"), bits)
    again_u, again_g = O.pooling_backprop(keys, O.SUM, sparse, off, bags, hot, None, O.F32, g_bits, gdt, dim)
    assert np.array_equal(again_u, uq)
    assert np.array_equal(again_g.view(bits.dtype), bits)

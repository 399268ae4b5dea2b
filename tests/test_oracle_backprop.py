"""Pins for the oracle's training backprop (orc_pooling_backprop), the
restatement of GradientCalculator::compute_gradients
(cuda_ops/gradient_calculator.cuh:238-301) and GradientDedup
(cuda_ops/dedup_grads_kernel.cuh:57-107).

The gradient of a lookup is fixed by calculus: the checks compare against
torch autograd through torch.nn.functional.embedding_bag / embedding in
float64 (Sum, Mean, WSum via per_sample_weights, WMean via weights
pre-divided by their bag's sum in float64, Concatenate), with exact equality
for dyadic Sum / Concatenate inputs (the reference test's own fixture idea,
tests/kernels/pooling_backprop_tests.cu: gradients nom / 2^k), and check that
the run length only regroups the additions."""
import numpy as np
import pytest

from oracle import oracle as O

torch = pytest.importorskip("torch")

SUM, MEAN, WSUM, WMEAN, CONCAT = O.SUM, O.MEAN, O.WSUM, O.WMEAN, O.CONCAT


def dense_grad_torch(keys, pooling, sparse, offsets, bags, hotness, weights, grads_in, rows):
    """d(sum(out * grads_in)) / d(table) in float64 with torch autograd."""
    dim = grads_in.shape[1]
    table = torch.zeros((rows, dim), dtype=torch.float64, requires_grad=True)
    k = torch.from_numpy(keys.astype(np.int64))
    if pooling == CONCAT:
        out = torch.nn.functional.embedding(k, table)
    else:
        if sparse == O.FIXED:
            off = torch.arange(0, bags * hotness + 1, hotness, dtype=torch.int64)
        else:
            off = torch.from_numpy(offsets.astype(np.int64))
        psw = None
        mode = "mean" if pooling == MEAN else "sum"
        if pooling in (WSUM, WMEAN):
            w = weights.astype(np.float64)
            if pooling == WMEAN:
                o = off.numpy()
                w = w.copy()
                for b in range(bags):
                    s, e = o[b], o[b + 1]
                    if e > s:
                        w[s:e] /= w[s:e].sum()
            psw = torch.from_numpy(w)
        out = torch.nn.functional.embedding_bag(k, table, off[:-1], mode=mode, per_sample_weights=psw,
                                                include_last_offset=False)
    (out * torch.from_numpy(grads_in.astype(np.float64))).sum().backward()
    return table.grad.numpy()


def sparse_to_dense(uq, g, rows, grad_dtype):
    dense = np.zeros((rows, g.shape[1]), np.float64)
    vals = g.view(np.float16).astype(np.float64) if grad_dtype == O.F16 else g.astype(np.float64)
    dense[uq.astype(np.int64)] = vals
    return dense


def dyadic(rng, shape):
    return (rng.integers(-8, 9, size=shape) / (1 << rng.integers(3, 10, size=shape))).astype(np.float32)


@pytest.mark.parametrize("pooling", [SUM, MEAN, WSUM, WMEAN])
@pytest.mark.parametrize("sparse", [O.FIXED, O.CSR])
@pytest.mark.parametrize("key_dtype", [np.int32, np.int64])
def test_pooled_gradient_matches_torch_autograd(pooling, sparse, key_dtype):
    rng = np.random.default_rng(5 + pooling + 10 * sparse)
    rows, dim, bags, hot = 300, 24, 40, 9
    if sparse == O.FIXED:
        offsets = None
        n = bags * hot
    else:
        lens = rng.integers(0, 30, size=bags)
        lens[3] = 0
        offsets = np.zeros(bags + 1, key_dtype)
        offsets[1:] = np.cumsum(lens)
        n = int(offsets[-1])
    keys = (rng.zipf(1.3, size=n) % rows).astype(key_dtype)
    w = rng.uniform(0.1, 1.0, size=n).astype(np.float32) if pooling in (WSUM, WMEAN) else None
    g = rng.normal(0, 1, size=(bags, dim)).astype(np.float32)
    uq, out = O.pooling_backprop(keys, pooling, sparse, offsets, bags, hot, w, O.F32, g, O.F32, dim)
    assert np.all(np.diff(uq.astype(np.int64)) > 0)  # unique, ascending
    assert set(uq.tolist()) == set(keys.tolist())
    ref = dense_grad_torch(keys, pooling, sparse, offsets, bags, hot, w, g, rows)
    got = sparse_to_dense(uq, out, rows, O.F32)
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("pooling", [SUM, CONCAT])
def test_dyadic_sums_are_exact(pooling):
    """Dyadic gradients (nom / 2^k) add exactly in fp32: no tolerance."""
    rng = np.random.default_rng(17)
    rows, dim, bags, hot = 200, 16, 60, 12
    keys = (rng.zipf(1.2, size=bags * hot) % rows).astype(np.int64)
    g = dyadic(rng, (bags * hot if pooling == CONCAT else bags, dim))
    uq, out = O.pooling_backprop(keys, pooling, O.FIXED, None, bags, hot, None, O.F32, g, O.F32, dim,
                                 block=5)
    ref = dense_grad_torch(keys, pooling, O.FIXED, None, bags, hot, None, g, rows)
    assert np.array_equal(sparse_to_dense(uq, out, rows, O.F32), ref)


def test_run_length_only_regroups():
    """The block size changes the grouping of the additions, not the sum: exact for
    dyadic values, within fp32 rounding otherwise; fp16 rows round once."""
    rng = np.random.default_rng(23)
    rows, dim, bags, hot = 50, 8, 100, 10
    keys = (rng.zipf(1.5, size=bags * hot) % rows).astype(np.int64)
    g = dyadic(rng, (bags, dim))
    a = O.pooling_backprop(keys, SUM, O.FIXED, None, bags, hot, None, O.F32, g, O.F32, dim, block=1)
    b = O.pooling_backprop(keys, SUM, O.FIXED, None, bags, hot, None, O.F32, g, O.F32, dim, block=1 << 20)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    g16 = rng.normal(0, 0.05, size=(bags, dim)).astype(np.float16)
    uq, out = O.pooling_backprop(keys, MEAN, O.FIXED, None, bags, hot, None, O.F16, g16.view(np.uint16),
                                 O.F16, dim)
    ref = dense_grad_torch(keys, MEAN, O.FIXED, None, bags, hot, None, g16.astype(np.float32), rows)
    got = sparse_to_dense(uq, out, rows, O.F16)
    # one fp16 rounding of an fp32-accumulated sum
    assert np.allclose(got, ref, rtol=2 ** -10, atol=2 ** -20)


def test_positions_outside_every_bag_add_nothing():
    rng = np.random.default_rng(29)
    rows, dim, bags = 40, 4, 5
    offsets = np.array([0, 3, 3, 7, 9, 12], np.int64)  # keys 12.. belong to no bag
    keys = rng.integers(0, rows, size=16).astype(np.int64)
    g = rng.normal(size=(bags, dim)).astype(np.float32)
    uq, out = O.pooling_backprop(keys, SUM, O.CSR, offsets, bags, 0, None, O.F32, g, O.F32, dim)
    ref = dense_grad_torch(keys[:12], SUM, O.CSR, offsets, bags, 0, None, g, rows)
    got = sparse_to_dense(uq, out, rows, O.F32)
    assert set(uq.tolist()) == set(keys.tolist())  # every key is reported, some with a zero row
    assert np.allclose(got, ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("block", [1, 3, 8, 32, 64])
def test_hot_keys_over_many_blocks(block):
    """Keys whose positions span many blocks (up to hundreds of pieces, so all
    eight sub-sequences are used and the last ones are short or empty) sum to the
    autograd gradient: exactly for dyadic values, within fp32 rounding
    otherwise."""
    rng = np.random.default_rng(31 + block)
    rows, dim, bags, hot = 40, 8, 120, 16
    keys = np.where(rng.random(bags * hot) < 0.6, 0, rng.integers(0, rows, bags * hot)).astype(np.int64)
    keys[:5] = 7  # a key whose few pieces leave quarters empty when block is large
    g = dyadic(rng, (bags, dim))
    uq, out = O.pooling_backprop(keys, SUM, O.FIXED, None, bags, hot, None, O.F32, g, O.F32, dim,
                                 block=block)
    ref = dense_grad_torch(keys, SUM, O.FIXED, None, bags, hot, None, g, rows)
    assert np.array_equal(sparse_to_dense(uq, out, rows, O.F32), ref)
    w = rng.uniform(0.1, 1.0, size=bags * hot).astype(np.float32)
    gn = rng.normal(0, 1, size=(bags, dim)).astype(np.float32)
    uq, out = O.pooling_backprop(keys, WMEAN, O.FIXED, None, bags, hot, w, O.F32, gn, O.F32, dim,
                                 block=block)
    ref = dense_grad_torch(keys, WMEAN, O.FIXED, None, bags, hot, w, gn, rows)
    assert np.allclose(sparse_to_dense(uq, out, rows, O.F32), ref, rtol=1e-5, atol=1e-5)

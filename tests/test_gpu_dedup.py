"""GPU parity of key dedup (Deduper::dedup, cuda_ops/deduper.cuh:136-221) and
of the dedup-then-gather of the C2 workload against the oracle.

Cases follow tests/kernels/deduper_tests.cu:139-348: all unique, all
identical, empty, single key, negative keys (signed order), random keys
checked for the round-trip invariants, plus the benchmark's 262,144 Zipf keys.
The gathered output must equal the plain gather bitwise."""
import ctypes

import numpy as np
import pytest

from nve_helpers import float_table, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def workspace(n):
    b = ctypes.c_uint64()
    _lib.call("nve_amd_dedup_workspace_size", n, ctypes.byref(b))
    return torch.empty(max(int(b.value), 1), dtype=torch.uint8, device="cuda"), int(b.value)


def gpu_dedup(keys):
    n = keys.size
    kt = _lib.KEY_INT32 if keys.dtype == np.int32 else _lib.KEY_INT64
    tdt = torch.int32 if keys.dtype == np.int32 else torch.int64
    d_keys = to_dev(keys) if n else torch.empty(1, dtype=tdt, device="cuda")
    outs = [torch.full((max(n, 1),), -7, dtype=tdt, device="cuda") for _ in range(4)]
    ws, wb = workspace(n)
    nu = ctypes.c_int64(-1)
    _lib.call("nve_amd_dedup", kt, n, vp(d_keys), *[vp(o) for o in outs], ctypes.byref(nu), vp(ws), wb,
              stream_ptr())
    torch.cuda.synchronize()
    u = nu.value
    uq, ct, inv, off = [o.cpu().numpy() for o in outs]
    return u, uq[:u], ct[:u], inv[:n], off[:u]


def check_against_oracle(keys):
    u, uq, ct, inv, off = gpu_dedup(keys)
    ru, rc, rinv, roff = O.dedup(keys)
    assert u == ru.size
    assert np.array_equal(uq, ru) and np.array_equal(ct, rc)
    assert np.array_equal(inv, rinv) and np.array_equal(off, roff)
    # invariants: ascending unique keys, counts sum, inverse covers every position once
    assert np.all(np.diff(uq) > 0)
    assert ct.sum() == keys.size
    assert np.array_equal(np.sort(inv), np.arange(keys.size))
    for k in range(min(u, 50)):
        pos = inv[off[k]:off[k] + ct[k]]
        assert np.all(keys[pos] == uq[k]) and np.all(np.diff(pos) > 0)


@pytest.mark.parametrize("dtype", [np.int64, np.int32])
def test_dedup_edge_cases(dtype):
    check_against_oracle(np.arange(1000, dtype=dtype)[::-1].copy())           # all unique
    check_against_oracle(np.full(3000, 42, dtype=dtype))                      # all identical
    check_against_oracle(np.array([5], dtype=dtype))                          # single key
    check_against_oracle(np.array([3, -1, 7, -1, -(2**31 - 1), 3, 0], dtype=dtype))  # signed order
    u, *_ = gpu_dedup(np.zeros(0, dtype=dtype))                                # empty
    assert u == 0


@pytest.mark.parametrize("n,hi", [(5000, 100), (70000, 2**40), (262144, 50_000_000)])
def test_dedup_random(n, hi):
    rng = np.random.default_rng(n)
    keys = rng.integers(-hi, hi, size=n).astype(np.int64)
    check_against_oracle(keys)


@pytest.mark.parametrize("case", ["below_bit_27", "bit_27_set_once", "high_common_bits", "int32_small",
                                  "negative_mixed"])
def test_dedup_sort_bits_first_assumed_then_checked(case):
    """The sort first assumes the keys differ only below bit 27 (three 9-bit
    passes, no host round trip) and checks the assumption against the key span
    it reduces on the way; a batch that differs higher up is deduplicated
    again on its exact bits.  Both sides of the boundary, keys sharing high
    bits, and keys whose sign bit differs."""
    rng = np.random.default_rng(27)
    n = 70000
    if case == "below_bit_27":
        keys = rng.integers(0, 2**27, size=n).astype(np.int64)
        keys[:2] = [0, 2**27 - 1]
    elif case == "bit_27_set_once":
        keys = rng.integers(0, 2**27, size=n).astype(np.int64)
        keys[n // 2] = 2**27
    elif case == "high_common_bits":
        keys = (2**40 + 12345 + rng.integers(0, 2**26, size=n)).astype(np.int64)
    elif case == "int32_small":
        keys = rng.integers(0, 5_000_000, size=n).astype(np.int32)
    else:
        keys = rng.integers(-1000, 1000, size=n).astype(np.int64)
    check_against_oracle(keys)


@pytest.mark.parametrize("n", [2, 3, 1023, 1024, 1025, 4096 * 1024, 4096 * 1024 + 1])
@pytest.mark.parametrize("distinct", [1, 7, None])
def test_dedup_run_block_edges(n, distinct):
    """The runs are written by 1024-key blocks that take the head counts and
    last heads of the blocks before them as carry-in, for up to 4096 blocks
    (one more block falls back to the scan-based path): sizes on either side
    of a block and of that limit, with one key (a single run through every
    block), seven keys (runs crossing block edges) and all-distinct keys."""
    rng = np.random.default_rng(n + (distinct or 0))
    if distinct is None:
        keys = rng.permutation(n).astype(np.int64)
    else:
        keys = rng.integers(0, distinct, size=n).astype(np.int64) * 1000003
    check_against_oracle(keys)


def test_dedup_multi_level_scans():
    """4096 * 4096 + 3001 keys: the run-head scan recurses twice (more than
    4096 blocks of 4096) and each radix digit row spans several 1024-tile
    chunks."""
    rng = np.random.default_rng(9)
    check_against_oracle(rng.integers(-500, 1500, size=4096 * 4096 + 3001).astype(np.int64))


def test_dedup_benchmark_zipf_keys_and_gather():
    """C2 shape: 262,144 Zipf(1.05) keys over 50M rows (reference generator),
    on a smaller table of the same row width (keys reduced modulo its rows)."""
    rng = np.random.default_rng(3)
    n, rows, dim = 262144, 200000, 128
    x = rng.random(n)
    keys = O.power_law(x, 1, 50_000_000, 1.05) % rows
    check_against_oracle(keys)
    tb = float_table(rng, rows, dim, O.F16, dyadic_values=False)
    d_tab, d_keys = to_dev(tb.reshape(-1)), to_dev(keys)
    out = torch.zeros((n, dim * 2), dtype=torch.uint8, device="cuda")
    ws, wb = workspace(n)
    _lib.call("nve_amd_dedup_gather", _lib.KEY_INT64, n, vp(d_keys), vp(d_tab), rows, dim * 2, vp(out),
              dim * 2, vp(ws), wb, stream_ptr())
    torch.cuda.synchronize()
    ref, hits = O.gather(keys, np.ascontiguousarray(tb).reshape(-1), dim * 2, rows)
    assert hits == n
    assert np.array_equal(out.cpu().numpy(), ref)


def test_dedup_gather_int32_and_out_of_range_keys_untouched():
    rng = np.random.default_rng(5)
    rows, dim = 3000, 24
    tb = float_table(rng, rows, dim, O.F32)
    keys = rng.integers(-50, rows + 50, size=5000).astype(np.int32)
    d_tab, d_keys = to_dev(tb.reshape(-1)), to_dev(keys)
    out = torch.full((keys.size, dim * 4), 0xCD, dtype=torch.uint8, device="cuda")
    ws, wb = workspace(keys.size)
    _lib.call("nve_amd_dedup_gather", _lib.KEY_INT32, keys.size, vp(d_keys), vp(d_tab), rows, dim * 4,
              vp(out), dim * 4, vp(ws), wb, stream_ptr())
    torch.cuda.synchronize()
    exp = np.full((keys.size, dim * 4), 0xCD, np.uint8)
    ref, _ = O.gather(keys, np.ascontiguousarray(tb).reshape(-1), dim * 4, rows, out=exp)
    assert np.array_equal(out.cpu().numpy(), ref)


@pytest.mark.parametrize("case", ["all_same", "one_key", "odd_width", "strided_out", "distinct"])
def test_dedup_gather_hash_edge_cases(case):
    """The hash dedup's corner cases against the oracle gather: every key the
    same (one owner, every other position copies it), a single key, 6-byte
    rows (2-byte copies), an output stride wider than the row (the padding
    untouched), all keys distinct (every position an owner)."""
    rng = np.random.default_rng(["all_same", "one_key", "odd_width", "strided_out", "distinct"].index(case))
    rows, dim, n = 4000, 32, 3000
    width = dim * 2
    if case == "odd_width":
        width = 6
    tb = rng.integers(0, 256, size=(rows, width), dtype=np.uint8)
    if case == "all_same":
        keys = np.full(n, 1234, np.int64)
    elif case == "one_key":
        keys = np.array([rows - 1], np.int64)
    elif case == "distinct":
        keys = rng.permutation(rows)[:n].astype(np.int64)
    else:
        keys = rng.integers(0, rows, size=n).astype(np.int64)
    stride = width + 32 if case == "strided_out" else width
    d_tab, d_keys = to_dev(tb.reshape(-1)), to_dev(keys)
    out = torch.full((keys.size, stride), 0x5A, dtype=torch.uint8, device="cuda")
    ws, wb = workspace(keys.size)
    ws.fill_(0x77)  # a workspace holding anything (the hash table is cleared by the call)
    _lib.call("nve_amd_dedup_gather", _lib.KEY_INT64, keys.size, vp(d_keys), vp(d_tab), rows, width, vp(out),
              stride, vp(ws), wb, stream_ptr())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got[:, :width], tb[keys])
    assert np.all(got[:, width:] == 0x5A)


def test_dedup_gather_reuses_a_workspace_across_batches():
    """Two batches through one workspace: the second sees no state of the first."""
    rng = np.random.default_rng(12)
    rows, dim = 5000, 16
    tb = float_table(rng, rows, dim, O.F32)
    d_tab = to_dev(tb.reshape(-1))
    ws, wb = workspace(4000)
    for n in (4000, 1500):
        keys = rng.integers(0, rows, size=n).astype(np.int64)
        d_keys = to_dev(keys)
        out = torch.zeros((n, dim * 4), dtype=torch.uint8, device="cuda")
        _lib.call("nve_amd_dedup_gather", _lib.KEY_INT64, n, vp(d_keys), vp(d_tab), rows, dim * 4, vp(out),
                  dim * 4, vp(ws), wb, stream_ptr())
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), np.ascontiguousarray(tb).reshape(rows, -1).view(np.uint8)[keys])


@pytest.mark.parametrize("case", ["wide_rows", "wide_keys"])
def test_dedup_gather_wide_rows_and_64_bit_table_keys(case):
    """Rows wider than one lane group's 1 KiB (each row copied in several
    pieces, by the owners and by the repeats), and a table that declares
    more than 2^32 rows, whose hash slots hold 64-bit keys (every key of the
    batch indexes the table's first rows, which are the ones allocated)."""
    rng = np.random.default_rng(31)
    n = 9000
    if case == "wide_rows":
        rows, width, declared = 700, 2064, 700  # 129 16-byte pieces: 3 pieces per lane group
    else:
        rows, width, declared = 3000, 64, 2**33 + 5
    tb = rng.integers(0, 256, size=(rows, width), dtype=np.uint8)
    keys = (O.power_law(rng.random(n), 1, rows, 1.05) % rows).astype(np.int64)
    keys[::97] = rng.integers(0, rows, size=keys[::97].size)
    d_tab, d_keys = to_dev(tb.reshape(-1)), to_dev(keys)
    out = torch.full((n, width), 0x3C, dtype=torch.uint8, device="cuda")
    ws, wb = workspace(n)
    ws.fill_(0x11)
    _lib.call("nve_amd_dedup_gather", _lib.KEY_INT64, n, vp(d_keys), vp(d_tab), declared, width, vp(out),
              width, vp(ws), wb, stream_ptr())
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy(), tb[keys])


@pytest.mark.parametrize("seed", range(4))
def test_dedup_gather_random_shapes(seed):
    """Seeded random batches: sizes across workgroup edges, row widths from 2
    bytes to several pieces per lane group, padded output strides, uniform /
    Zipf / out-of-range / single-key batches, int32 and int64 keys, and a
    workspace holding arbitrary bytes; every output row must be the table's
    row of its key, and rows of keys outside the table untouched."""
    rng = np.random.default_rng(500 + seed)
    for _ in range(6):
        n = int(rng.choice([1, 2, 1023, 1025, 4097])) if rng.random() < 0.3 else int(rng.integers(1, 120_000))
        rows = int(rng.integers(1, 100_000))
        width = int(rng.choice([2, 6, 16, 64, 256, 260, 1040, 2064]))
        stride = width + int(rng.choice([0, 0, 16, 2]))
        kind = int(rng.integers(0, 4))
        if kind == 0:
            keys = rng.integers(0, rows, size=n)
        elif kind == 1:
            keys = (rng.zipf(1.05 + rng.random(), size=n) - 1) % rows
        elif kind == 2:
            keys = rng.integers(-5, rows + 5, size=n)
        else:
            keys = np.full(n, rng.integers(0, rows))
        kdt = np.int32 if rng.random() < 0.3 else np.int64
        keys = keys.astype(kdt)
        tb = rng.integers(0, 256, size=(rows, width), dtype=np.uint8)
        d_tab, d_keys = to_dev(tb.reshape(-1)), to_dev(keys)
        out = torch.full((n, stride), 0x5A, dtype=torch.uint8, device="cuda")
        ws, wb = workspace(n)
        ws.fill_(int(rng.integers(0, 256)))
        kt = _lib.KEY_INT32 if kdt == np.int32 else _lib.KEY_INT64
        _lib.call("nve_amd_dedup_gather", kt, n, vp(d_keys), vp(d_tab), rows, width, vp(out), stride, vp(ws), wb,
                  stream_ptr())
        torch.cuda.synchronize()
        k64 = keys.astype(np.int64)
        ok = (k64 >= 0) & (k64 < rows)
        exp = np.full((n, stride), 0x5A, np.uint8)
        exp[ok, :width] = tb[k64[ok]]
        assert np.array_equal(out.cpu().numpy(), exp), (n, rows, width, stride, kind, kdt)

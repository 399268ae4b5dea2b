"""Pins for the oracle's set-associative cache model, histogram and dedup.

Checks are closed forms (set/tag arithmetic, sizing), brute force (Counter,
sorted()), an independent sort-based formulation of the replacement policy for
tie-free priorities (the same idea as the reference's own CPU model in
tests/kernels/gpu_insert_tests.cu:313-470), and hand-derived lane traces of
the 8-lane bitonic networks for the tie cases.
"""
import collections

import numpy as np
import pytest

from oracle import oracle as O


def test_num_sets_closed_form():
    # per set: 8*8 tag bytes + 8*256 data bytes + 8*4 counter bytes = 2144
    assert O.cache_num_sets(32 * 2**30, 256, 8) == 32 * 2**30 // 2144 == 16025997
    assert O.cache_num_sets(32 * 10**9, 256, 8) == 14925373
    # int32 tags: 32 B; unaligned row 260 B -> 2080 B data per set
    assert O.cache_num_sets(10**6, 260, 4) == 10**6 // (32 + 2080 + 32)
    assert O.cache_num_sets(100, 256, 8) == 0


@pytest.mark.parametrize("key_bytes", [4, 8])
def test_set_tag_round_trip(key_bytes):
    c = O.Cache(1 << 20, 64, key_bytes)
    S = c.num_sets
    rng = np.random.default_rng(0)
    hi = 2**31 - 1 if key_bytes == 4 else 2**62
    for k in rng.integers(0, hi, size=2000).tolist():
        s, t = c.set_of(k), c.tag_of(k)
        assert s == k % S and t == k // S
        assert c.key_of(t, s) == k


def test_negative_keys_use_unsigned_arithmetic():
    c = O.Cache(1 << 20, 64, 8)
    S = c.num_sets
    for k in (-1, -5, -(2**40)):
        u = k % (2**64)
        assert c.set_of(k) == u % S
        assert c.key_of(c.tag_of(k), c.set_of(k)) == k


def _uvm(rows, rb, seed=0):
    return np.random.default_rng(seed).integers(0, 256, size=rows * rb, dtype=np.uint8)


def test_first_insert_into_empty_set_lands_in_way_7():
    # Empty set: all way counters are 0, SortBlock swaps nothing, the reversal
    # maps lane 0 to way 7 (ec_set_associative_modify.cuh:264-276).
    rb = 32
    c = O.Cache(1 << 16, rb, 8)
    uvm = _uvm(1000, rb)
    c.insert_keys(np.array([123], np.int64), uvm=uvm)
    assert c.find_way(123) == 7
    s = c.set_of(123)
    assert c.counters()[s * 8 + 7] == np.float32(1.0)
    row = c.data()[(s * 8 + 7) * rb:(s * 8 + 8) * rb]
    assert np.array_equal(row, uvm[123 * rb:124 * rb])


def test_nine_equal_priorities_collapse_onto_one_key():
    # MergeBlock (:73-103) has no equality guard: with equal priorities every
    # lower lane copies its partner, so after j=4,2,1 all lanes hold chunk-0
    # lane 7.  Hand trace: pos=[c0..c7] -> [c4,c5,c6,c7,c4,..] -> [c6,c7,..] -> [c7]*8.
    rb = 16
    c = O.Cache(1 << 16, rb, 8)
    S = c.num_sets
    keys = np.array([5 + S * i for i in range(1, 10)], np.int64)  # 9 keys, one set
    uvm = _uvm(int(keys.max()) + 1, rb)
    c.insert_keys(keys, uvm=uvm)
    # histogram order: equal counts -> ascending key; candidate 7 is keys[7]
    ways = [c.find_way(int(k)) for k in keys]
    tags = c.tags()[5 * 8:6 * 8]
    assert all(c.key_of(t, 5) == keys[7] for t in tags)
    assert ways[7] == 0 and all(w == -1 for i, w in enumerate(ways) if i != 7)


def test_eight_equal_priorities_all_resident():
    # one chunk only: SortBlock has an equality guard, no duplication
    rb = 16
    c = O.Cache(1 << 16, rb, 8)
    S = c.num_sets
    keys = np.array([9 + S * i for i in range(8)], np.int64)
    uvm = _uvm(int(keys.max()) + 1, rb)
    c.insert_keys(keys, uvm=uvm)
    ways = sorted(c.find_way(int(k)) for k in keys)
    assert ways == list(range(8))


def _sort_policy(sets_state, cand, priority, ukeys, key_of_set):
    """Tie-free formulation: best <=8 new candidates by priority replace the
    lowest-counter ways when strictly better."""
    tags, ctr = sets_state
    new = []
    for loc in cand:
        hit = [w for w in range(8) if key_of_set(tags[w]) == ukeys[loc]]
        for w in hit:
            ctr[w] += priority[loc]
        if not hit:
            new.append(loc)
    num_repl = min(8, len(cand))
    best = sorted(new, key=lambda l: -priority[l])[:num_repl]
    order = sorted(range(8), key=lambda w: (0.0 if tags[w] == -1 else ctr[w]))
    eff = [0.0 if tags[w] == -1 else ctr[w] for w in order]
    out = []
    for x, loc in enumerate(best):
        if priority[loc] > eff[x]:
            out.append((order[x], loc))
    return out


def test_replacement_tie_free_matches_sort_formulation():
    rng = np.random.default_rng(42)
    rb = 8
    c = O.Cache(4 * (64 + 64 + 32) + 10, rb, 8)  # 4 sets
    S = c.num_sets
    assert S == 4
    uvm = _uvm(4000, rb)
    for rnd in range(30):
        m = int(rng.integers(1, 40))
        ukeys = rng.choice(4000, size=m, replace=False).astype(np.int64)
        # distinct priorities, and never equal to existing counters (tie-free)
        priority = (rng.permutation(m) + 1).astype(np.float32) / np.float32(7.0) + np.float32(rnd * 0.001)
        tags_before = c.tags().reshape(S, 8)
        ctr_before = c.counters().reshape(S, 8).astype(np.float64)
        ts = c.c.global_ts + 1
        expected = {}
        for s in range(S):
            cand = [i for i in range(m) if ukeys[i] % S == s]
            tags = list(tags_before[s])
            resident = {c.key_of(t, s) for t in tags if t != -1}
            if cand:
                # decay as defined by the oracle: float32(float64(0.95f) ** delta)
                st = np.ctypeslib.as_array(O.ctypes.cast(c.c.set_ts, O.ctypes.POINTER(O.ctypes.c_int64)), (S,))[s]
                d = ts - st
                ctr = [np.float32(v) for v in ctr_before[s]]
                if d > 0:
                    f = np.float32(np.power(np.float64(np.float32(0.95)), d))
                    ctr = [np.float32(v * f) for v in ctr]
                key_of = (lambda t, s=s: c.key_of(t, s) if t != -1 else None)
                for w, loc in _sort_policy((tags, ctr), cand, priority, ukeys, key_of):
                    old = key_of(tags[w])
                    resident.discard(old)
                    resident.add(int(ukeys[loc]))
            expected[s] = resident
        src = (ukeys.astype(np.uint64) * np.uint64(rb) + np.uint64(uvm.ctypes.data))
        sets, ways = c.insert_hist(ukeys, priority, src)
        tags_after = c.tags().reshape(S, 8)
        got = {s: {c.key_of(t, s) for t in tags_after[s] if t != -1} for s in range(S)}
        assert got == expected, (rnd, got, expected)
        for s, w in zip(sets, ways):
            k = c.key_of(tags_after[s][w], s)
            assert np.array_equal(c.data()[(s * 8 + w) * rb:(s * 8 + w + 1) * rb], uvm[k * rb:(k + 1) * rb])


def test_hits_increment_counters_and_never_duplicate():
    rb = 8
    c = O.Cache(1 << 14, rb, 8)
    uvm = _uvm(100, rb)
    c.insert_keys(np.array([3], np.int64), uvm=uvm)
    s = c.set_of(3)
    w = c.find_way(3)
    c.insert_keys(np.array([3, 3, 4], np.int64), uvm=uvm)
    # decay once (delta 1) then + 2/3
    exp = np.float32(np.float32(1.0) * np.float32(np.power(np.float64(np.float32(0.95)), 1))) + np.float32(2.0) * np.float32(1.0 / np.float32(3))
    assert c.find_way(3) == w
    got = c.counters()[s * 8 + w]
    assert abs(got - exp) <= 1e-7
    assert sum(1 for t in c.tags()[s * 8:s * 8 + 8] if c.key_of(t, s) == 3) == 1


def test_erase_invalidates_every_matching_way():
    rb = 8
    c = O.Cache(1 << 14, rb, 8)
    uvm = _uvm(100, rb)
    c.insert_keys(np.array([1, 2, 3], np.int64), uvm=uvm)
    assert all(c.find_way(k) >= 0 for k in (1, 2, 3))
    assert c.erase(np.array([2, 77], np.int64)) == 1
    assert c.find_way(2) == -1 and c.find_way(1) >= 0 and c.find_way(3) >= 0


def test_resolve_hits_and_misses():
    rb = 16
    c = O.Cache(1 << 14, rb, 8)
    uvm = _uvm(500, rb)
    c.insert_keys(np.array([10, 20, 30], np.int64), uvm=uvm)
    keys = np.array([10, 11, 20, 499, 30], np.int64)
    rows, hits, misses = c.resolve(keys, uvm)
    assert misses == 2
    assert int(hits[0]) == 0b10101
    assert rows[1] == uvm.ctypes.data + 11 * rb


def test_histogram_brute_force():
    rng = np.random.default_rng(9)
    keys = rng.integers(-50, 50, size=1000).astype(np.int64)
    uk, pr, fi = O.histogram(keys)
    cnt = collections.Counter(keys.tolist())
    exp = sorted(cnt.items(), key=lambda kv: (-kv[1], kv[0]))
    assert uk.tolist() == [k for k, _ in exp]
    norm = np.float32(1.0) / np.float32(1000)
    assert np.array_equal(pr, np.array([np.float32(c) * norm for _, c in exp], np.float32))
    first = {}
    for i, k in enumerate(keys.tolist()):
        first.setdefault(k, i)
    assert fi.tolist() == [first[k] for k, _ in exp]


@pytest.mark.parametrize("n", [0, 1, 2, 1000])
def test_dedup_round_trip(n):
    rng = np.random.default_rng(n)
    keys = rng.integers(-30, 200, size=n).astype(np.int64)
    uq, ct, inv, off = O.dedup(keys)
    assert uq.tolist() == sorted(set(keys.tolist()))
    assert ct.sum() == n
    assert sorted(inv.tolist()) == list(range(n))
    for u in range(uq.size):
        pos = inv[off[u]:off[u] + ct[u]]
        assert (keys[pos] == uq[u]).all()
        assert (np.diff(pos) > 0).all()  # stable: ascending original positions


def test_power_law_range_and_skew():
    rng = np.random.default_rng(0)
    x = rng.random(200000)
    y = O.power_law(x, 1, 1000, 1.05)
    assert y.min() >= 1 and y.max() <= 999
    c = np.bincount(y, minlength=1000)
    # Zipf-like: frequency decreases with the index, index 1 is the mode
    assert c[1] == c.max() and c[1] > 5 * c[100]


@pytest.mark.parametrize("host_modify", [False, True])
def test_insert_from_uvm_skips_keys_without_a_source_row(host_modify):
    """Closed form on an empty cache with room for every key: insert_from_uvm
    makes exactly the distinct keys inside the backing table resident, with
    their rows; keys below 0 or past the table never become resident."""
    rows, width = 500, 16
    uvm = np.arange(rows * width, dtype=np.uint32).astype(np.uint8).reshape(rows, width)
    c = O.Cache(2_000_000, width, 8, host_modify=host_modify)
    keys = np.array([3, 3, 499, 500, 501, -1, -7, 42, 10_000, 42], np.int64)
    c.insert_keys(keys, uvm=uvm.reshape(-1))
    tags = c.tags()
    ways = np.nonzero(tags != -1)[0]
    resident = set((tags[ways] * c.num_sets + ways // 8).tolist())
    assert resident == {3, 42, 499}
    for k in (3, 42, 499):
        slot = c.set_of(k) * 8 + c.find_way(k)
        assert np.array_equal(c.data().reshape(-1, width)[slot], uvm[k])

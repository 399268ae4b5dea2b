"""Pins for the oracle's host-metadata cache policy (modify_on_gpu = false):
the CPU DefaultHistogram (embed_cache.h:188-229) and CacheSAHostModify::insert
(ec_set_associative_host_modify.h:218-296).

Each expected value below is derived by hand from the policy's rules, written
as literals, so a dropped decay, a strict-vs-non-strict compare, a wrong
min-way choice or a missing one-record-per-way rule fails a case:
  * candidates are visited in histogram order (count descending);
  * a set is decayed once per call, on its first touch, by
    (float)pow(0.95, calls since it was last touched);
  * a resident key adds its priority to its way's counter;
  * otherwise the FIRST way with the smallest counter is replaced when
    priority >= that counter (empty ways keep whatever counter they had) and
    that way was not already replaced in this call.
"""
import collections
import ctypes

import numpy as np
import pytest

from oracle import oracle as O

ROW = 16  # bytes per row; a set costs 64 (tags) + 128 (rows) bytes on the device


def one_set_cache(key_bytes=8):
    c = O.Cache(192, ROW, key_bytes, host_modify=True)
    assert c.num_sets == 1
    return c


def views(c):
    n = c.num_sets * 8
    tags = np.ctypeslib.as_array(ctypes.cast(c.c.tags, ctypes.POINTER(ctypes.c_int64)), (n,))
    ctr = np.ctypeslib.as_array(ctypes.cast(c.c.counters, ctypes.POINTER(ctypes.c_float)), (n,))
    ts = np.ctypeslib.as_array(ctypes.cast(c.c.set_ts, ctypes.POINTER(ctypes.c_int64)), (c.num_sets,))
    return tags, ctr, ts


def no_decay_next_call(c):
    """Stamp every set with the next call's clock, so it is not decayed."""
    _, _, ts = views(c)
    ts[:] = c.c.global_ts + 1


F32 = np.float32


def test_num_sets_host_has_no_counter_term():
    # per set 8*8 tag bytes + 8*256 row bytes = 2112 (the device policy adds 32)
    assert O.cache_num_sets(32 * 2**30, 256, 8, host_modify=True) == 32 * 2**30 // 2112
    assert O.cache_num_sets(32 * 2**30, 256, 8, host_modify=False) == 32 * 2**30 // 2144
    assert O.cache_num_sets(10**6, 260, 4, host_modify=True) == 10**6 // (32 + 2080)
    assert O.Cache(32 * 2**20, 256, 8, host_modify=True).num_sets == 32 * 2**20 // 2112


@pytest.mark.parametrize("n", [1, 7, 500, 4000])
def test_histogram_host_brute_force(n):
    rng = np.random.default_rng(n)
    keys = rng.integers(-50, 200, size=n).astype(np.int64)
    cnt = collections.Counter(keys.tolist())
    first = {}
    for i, k in enumerate(keys.tolist()):
        first.setdefault(k, i)
    order = sorted(cnt, key=lambda k: (-cnt[k], first[k]))  # stable: first occurrence breaks ties
    uk, pr, fi = O.histogram_host(keys)
    assert uk.tolist() == order
    assert fi.tolist() == [first[k] for k in order]
    exp = np.array([F32(cnt[k]) / F32(n) for k in order], np.float32)  # a division, not * (1/n)
    assert np.array_equal(pr.view(np.uint32), exp.view(np.uint32))
    # the device histogram differs on ties: ascending key, and count * (1/n)
    duk, _, _ = O.histogram(keys)
    assert sorted(duk.tolist()) == sorted(uk.tolist())


def test_histogram_host_priority_is_a_division():
    # 3/7 rounds differently from 3 * (1/7) in float32
    keys = np.array([5, 5, 5, 1, 2, 3, 4], np.int64)
    _, pr, _ = O.histogram_host(keys)
    assert pr[0] == F32(3) / F32(7)
    assert F32(3) / F32(7) != F32(3) * (F32(1) / F32(7))


def test_fill_order_and_overflow():
    """Empty set: the first smallest counter is way 0, then way 1, ...; the 9th
    and 10th candidates meet min counter p7 > their priority and are skipped."""
    c = one_set_cache()
    ukeys = np.arange(100, 110, dtype=np.int64)
    prio = np.array([0.9, 0.8, 0.7, 0.6, 0.5, 0.4, 0.3, 0.2, 0.1, 0.05], np.float32)
    s, w = c.insert_hist_host(ukeys, prio)
    assert w.tolist() == [0, 1, 2, 3, 4, 5, 6, 7] and s.tolist() == [0] * 8
    tags, ctr, ts = views(c)
    assert tags.tolist() == list(range(100, 108))
    # first touch at clock 1: decay by 0.95^1 of zero counters, then set to p
    assert np.array_equal(ctr, prio[:8])
    assert ts.tolist() == [1] and c.c.global_ts == 1


def test_replacement_is_non_strict_after_decay():
    """Second call (clock 2, set last touched at 1): every counter *= f with
    f = (float)pow(0.95, 1).  A candidate whose priority equals the decayed
    minimum replaces that way; one ulp less does not."""
    f = F32(np.float64(F32(0.95)) ** 1)
    for delta_ulp, replaced in ((0, True), (-1, False)):
        c = one_set_cache()
        prio = np.array([0.8, 0.7, 0.6, 0.5, 0.4, 0.3, 0.2, 0.1], np.float32)
        c.insert_hist_host(np.arange(8, dtype=np.int64), prio)
        target = F32(prio[7] * f)
        p = target if delta_ulp == 0 else np.nextafter(target, F32(0))
        s, w = c.insert_hist_host(np.array([42], np.int64), np.array([p], np.float32))
        tags, ctr, _ = views(c)
        if replaced:
            assert w.tolist() == [7] and tags[7] == 42 and ctr[7] == p
        else:
            assert w.size == 0 and tags[7] == 7 and ctr[7] == target
        assert np.array_equal(ctr[:7], (prio[:7] * f).astype(np.float32))


def test_decay_spans_calls_since_last_touch():
    """A set untouched for 3 calls is decayed once by (float)pow(0.95, 3)."""
    c = O.Cache(192 * 4, ROW, 8, host_modify=True)
    assert c.num_sets == 4
    c.insert_hist_host(np.array([1], np.int64), np.array([0.5], np.float32))  # set 1, clock 1
    for _ in range(2):  # clocks 2, 3: touch set 0 only
        c.insert_hist_host(np.array([4], np.int64), np.array([0.25], np.float32))
    c.insert_hist_host(np.array([1], np.int64), np.array([0.125], np.float32))  # clock 4: hit
    _, ctr, ts = views(c)
    f3 = F32(np.float64(F32(0.95)) ** 3)
    assert ctr[8] == F32(F32(0.5) * f3) + F32(0.125)
    assert ts.tolist() == [3, 4, 0, 0]


def test_hit_adds_priority_and_does_not_move():
    c = one_set_cache()
    c.insert_hist_host(np.array([7, 8], np.int64), np.array([0.5, 0.25], np.float32))
    no_decay_next_call(c)
    s, w = c.insert_hist_host(np.array([8], np.int64), np.array([0.5], np.float32))
    tags, ctr, _ = views(c)
    assert w.size == 0 and tags[1] == 8 and ctr[1] == F32(0.75) and ctr[0] == F32(0.5)


def test_one_record_per_way_per_call():
    """Full set, way 3 the only small counter.  A (0.3) replaces way 3; B (0.3)
    then finds way 3 (now 0.3) as the first smallest, passes 0.3 >= 0.3, and is
    dropped because way 3 already has a record in this call."""
    c = one_set_cache()
    c.insert_hist_host(np.arange(8, dtype=np.int64), np.array([0.9, 0.9, 0.9, 0.1, 0.9, 0.9, 0.9, 0.9], np.float32))
    tags, ctr, _ = views(c)
    assert tags[3] == 3 and ctr[3] == F32(0.1)
    no_decay_next_call(c)
    s, w = c.insert_hist_host(np.array([50, 51], np.int64), np.array([0.3, 0.3], np.float32))
    assert w.tolist() == [3]
    tags, ctr, _ = views(c)
    assert tags[3] == 50 and 51 not in tags.tolist() and ctr[3] == F32(0.3)


def test_erased_way_keeps_its_counter():
    """Erase empties the tag but not the counter, so a weak candidate still
    loses to the stale counter (the device policy would count it as 0)."""
    c = one_set_cache()
    prio = np.array([0.9, 0.2, 0.8, 0.8, 0.8, 0.8, 0.8, 0.8], np.float32)
    c.insert_hist_host(np.arange(8, dtype=np.int64), prio)
    assert c.erase(np.array([1], np.int64)) == 1
    tags, ctr, _ = views(c)
    assert tags[1] == -1 and ctr[1] == F32(0.2)
    no_decay_next_call(c)
    s, w = c.insert_hist_host(np.array([60], np.int64), np.array([0.1], np.float32))
    assert w.size == 0 and tags[1] == -1
    s, w = c.insert_hist_host(np.array([61], np.int64), np.array([0.2], np.float32))
    # clock advanced again: the set decays first (0.2 * f < 0.2), then 61 wins way 1
    assert w.tolist() == [1] and tags[1] == 61


def test_max_update_truncates_in_histogram_order():
    c = O.Cache(192 * 16, ROW, 8, host_modify=True)
    assert c.num_sets == 16
    ukeys = np.arange(10, dtype=np.int64)  # ten different sets
    prio = np.linspace(0.9, 0.1, 10).astype(np.float32)
    s, w = c.insert_hist_host(ukeys, prio, max_update=3)
    assert s.tolist() == [0, 1, 2] and w.tolist() == [0, 0, 0]
    tags, ctr, ts = views(c)
    assert sorted(t for t in tags.tolist() if t != -1) == [0, 0, 0]  # tag = key // 16
    # the loop stops before the 4th candidate: its set is not even decayed / stamped
    assert ts.tolist()[:4] == [1, 1, 1, 0]


def test_insert_keys_rows_and_priorities():
    """insert_keys: histogram (first-occurrence rows) + policy + row copy."""
    rng = np.random.default_rng(3)
    c = O.Cache(192 * 8, ROW, 8, host_modify=True)
    keys = np.array([3, 11, 3, 19, 3, 11, 27, 35], np.int64)  # set 3 = {3, 11, 19, 27, 35}
    vals = rng.integers(0, 256, size=(keys.size, ROW), dtype=np.uint8)
    r = c.insert_keys(keys, values=vals.reshape(-1), value_stride=ROW)
    assert r == 5
    tags, ctr, _ = views(c)
    set3 = tags[24:32].tolist()
    # order: 3 (x3), 11 (x2), 19, 27, 35 (first occurrence) -> ways 0..4; tag = key // 8
    assert set3 == [0, 1, 2, 3, 4, -1, -1, -1]
    assert ctr[24:29].tolist() == [F32(3) / F32(8), F32(2) / F32(8)] + [F32(1) / F32(8)] * 3
    data = c.data().reshape(-1, ROW)
    for way, pos in enumerate([0, 1, 3, 6, 7]):  # first occurrence of each key
        assert np.array_equal(data[3 * 8 + way], vals[pos])


@pytest.mark.parametrize("host_modify", [True, False])
def test_clear(host_modify):
    c = O.Cache(192 * 4, ROW, 8, host_modify=host_modify)
    c.insert_keys(np.arange(20, dtype=np.int64), values=np.zeros(20 * ROW, np.uint8), value_stride=ROW)
    assert c.c.global_ts == 1
    before = views(c)[1].copy()
    c.clear()
    tags, ctr, ts = views(c)
    assert np.all(tags == -1) and np.all(ts == 0) and c.c.global_ts == 0
    if host_modify:
        assert np.all(ctr == 0)
    else:  # the device clear leaves counters (empty ways count as 0 there)
        assert np.array_equal(ctr, before)


def test_random_sequence_invariants():
    rng = np.random.default_rng(11)
    c = O.Cache(192 * 37, ROW, 8, host_modify=True)
    for step in range(8):
        keys = (rng.zipf(1.3, size=600) % 3000).astype(np.int64)
        uk, pr, _ = O.histogram_host(keys)
        s, w = c.insert_hist_host(uk, pr, max_update=50)
        tags, ctr, ts = views(c)
        assert s.size <= 50
        slots = s * 8 + w
        assert len(set(slots.tolist())) == slots.size  # one record per way
        # every recorded way now holds one of this call's candidates, counter = its priority
        pos = {int(k): i for i, k in enumerate(uk.tolist())}
        for sl in slots.tolist():
            key = int(tags[sl]) * c.num_sets + sl // 8
            assert key in pos and ctr[sl] == pr[pos[key]]
        # no key is resident twice; every resident key is in its own set
        for st in range(c.num_sets):
            ks = [int(t) * c.num_sets + st for t in tags[st * 8:st * 8 + 8].tolist() if t != -1]
            assert len(ks) == len(set(ks))
            assert all(k % c.num_sets == st for k in ks)
        assert c.c.global_ts == step + 1

"""GPU parity of the cache insert's hashed histogram (caches with at least as
many sets as the batch has keys) against the oracle's lane-exact model of the
reference's insert: after every insert the tags, way counters (bitwise), set
timestamps and cached rows equal the model's.

The hashed histogram replaces the sorted one (ten radix passes and two
readbacks) by hash counts, per-set candidate chains and a sort of each set's
few candidates into histogram order (count descending, then key ascending in
the key's signed order), so these cases aim at what that order decides: ties
of counts, repeats, negative and wide keys, the 64-bit key -1, the first
occurrence's values, keys outside the backing table, decay across inserts, and
a set with more candidates than the hashed path takes (the insert then falls
back to the sorted histogram with the same result)."""
import numpy as np
import pytest

from nve_helpers import float_table, to_dev, vp
from oracle import oracle as O
from pynve import _lib
from test_gpu_cache_insert import assert_same_state, table_insert
from test_gpu_cache_lookup import CachedTable

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

BIG = 8 * 1024 * 1024  # 16 x 4-byte columns: ~13,000 sets, more than any batch below


@pytest.mark.parametrize("key_bytes", [8, 4])
def test_hashed_sequence_matches_model(key_bytes):
    rng = np.random.default_rng(301 + key_bytes)
    rows, dim = 50000, 16
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, BIG, key_bytes)
    assert ct.num_sets >= 3000
    kdt = np.int64 if key_bytes == 8 else np.int32
    for step in range(8):
        # Zipf repeats (counts differ, many ties among singletons), and sets
        # that fill up over the steps: keys confined to 1/8 of the sets' range
        keys = (rng.zipf(1.3, size=3000) % 20000).astype(kdt)
        keys = (keys // 8 * 8 * (1 + step % 2) % rows).astype(kdt) if step >= 4 else keys
        vals = uvm[keys.astype(np.int64)]
        table_insert(ct, keys, vals, ct.width)
        ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
        assert_same_state(ct)
    ct.close()


def test_hashed_all_ties_and_full_sets():
    """Every key once (all priorities equal), eight to twenty keys per set:
    the candidates' order inside a set and the networks' tie rules decide."""
    rng = np.random.default_rng(307)
    rows, dim = 200000, 8
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, 1024 * 1024, 8)
    ns = ct.num_sets
    n = min(ns, 4000)
    for step in range(4):
        sets = rng.integers(0, max(1, n // 12), size=n)  # a few hundred sets, ~12 keys each
        keys = (sets + ns * rng.integers(0, rows // ns, size=n)).astype(np.int64)
        keys = np.unique(keys)
        keys = rng.permutation(keys)
        vals = uvm[keys % rows]
        table_insert(ct, keys, vals, ct.width)
        ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
        assert_same_state(ct)
    ct.close()


@pytest.mark.parametrize("case", ["wide_int64", "negative_int32", "minus_one_int64", "bit_32"])
def test_hashed_any_integer_keys(case):
    rng = np.random.default_rng(["wide_int64", "negative_int32", "minus_one_int64", "bit_32"].index(case) + 311)
    rows, dim = 4000, 8
    uvm = float_table(rng, rows, dim, O.F32)
    kb = 4 if case == "negative_int32" else 8
    ct = CachedTable(uvm, BIG, kb)
    n = 3000
    base = rng.zipf(1.2, size=n) % 900
    if case == "wide_int64":
        keys = (base.astype(np.int64) * 0x1E3779B97F4A7C15 % (2**62)).astype(np.int64) - 2**61
    elif case == "negative_int32":
        keys = (base - 450).astype(np.int32) * 3_000_017
    elif case == "minus_one_int64":
        keys = (base - 450).astype(np.int64)
        keys[::7] = -1  # the all-ones key word: the hash table's extra slot
    else:
        keys = (base * 6_000_011 % (2**32)).astype(np.int64)
        keys[n // 2] = 2**32
    assert keys.size <= ct.num_sets
    for step in range(2):
        vals = rng.integers(0, 256, size=(keys.size, ct.width), dtype=np.uint8)
        table_insert(ct, keys, vals, ct.width)
        ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
        assert_same_state(ct)
        keys = rng.permutation(keys)
    ct.close()


def test_hashed_values_use_first_occurrence_and_padded_stride():
    rng = np.random.default_rng(313)
    rows, dim = 2000, 12
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, BIG, 8)
    keys = rng.integers(0, 300, size=1500).astype(np.int64)
    stride = ct.width + 16
    vals = rng.integers(0, 256, size=(keys.size, stride), dtype=np.uint8)  # each occurrence differs
    table_insert(ct, keys, vals, stride)
    ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=stride)
    assert_same_state(ct)
    ct.close()


@pytest.mark.parametrize("key_bytes", [8, 4])
def test_hashed_insert_from_uvm_with_keys_outside_the_backing_table(key_bytes):
    rng = np.random.default_rng(317 + key_bytes)
    rows, dim = 3000, 16
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, BIG, key_bytes)
    kdt = np.int64 if key_bytes == 8 else np.int32
    outside = np.array([rows + 5, -3], kdt)
    vals = rng.integers(0, 256, size=(1, ct.width), dtype=np.uint8)
    table_insert(ct, outside[:1], vals, ct.width)  # resident with its own values
    ct.model.insert_keys(outside[:1], values=vals.reshape(-1), value_stride=ct.width)
    for step in range(4):
        keys = (rng.zipf(1.2, size=2500) % (rows + 400) - 100).astype(kdt)  # about 17 % outside
        keys[::50] = outside[step % 2]
        _lib.call("nve_amd_table_insert_from_uvm", ct.table, ct.ctx, keys.size, vp(to_dev(keys)))
        ct.model.insert_keys(keys, uvm=ct.uvm_np.reshape(-1))
        assert_same_state(ct)
    assert ct.model.find_way(rows + 5) >= 0
    assert ct.model.find_way(-3) < 0
    ct.close()


@pytest.mark.parametrize("key_bytes", [8, 4])
def test_hashed_set_past_its_candidate_limit_falls_back(key_bytes):
    """40 keys of one set (the hashed path takes 32 per set): the insert is
    redone by the sorted histogram, with the same state as the model, and the
    next insert takes the hashed path again."""
    rng = np.random.default_rng(331 + key_bytes)
    rows, dim = 60000, 8
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, BIG, key_bytes)
    ns = ct.num_sets
    kdt = np.int64 if key_bytes == 8 else np.int32
    crowd = 17 + ns * np.arange(40)  # all in set 17
    others = rng.integers(0, rows, size=500)
    for step, keys in enumerate([np.concatenate([crowd, others, crowd[:5]]), rng.integers(0, rows, size=800)]):
        keys = rng.permutation(keys).astype(kdt)
        assert keys.size <= ns
        vals = uvm[keys.astype(np.int64) % rows]
        table_insert(ct, keys, vals, ct.width)
        ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
        assert_same_state(ct)
    ct.close()


@pytest.mark.parametrize("seed", range(12))
def test_hashed_random_shapes(seed):
    """Seeded random shapes: key width, row width, batch size, key spread and
    repeats, values or backing rows, against the model over three inserts."""
    rng = np.random.default_rng(1000 + seed)
    key_bytes = int(rng.choice([4, 8]))
    dim = int(rng.choice([4, 8, 16, 33]))
    rows = int(rng.integers(500, 40000))
    uvm = float_table(rng, rows, dim, O.F32)
    ct = CachedTable(uvm, int(rng.choice([2, 4, 8])) * 1024 * 1024, key_bytes)
    kdt = np.int64 if key_bytes == 8 else np.int32
    for step in range(3):
        n = int(rng.integers(2, min(ct.num_sets, 5000) + 1))
        spread = int(rng.integers(2, 4 * rows))
        keys = (rng.zipf(float(rng.uniform(1.05, 2.0)), size=n) % spread).astype(np.int64)
        if rng.random() < 0.3:
            keys = keys - spread // 2  # negative keys too
        keys = keys.astype(kdt)
        if rng.random() < 0.5:
            _lib.call("nve_amd_table_insert_from_uvm", ct.table, ct.ctx, keys.size, vp(to_dev(keys)))
            ct.model.insert_keys(keys, uvm=ct.uvm_np.reshape(-1))
        else:
            vals = rng.integers(0, 256, size=(keys.size, ct.width), dtype=np.uint8)
            table_insert(ct, keys, vals, ct.width)
            ct.model.insert_keys(keys, values=vals.reshape(-1), value_stride=ct.width)
        assert_same_state(ct)
    ct.close()


def test_c3_shaped_batch_into_an_empty_large_cache():
    """A C3-shaped batch (262,144 Zipf(1.2) keys over 4 M rows of 128 fp16,
    permuted) inserted from the backing table into an empty cache of 2^20 sets
    (the hashed path at full batch size; the oracle's model of a cache this
    large would take gigabytes, so the result is held to what an empty cache
    fixes): every set with at most 8 distinct candidates holds all of them, a
    fuller set holds 8 of them and none it left out has a higher count, each
    resident way's counter is its key's priority float(count) * (1 / float(n))
    bit for bit, touched sets carry timestamp 1 and the others nothing; then,
    with every backing row changed on the host, lookups return the old row for
    exactly the resident keys."""
    import ctypes
    rows, width, n = 4_000_000, 256, 262144
    ns_want = 1 << 20
    L = _lib.load()
    host = torch.arange(rows * (width // 4), dtype=torch.int32).view(torch.uint8).pin_memory()
    cfg = L.nve_gpu_table_config_default()
    cfg.cache_size = ns_want * 2144  # 64 B of tags, 2 KiB of rows, 32 B of counters per set
    cfg.row_size_in_bytes = width
    cfg.value_dtype = _lib.DT_F16
    cfg.uvm_table = host.data_ptr()
    cfg.uvm_num_rows = rows
    table = ctypes.c_void_p()
    _lib.call("nve_gpu_table_create", ctypes.byref(table), _lib.KEY_INT64, ctypes.byref(cfg), None)
    ctx = ctypes.c_void_p()
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    _lib.call("nve_table_create_execution_context", table, ctypes.byref(ctx), s, s, None, None)
    try:
        nsv = ctypes.c_int64()
        _lib.call("nve_amd_gpu_table_num_sets", table, ctypes.byref(nsv))
        ns = nsv.value
        assert ns == ns_want
        rng = np.random.default_rng(2024)
        perm = rng.permutation(rows)
        keys = perm[O.power_law(rng.random(n), 1, rows, 1.2).astype(np.int64) - 1].astype(np.int64)
        d_keys = to_dev(keys)
        _lib.call("nve_amd_table_insert_from_uvm", table, ctx, n, vp(d_keys))
        _lib.call("nve_context_wait", ctx)

        tags = np.zeros(ns * 8, np.int64)
        ctr = np.zeros(ns * 8, np.float32)
        ts = np.zeros(ns, np.int64)
        gts = ctypes.c_int64()
        _lib.call("nve_amd_gpu_table_export_state", table, tags.ctypes.data_as(ctypes.c_void_p),
                  ctr.ctypes.data_as(ctypes.c_void_p), ts.ctypes.data_as(ctypes.c_void_p), ctypes.byref(gts))
        assert gts.value == 1

        uk, cnt = np.unique(keys, return_counts=True)
        useti = uk % ns
        norm = np.float32(1.0) / np.float32(n)
        prio = cnt.astype(np.float32) * norm
        occ = np.nonzero(tags != -1)[0]
        res_set = occ // 8
        res_key = tags[occ] * ns + res_set
        # residents are candidates of their set, each once
        pos = np.searchsorted(uk, res_key)
        assert np.all(pos < uk.size) and np.array_equal(uk[pos], res_key)
        assert np.unique(res_key).size == res_key.size
        assert np.array_equal(ctr[occ].view(np.uint32), prio[pos].view(np.uint32))
        assert np.all(ctr[tags == -1] == 0.0)
        touched = np.zeros(ns, bool)
        touched[useti] = True
        assert np.array_equal(ts, touched.astype(np.int64))
        # per set: all candidates when at most 8, else 8 with no left-out count above a resident's
        per_set = np.bincount(useti, minlength=ns)
        held = np.bincount(res_set, minlength=ns)
        assert np.array_equal(held, np.minimum(per_set, 8))
        resident = np.zeros(uk.size, bool)
        resident[pos] = True
        full = np.nonzero(per_set > 8)[0]
        for st in full:
            idx = np.nonzero(useti == st)[0]
            assert cnt[idx][resident[idx]].min() >= cnt[idx][~resident[idx]].max()

        # backing rows changed on the host: resident keys still return the old row
        host.view(torch.int32).bitwise_xor_(0x5A5A5A5A)
        out = torch.zeros((uk.size, width), dtype=torch.uint8, device="cuda")
        d_uk = to_dev(uk)
        _lib.call("nve_table_find", table, ctx, uk.size, vp(d_uk), None, width, vp(out), None)
        _lib.call("nve_context_wait", ctx)
        torch.cuda.synchronize()
        got = out.cpu().view(torch.int32).numpy().reshape(uk.size, width // 4)
        base = (uk[:, None] * (width // 4) + np.arange(width // 4)[None, :]).astype(np.int32)
        want = np.where(resident[:, None], base, base ^ np.int32(0x5A5A5A5A))
        assert np.array_equal(got, want)
    finally:
        _lib.call("nve_context_wait", ctx)
        _lib.call("nve_context_destroy", ctx)
        _lib.call("nve_table_destroy", table)

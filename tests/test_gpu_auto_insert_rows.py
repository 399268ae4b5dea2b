"""LinearUVM auto-insert: where the inserted rows come from.

A collection of plain (or raw Concatenate) lookups keeps their output rows
and inserts those (layer_utils.cpp:145-213, the data copy at :187-193); a
pooled lookup has no per-key rows, so a collection that one starts or joins
promotes the rows from the backing table, and stays that way until it is
inserted (layer_utils.cpp:112-131, linear_embedding_layer.cu:197-206).  A
collection of rows needs one output stride throughout (layer_utils.cpp:120).

To see which rows went in, the backing table's rows of the first batch are
changed between the two lookups of a collection: rows taken from the
lookups are the old ones, rows promoted from the backing table the new ones.
The cache state after the insert (tags, way counters, set timestamps and
rows) must equal the oracle's insert of the same keys from that source."""
import ctypes

import numpy as np
import pytest

from nve_helpers import float_table, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib
from test_gpu_cache_insert import assert_same_state, gpu_state
from test_gpu_cache_lookup import CachedTable

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

ROWS, DIM = 12000, 32  # fp32 rows of 128 bytes


class Layer:
    def __init__(self, ct, min_size, default_row=-1):
        L = _lib.load()
        lc = L.nve_linear_uvm_layer_config_default()
        lc.min_insert_size_gpu = min_size
        lc.min_insert_freq_gpu = 0
        lc.default_row_index = default_row
        self.layer = ctypes.c_void_p()
        kt = _lib.KEY_INT32 if ct.key_bytes == 4 else _lib.KEY_INT64
        _lib.call("nve_linear_uvm_layer_create", ctypes.byref(self.layer), kt, ctypes.byref(lc), ct.table, None)
        self.ctx = ctypes.c_void_p()
        s = stream_ptr()
        _lib.call("nve_layer_create_execution_context", self.layer, ctypes.byref(self.ctx), s, s, None, None)
        self.ct = ct
        self.hr = (ctypes.c_float * 1)()

    def plain(self, keys, stride=None):
        stride = stride or self.ct.width
        out = torch.zeros(keys.size * stride, dtype=torch.uint8, device="cuda")
        d_keys = to_dev(keys)
        _lib.call("nve_layer_lookup", self.layer, self.ctx, keys.size, vp(d_keys), vp(out), stride, None, self.hr)
        return out.cpu().numpy().reshape(keys.size, stride)[:, :self.ct.width]

    def pooled(self, keys, stride=DIM * 4, hot=4):
        assert keys.size % hot == 0
        bags = keys.size // hot
        out = torch.zeros(bags * stride, dtype=torch.uint8, device="cuda")
        d_keys = to_dev(keys)
        _lib.call("nve_layer_lookup_pooled", self.layer, self.ctx, keys.size, vp(d_keys), vp(out), stride, None,
                  _lib.POOL_SUM, _lib.SPARSE_FIXED, None, 0, hot, None, 0, _lib.DT_F32, self.hr)

    def wait(self):
        _lib.call("nve_context_wait", self.ctx)

    def close(self):
        self.wait()
        _lib.call("nve_context_destroy", self.ctx)
        _lib.call("nve_layer_destroy", self.layer)


def host_rows(ct):
    """Writable view of the pinned backing table the GPU table reads."""
    return ct.h_uvm.numpy().reshape(ct.rows, ct.width)


@pytest.mark.parametrize("cache_bytes", [1 << 20, 16 << 20], ids=["sorted_insert", "hashed_insert"])
@pytest.mark.parametrize("kinds", [("plain", "plain"), ("concat", "plain"), ("pooled", "pooled"),
                                   ("plain", "pooled"), ("pooled", "plain")])
def test_collection_source_of_rows(kinds, cache_bytes):
    rng = np.random.default_rng(sum(map(len, kinds)) + cache_bytes % 97)
    uvm = float_table(rng, ROWS, DIM, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, cache_bytes, 8)
    lay = Layer(ct, min_size=2048)
    a = (rng.zipf(1.2, size=1024) % 6000).astype(np.int64)
    b = (6000 + rng.zipf(1.2, size=1024) % 6000).astype(np.int64)
    old = host_rows(ct).copy()

    def run(kind, keys):
        if kind == "plain":
            got = lay.plain(keys)
            assert np.array_equal(got, host_rows(ct)[keys])
        elif kind == "concat":  # raw Concatenate (stored type out): per-key rows like a plain lookup
            out = torch.zeros(keys.size * ct.width, dtype=torch.uint8, device="cuda")
            d_keys = to_dev(keys)
            _lib.call("nve_layer_lookup_pooled", lay.layer, lay.ctx, keys.size, vp(d_keys), vp(out), ct.width,
                      None, _lib.POOL_CONCAT, _lib.SPARSE_FIXED, None, 0, 1, None, 0, _lib.DT_F32, lay.hr)
            assert np.array_equal(out.cpu().numpy().reshape(keys.size, ct.width), host_rows(ct)[keys])
        else:
            lay.pooled(keys)

    run(kinds[0], a)
    assert lay.hr[0] == 0.0  # an empty cache: the default heuristic starts the collection
    lay.wait()
    assert np.all(gpu_state(ct)[0] == -1)  # collected, not inserted yet
    h = host_rows(ct)
    h[np.unique(a), 3::4] ^= np.uint8(0x80)  # negate the first batch's backing rows
    run(kinds[1], b)
    lay.wait()  # joins the insert the second lookup launched
    keys = np.concatenate([a, b])
    if "pooled" in kinds:
        ct.model.insert_keys(keys, uvm=host_rows(ct).reshape(-1))
        src = host_rows(ct)
    else:
        src = old
        ct.model.insert_keys(keys, values=old[keys].reshape(-1), value_stride=ct.width)
    assert_same_state(ct)
    # every resident row of the first batch carries the rows of its source
    mt = ct.model.tags()
    ways = np.nonzero(mt != -1)[0]
    resident = mt[ways] * ct.num_sets + ways // 8
    first = np.isin(resident, a)
    assert first.any()
    data = gpu_state(ct)[4].reshape(-1, ct.width)
    assert np.array_equal(data[ways[first]], src[resident[first]])
    lay.close()
    ct.close()


def test_consecutive_collections_reuse_rows_with_padded_stride():
    """Several inserts in a row from lookups with a padded output stride,
    alternating with one promoted from the backing table; each batch's keys
    are new to the cache, so its hit rate is 0 and the heuristic fires."""
    rng = np.random.default_rng(5)
    uvm = float_table(rng, ROWS, DIM, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 1 << 20, 8)
    lay = Layer(ct, min_size=1500)
    stride = ct.width + 48
    for r in range(6):
        keys = (r * 2000 + rng.zipf(1.3, size=1500) % 2000).astype(np.int64)
        if r % 3 == 2:
            lay.pooled(keys, hot=3)
        else:
            got = lay.plain(keys, stride=stride)
            assert np.array_equal(got, uvm[keys])
        assert lay.hr[0] == 0.0
        lay.wait()
        if r % 3 == 2:
            ct.model.insert_keys(keys, uvm=ct.uvm_np.reshape(-1))
        else:
            ct.model.insert_keys(keys, values=uvm[keys].reshape(-1), value_stride=ct.width)
        assert_same_state(ct)
    lay.close()
    ct.close()


def test_collection_of_rows_needs_one_stride():
    """A plain lookup with another stride cannot join a collection of rows
    (the lookup itself reports it); a pooled one with its own stride joins,
    and the collection then promotes from the backing table."""
    rng = np.random.default_rng(8)
    uvm = float_table(rng, ROWS, DIM, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 1 << 20, 8)
    lay = Layer(ct, min_size=2048)
    a = (rng.zipf(1.2, size=1024) % 6000).astype(np.int64)
    b = (6000 + rng.zipf(1.2, size=1024) % 6000).astype(np.int64)
    lay.plain(a)
    with pytest.raises(_lib.NVEError) as ei:
        lay.plain(b, stride=ct.width + 16)
    assert ei.value.status == _lib.RUNTIME
    assert "Output stride must be fixed during accumulation" in str(ei.value)
    lay.wait()
    assert np.all(gpu_state(ct)[0] == -1)
    lay.pooled(b, stride=DIM * 4 - 16)  # 28 of the 32 values: another stride, fine for a pooled lookup
    lay.wait()
    ct.model.insert_keys(np.concatenate([a, b]), uvm=ct.uvm_np.reshape(-1))
    assert_same_state(ct)
    lay.close()
    ct.close()


@pytest.mark.parametrize("key_bytes", [8, 4])
def test_keys_outside_the_table_drop_with_their_rows(key_bytes):
    """Keys outside the backing table (no default row) are dropped from a
    collection of rows together with their output rows, in runs: the rows
    that stay must still line up with their keys."""
    rng = np.random.default_rng(30 + key_bytes)
    uvm = float_table(rng, ROWS, DIM, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 1 << 20, key_bytes)
    kdt = np.int64 if key_bytes == 8 else np.int32
    keys = (rng.zipf(1.2, size=1200) % ROWS).astype(kdt)
    keys[5:9] = ROWS + 3
    keys[100] = ROWS + 1000
    keys[101] = -5
    keys[500:640] = -1
    keys[-3:] = ROWS
    keep = (keys >= 0) & (keys < ROWS)
    lay = Layer(ct, min_size=int(keep.sum()))
    got = lay.plain(keys)
    assert np.array_equal(got[keep], uvm[keys[keep].astype(np.int64)])
    lay.wait()
    kk = keys[keep]
    ct.model.insert_keys(kk, values=uvm[kk.astype(np.int64)].reshape(-1), value_stride=ct.width)
    assert_same_state(ct)
    lay.close()
    ct.close()

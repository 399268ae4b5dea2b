"""GPU parity of row updates: GpuTable::update / update_accumulate
(gpu_table.cu:579-1046), the GPU layer's update / accumulate
(gpu_embedding_layer.cu:500-639) and the LinearUVM layer's
(linear_embedding_layer.cu:230-285).

Closed forms checked: an update makes every resident key's cache row and every
in-range backing row equal to the update row, and leaves tags, counters and
all other rows alone; accumulate adds every update row (repeated keys add
several) -- on dyadic-fraction values, whose sums are exact in fp32 and fp16,
so the result does not depend on the order of the atomic adds.  Keys outside
the backing table are ignored there (update_accumulate.cuh key_in_range)."""
import ctypes

import numpy as np
import pytest

from nve_helpers import dyadic, float_table, hip_memcpy, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib
from test_gpu_cache_lookup import CachedTable, warm
from test_gpu_layer import GpuLayer

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def cache_state(ct):
    ns = ct.num_sets
    tags = np.zeros(ns * 8, np.int64 if ct.key_bytes == 8 else np.int32)
    cnt = np.zeros(ns * 8, np.float32)
    ts = np.zeros(ns, np.int64)
    gts = ctypes.c_int64()
    _lib.call("nve_amd_gpu_table_export_state", ct.table, tags.ctypes.data_as(ctypes.c_void_p),
              cnt.ctypes.data_as(ctypes.c_void_p), ts.ctypes.data_as(ctypes.c_void_p), ctypes.byref(gts))
    data = ctypes.c_void_p()
    _lib.call("nve_amd_gpu_table_data", ct.table, ctypes.byref(data))
    rows = np.zeros((ns * 8, ct.width), np.uint8)
    hip_memcpy(rows.ctypes.data, data.value, rows.nbytes)
    return tags, cnt, ts, rows


def slots_of(tags, num_sets, key):
    """Every way set*8+w whose rebuilt key (tag*num_sets + set, in the key's
    width) equals key -- the cache's closed-form set/tag math, empty ways
    included, as the update kernel compares them."""
    bits = 64 if tags.dtype == np.int64 else 32
    mask = (1 << bits) - 1
    uk = int(key) & mask
    s = uk % num_sets
    return [s * 8 + w for w in range(8) if ((int(tags[s * 8 + w]) & mask) * num_sets + s) & mask == uk]


def slot_of(tags, num_sets, key):
    sl = slots_of(tags, num_sets, key)
    return sl[0] if sl else -1


def table_host(ct):
    return ct.h_uvm.numpy().reshape(ct.rows, ct.width)


@pytest.mark.parametrize("key_bytes", [8, 4])
@pytest.mark.parametrize("disable_uvm_update", [False, True])
def test_table_update(key_bytes, disable_uvm_update):
    rng = np.random.default_rng(30 + key_bytes + disable_uvm_update)
    rows, dim = 5000, 32
    uvm = float_table(rng, rows, dim, O.F32, dyadic_values=False)
    ct = CachedTable(uvm, 200 * 1024, key_bytes)
    if disable_uvm_update:
        # recreate with the flag set (the helper builds the default config)
        ct.close()
        L = _lib.load()
        cfg = L.nve_gpu_table_config_default()
        cfg.cache_size, cfg.row_size_in_bytes, cfg.value_dtype = 200 * 1024, dim * 4, _lib.DT_F32
        cfg.uvm_table, cfg.uvm_num_rows, cfg.disable_uvm_update = ct.h_uvm.data_ptr(), rows, 1
        kt = _lib.KEY_INT32 if key_bytes == 4 else _lib.KEY_INT64
        _lib.call("nve_gpu_table_create", ctypes.byref(ct.table), kt, ctypes.byref(cfg), None)
        s = stream_ptr()
        _lib.call("nve_table_create_execution_context", ct.table, ctypes.byref(ct.ctx), s, s, None, None)
    warm(ct, rng, 1500, np.arange(0, 1200))
    tags0, cnt0, ts0, rows0 = cache_state(ct)
    uvm0 = table_host(ct).copy()
    kdt = np.int64 if key_bytes == 8 else np.int32
    resident = [k for k in range(1200) if slot_of(tags0, ct.num_sets, k) >= 0]
    keys = np.concatenate([rng.choice(resident, size=60, replace=False),
                           rng.choice(np.arange(2000, rows), size=40, replace=False),
                           np.array([rows, rows + 11, -1, -77])]).astype(kdt)
    vals = float_table(rng, keys.size, dim, O.F32, dyadic_values=False)
    d_keys, d_vals = to_dev(keys), to_dev(vals.reshape(-1))
    _lib.call("nve_table_update", ct.table, ct.ctx, keys.size, vp(d_keys), dim * 4, dim * 4, vp(d_vals))
    torch.cuda.synchronize()
    tags1, cnt1, ts1, rows1 = cache_state(ct)
    assert np.array_equal(tags1, tags0) and np.array_equal(cnt1, cnt0) and np.array_equal(ts1, ts0)
    exp_rows = rows0.copy()
    exp_uvm = uvm0.copy()
    for i, k in enumerate(keys):
        for sl in slots_of(tags0, ct.num_sets, int(k)):
            exp_rows[sl] = vals[i]
        if 0 <= k < rows and not disable_uvm_update:
            exp_uvm[k] = vals[i]
    assert np.array_equal(rows1, exp_rows)
    assert np.array_equal(table_host(ct), exp_uvm)
    # lookups now return the updated rows wherever they are served from
    inr = keys[(keys >= 0) & (keys < rows)]
    out = torch.zeros((inr.size, dim * 4), dtype=torch.uint8, device="cuda")
    d_in = to_dev(inr)
    _lib.call("nve_table_find", ct.table, ct.ctx, inr.size, vp(d_in), None, dim * 4, vp(out), None)
    got = out.cpu().numpy()
    for j, k in enumerate(inr):
        sl = slot_of(tags0, ct.num_sets, int(k))
        exp = exp_rows[sl] if sl >= 0 else exp_uvm[k]
        assert np.array_equal(got[j], exp)
    ct.close()


@pytest.mark.parametrize("dtype", [O.F32, O.F16])
def test_table_update_accumulate(dtype):
    rng = np.random.default_rng(40 + dtype)
    rows, dim = 4000, 24
    npdt = np.float32 if dtype == O.F32 else np.float16
    ddt = _lib.DT_F32 if dtype == O.F32 else _lib.DT_F16
    es = 4 if dtype == O.F32 else 2
    uvm = dyadic(rng, (rows, dim)).astype(npdt).view(np.uint8).reshape(rows, dim * es)
    ct = CachedTable(uvm, 150 * 1024, 8, value_dtype=ddt)
    warm(ct, rng, 1200, np.arange(0, 1000), elem_bytes=es)
    tags0, cnt0, ts0, rows0 = cache_state(ct)
    uvm0 = table_host(ct).copy()
    resident = [k for k in range(1000) if slot_of(tags0, ct.num_sets, k) >= 0]
    base = np.concatenate([rng.choice(resident, size=50, replace=False),
                           rng.choice(np.arange(1500, rows), size=30, replace=False)])
    keys = np.concatenate([base, base[:20], base[:5], np.array([rows + 3, -2])]).astype(np.int64)
    upd = dyadic(rng, (keys.size, dim)).astype(npdt)
    d_keys, d_upd = to_dev(keys), to_dev(upd.view(np.uint8).reshape(-1))
    _lib.call("nve_table_update_accumulate", ct.table, ct.ctx, keys.size, vp(d_keys), dim * es, dim * es,
              vp(d_upd), ddt)
    torch.cuda.synchronize()
    tags1, cnt1, ts1, rows1 = cache_state(ct)
    assert np.array_equal(tags1, tags0) and np.array_equal(cnt1, cnt0)
    exp_rows = rows0.copy().view(npdt).astype(np.float64)
    exp_uvm = uvm0.copy().view(npdt).astype(np.float64)
    for i, k in enumerate(keys):
        for sl in slots_of(tags0, ct.num_sets, int(k)):
            exp_rows[sl] += upd[i].astype(np.float64)
        if 0 <= k < rows:
            exp_uvm[k] += upd[i].astype(np.float64)
    # dyadic sums are exact in the table type
    assert np.array_equal(rows1.view(npdt), exp_rows.astype(npdt))
    assert np.array_equal(table_host(ct).view(npdt), exp_uvm.astype(npdt))
    ct.close()


@pytest.mark.parametrize("dim", [40, 39])
def test_accumulate_contended_fp16_row(dim):
    """300 adds of 2^-9 to the same fp16 row, all at once: every add lands,
    whether the row is added a 32-bit word (two elements) per lane (80-byte
    rows) or an element per lane (78-byte rows, half of them 2-byte aligned)."""
    rows = 100
    uvm = np.zeros((rows, dim), np.float16).view(np.uint8).reshape(rows, dim * 2)
    ct = CachedTable(uvm, 64 * 1024, 8, value_dtype=_lib.DT_F16)
    vals = np.zeros((1, dim * 2), np.uint8)
    ct.model.insert_keys(np.array([7], np.int64), uvm=ct.uvm_np.reshape(-1))
    ct.load_model()
    keys = np.full(300, 7, np.int64)
    upd = np.full((300, dim), 2.0 ** -9, np.float16)
    d_keys, d_upd = to_dev(keys), to_dev(upd.view(np.uint8).reshape(-1))
    _lib.call("nve_table_update_accumulate", ct.table, ct.ctx, keys.size, vp(d_keys), dim * 2, dim * 2,
              vp(d_upd), _lib.DT_F16)
    torch.cuda.synchronize()
    tags, _, _, rows1 = cache_state(ct)
    sl = slot_of(tags, ct.num_sets, 7)
    assert sl >= 0
    assert np.all(rows1[sl].view(np.float16) == np.float16(300 * 2.0 ** -9))
    assert np.all(table_host(ct)[7].view(np.float16) == np.float16(300 * 2.0 ** -9))
    del vals
    ct.close()


@pytest.mark.parametrize("dtype", [O.F32, O.F16])
def test_backing_accumulate_of_spread_repeats_is_in_position_order(dtype):
    """Repeated keys spread over 6000 positions (far beyond one worker's share
    of the batch): every backing row gets its updates one at a time, in
    position order -- bit for bit the sequential sum, on values whose sums
    round (not dyadic), so a lost add or another order shows."""
    rng = np.random.default_rng(60 + dtype)
    rows, dim, n = 50, 24, 6000
    npd = np.float32 if dtype == O.F32 else np.float16
    base = rng.normal(0, 1, size=(rows, dim)).astype(npd)
    uvm = base.view(np.uint8).reshape(rows, -1)
    ct = CachedTable(uvm, 64 * 1024, 8, value_dtype=_lib.DT_F32 if dtype == O.F32 else _lib.DT_F16)
    keys = rng.integers(0, rows, size=n).astype(np.int64)
    upd = rng.normal(0, 1, size=(n, dim)).astype(npd)
    d_keys, d_upd = to_dev(keys), to_dev(upd.view(np.uint8).reshape(-1))
    _lib.call("nve_table_update_accumulate", ct.table, ct.ctx, n, vp(d_keys), dim * upd.itemsize,
              dim * upd.itemsize, vp(d_upd), _lib.DT_F32 if dtype == O.F32 else _lib.DT_F16)
    torch.cuda.synchronize()
    want = base.copy()
    for i in range(n):  # fp32 add per element, rounded back to the row type
        want[keys[i]] = (want[keys[i]].astype(np.float32) + upd[i].astype(np.float32)).astype(npd)
    got = table_host(ct).view(npd).reshape(rows, dim)
    assert np.array_equal(got.view(np.uint8), want.view(np.uint8))
    ct.close()


def test_accumulate_rejects_other_value_types():
    rows, dim = 100, 8
    ct = CachedTable(np.zeros((rows, dim * 4), np.uint8), 64 * 1024, 8)
    keys = to_dev(np.arange(4, dtype=np.int64))
    upd = to_dev(np.zeros(4 * dim * 4, np.uint8))
    with pytest.raises(_lib.NVEError, match="Unsupported update type"):
        _lib.call("nve_table_update_accumulate", ct.table, ct.ctx, 4, vp(keys), dim * 4, dim * 4, vp(upd),
                  _lib.DT_F16)
    with pytest.raises(_lib.NVEError, match="size mismatch"):
        _lib.call("nve_table_update_accumulate", ct.table, ct.ctx, 4, vp(keys), dim * 4, dim * 2, vp(upd),
                  _lib.DT_F32)
    ct.close()


@pytest.mark.parametrize("dtype", [O.F32, O.F16])
def test_gpu_layer_update_and_accumulate(dtype):
    rng = np.random.default_rng(50 + dtype)
    rows, dim = 3000, 48
    npdt = np.float32 if dtype == O.F32 else np.float16
    ddt = _lib.DT_F32 if dtype == O.F32 else _lib.DT_F16
    es = 4 if dtype == O.F32 else 2
    tb = dyadic(rng, (rows, dim)).astype(npdt)
    lay = GpuLayer(tb.view(np.uint8).reshape(rows, dim * es), ddt)
    # update: in-range keys take the new rows, others are ignored
    keys = np.concatenate([rng.choice(rows, size=200, replace=False), [rows, -5]]).astype(np.int64)
    vals = dyadic(rng, (keys.size, dim)).astype(npdt)
    d_keys, d_vals = to_dev(keys), to_dev(vals.view(np.uint8).reshape(-1))
    _lib.call("nve_layer_update", lay.layer, lay.ctx, keys.size, vp(d_keys), dim * es, dim * es, vp(d_vals), 0)
    exp = tb.astype(np.float64)
    for i, k in enumerate(keys):
        if 0 <= k < rows:
            exp[k] = vals[i]
    got = lay.d_table.cpu().numpy().view(npdt).reshape(rows, dim)
    assert np.array_equal(got, exp.astype(npdt))
    # accumulate with repeated keys
    akeys = np.concatenate([keys[:100], keys[:30], keys[:3], [rows + 1]]).astype(np.int64)
    upd = dyadic(rng, (akeys.size, dim)).astype(npdt)
    d_ak, d_upd = to_dev(akeys), to_dev(upd.view(np.uint8).reshape(-1))
    _lib.call("nve_layer_accumulate", lay.layer, lay.ctx, akeys.size, vp(d_ak), dim * es, dim * es,
              vp(d_upd), ddt, 0)
    for i, k in enumerate(akeys):
        if 0 <= k < rows:
            exp[k] += upd[i].astype(np.float64)
    got = lay.d_table.cpu().numpy().view(npdt).reshape(rows, dim)
    assert np.array_equal(got, exp.astype(npdt))
    # lookups see the new rows
    out = torch.zeros((rows, dim * es), dtype=torch.uint8, device="cuda")
    all_keys = to_dev(np.arange(rows, dtype=np.int64))
    lay.lookup(all_keys, rows, out, dim * es)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(npdt), exp.astype(npdt))
    # insert / clear / erase have no effect on a linear table (gpu_embedding_layer.cu:500-650)
    _lib.call("nve_layer_insert", lay.layer, lay.ctx, keys.size, vp(d_keys), dim * es, dim * es, vp(d_vals), 0)
    _lib.call("nve_layer_clear", lay.layer, lay.ctx)
    _lib.call("nve_layer_erase", lay.layer, lay.ctx, keys.size, vp(d_keys), 0)
    assert np.array_equal(lay.d_table.cpu().numpy().view(npdt).reshape(rows, dim), exp.astype(npdt))
    # wrong value type / size
    with pytest.raises(_lib.InvalidArgument):
        _lib.call("nve_layer_accumulate", lay.layer, lay.ctx, akeys.size, vp(d_ak), dim * es, dim * es,
                  vp(d_upd), _lib.DT_F32 if dtype == O.F16 else _lib.DT_F16, 0)
    with pytest.raises(_lib.InvalidArgument):
        _lib.call("nve_layer_update", lay.layer, lay.ctx, keys.size, vp(d_keys), dim * es, dim * es - 2,
                  vp(d_vals), 0)
    lay.close()


def test_gpu_layer_accumulate_rejects_quantized_tables():
    rng = np.random.default_rng(55)
    from nve_helpers import quant_table
    tb = quant_table(rng, 100, 32, O.QI8_F32)
    lay = GpuLayer(tb, _lib.DT_QI8_F32)
    keys = to_dev(np.arange(4, dtype=np.int64))
    upd = to_dev(np.zeros(4 * tb.shape[1], np.uint8))
    with pytest.raises(_lib.NVEError, match="quantized"):
        _lib.call("nve_layer_accumulate", lay.layer, lay.ctx, 4, vp(keys), tb.shape[1], tb.shape[1], vp(upd),
                  _lib.DT_QI8_F32, 0)
    lay.close()


@pytest.mark.parametrize("device_policy", [True, False])
@pytest.mark.parametrize("accumulate", [False, True])
def test_update_reaches_every_way_whose_rebuilt_key_matches(accumulate, device_policy):
    """An empty way's tag rebuilds to the key sentinel * num_sets + set (in
    unsigned 64-bit arithmetic), and when num_sets divides 2^64 that key falls
    in the same set: it then matches all eight empty ways of the set.  The
    device policy's SetUpdateDataKernel records every matching way with the
    key's own tag, key / num_sets (ec_set_associative_modify.cuh:541-561), and
    tag_update_kernel commits it (ec_set_associative.cuh:252-261): the eight
    ways then hold 2^57 - 1 (128 sets), no longer the sentinel, and each gets
    the row (or the sum).  The host policy records only the first matching way
    and commits its current tag (ec_set_associative_host_modify.h:489-512): one
    way gets the row, every tag stays.  An ordinary resident key is updated
    beside it either way."""
    rng = np.random.default_rng(77 + int(accumulate) + 2 * int(device_policy))
    rows, dim = 2000, 16
    uvm = float_table(rng, rows, dim, O.F32)
    per_set = 8 * 8 + 8 * dim * 4 + (8 * 4 if device_policy else 0)  # tags, rows, counters
    ct = CachedTable(uvm, 128 * per_set, 8, modify_on_gpu=device_policy)
    assert ct.num_sets == 128
    ct.model.insert_keys(np.array([11], np.int64), uvm=ct.uvm_np.reshape(-1))
    ct.load_model()
    s = 5 if ct.model.set_of(11) != 5 else 6
    odd = s - ct.num_sets  # rebuilt key of every empty way of set s
    # accumulate: the odd key twice (both add to every matching way); update:
    # once (two rows copied to one way at once may interleave)
    keys = np.array([odd, 11, odd] if accumulate else [odd, 11], np.int64)
    upd = dyadic(rng, (keys.size, dim)).astype(np.float32)
    tags0, _, _, rows0 = cache_state(ct)
    ways0 = slots_of(tags0, ct.num_sets, odd)
    assert ways0 == [s * 8 + w for w in range(8)]
    d_keys, d_upd = to_dev(keys), to_dev(upd.view(np.uint8).reshape(-1))
    if accumulate:
        _lib.call("nve_table_update_accumulate", ct.table, ct.ctx, keys.size, vp(d_keys), dim * 4, dim * 4,
                  vp(d_upd), _lib.DT_F32)
    else:
        _lib.call("nve_table_update", ct.table, ct.ctx, keys.size, vp(d_keys), dim * 4, dim * 4, vp(d_upd))
    torch.cuda.synchronize()
    tags1, _, _, rows1 = cache_state(ct)
    own_tag = (odd % (1 << 64)) // ct.num_sets
    assert own_tag == (1 << 57) - 1
    exp_tags = tags0.copy()
    written = ways0 if device_policy else ways0[:1]
    if device_policy:
        exp_tags[ways0] = own_tag
    assert np.array_equal(tags1, exp_tags)
    # the committed tags still rebuild to the odd key
    assert slots_of(tags1, ct.num_sets, odd) == ways0
    sl11 = slot_of(tags1, ct.num_sets, 11)
    assert sl11 not in ways0
    r11 = rows1[sl11].view(np.float32)
    if accumulate:
        assert np.array_equal(r11, rows0[sl11].view(np.float32) + upd[1])
        for w in written:  # both occurrences of the odd key add to every recorded way
            assert np.array_equal(rows1[w].view(np.float32), rows0[w].view(np.float32) + upd[0] + upd[2])
    else:
        assert np.array_equal(r11, upd[1])
        for w in written:
            assert np.array_equal(rows1[w].view(np.float32), upd[0])
    for w in ways0:
        if w not in written:
            assert np.array_equal(rows1[w], rows0[w])
    ct.close()

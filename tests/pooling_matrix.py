"""The layer pooling capability matrix: every layer x pooling x sparse layout x
stored dtype x output dtype x weight dtype x key type, sorted into cases that
must match the reference reduction and cases the layer must refuse.

This restates the classification of the reference's capability suite
(tests/layer_pooling/layer_pooling_harness.hpp:131-190, case generation
:269-329, fixed sizes :271-274) for the three layers of this build (GPU,
LinearUVM, Host; the hierarchical layers are out of scope).  Its totals are
the ones the reference's README states per layer
(tests/layer_pooling/README.md "Support matrix": GPU 152 enabled + 112
rejected, LinearUVM 168 + 112, Host 336 + 0), which the CPU suite checks.

Each enabled case is held to two references: the oracle (bit for bit: the
same reduction order as the product's kernels, or the HostLayer's CPU order)
and an independent float64 reduction of the same rows, within the path's
pooling tolerance (1e-5 relative to the bag's magnitude for fp32 output; that
plus one fp16 ulp for fp16 output)."""
import itertools

import numpy as np

from nve_helpers import quant_table
from oracle import oracle as O

GPU, UVM, HOST = "GPU", "LinearUVM", "Host"
LAYERS = (GPU, UVM, HOST)
POOLS = (O.CONCAT, O.SUM, O.MEAN, O.WSUM, O.WMEAN)
POOL_NAME = {O.CONCAT: "Concat", O.SUM: "Sum", O.MEAN: "Mean", O.WSUM: "WSum", O.WMEAN: "WMean"}
SPARSES = (O.FIXED, O.CSR)
INS = (O.F32, O.F16, O.QI8_F32, O.QI8_F16, O.QU8_F32, O.QU8_F16)
OUTS = (O.F32, O.F16)
DT_NAME = {O.F32: "F32", O.F16: "F16", O.QI8_F32: "QI8F32", O.QI8_F16: "QI8F16", O.QU8_F32: "QU8F32",
           O.QU8_F16: "QU8F16"}
QUANT = (O.QI8_F32, O.QI8_F16, O.QU8_F32, O.QU8_F16)

# fixed sizes of the reference's suite (layer_pooling_harness.hpp:271-274)
VALUE_COUNT, HOTNESS, NUM_KEYS, NUM_ROWS = 64, 8, 1 << 10, 1 << 16
# the reference README's per-layer totals (enabled, rejected)
REFERENCE_TOTALS = {GPU: (152, 112), UVM: (168, 112), HOST: (336, 0)}


def weighted(pool):
    return pool in (O.WSUM, O.WMEAN)


def classify(layer, pool, sparse, din, dout, wdt):
    """'enabled', 'rejected' or None (not generated); layer_pooling_harness.hpp:131-190."""
    quant = din in QUANT
    if not quant and dout != din and layer != HOST:
        return None  # the GPU kernels have no float -> float cast
    if layer == GPU:
        if quant:
            return "enabled" if dout == O.native_out(din) else "rejected"
        if weighted(pool) and wdt != din:
            return None  # the GPU layer's weights have the table's type
        return "enabled"
    if layer == UVM:
        if quant and dout != O.native_out(din):
            return "rejected"
        return "enabled"
    return "enabled"


def cases():
    """(label, case) for every generated case, in the reference's loop order."""
    out = []
    for layer, pool, sparse, din, dout, k64 in itertools.product(LAYERS, POOLS, SPARSES, INS, OUTS,
                                                                  (True, False)):
        for wdt in ((O.F32, O.F16) if weighted(pool) else (0,)):
            status = classify(layer, pool, sparse, din, dout, wdt)
            if status is None:
                continue
            label = (f"{layer}_{POOL_NAME[pool]}_{'Fixed' if sparse == O.FIXED else 'CSR'}_in{DT_NAME[din]}"
                     f"_out{DT_NAME[dout]}_k{64 if k64 else 32}" + (f"_w{DT_NAME[wdt]}" if wdt else ""))
            out.append((label, dict(layer=layer, pool=pool, sparse=sparse, din=din, dout=dout, k64=k64,
                                    wdt=wdt, status=status)))
    return out


# ---------------------------------------------------------------------------
# data: one table per stored dtype, keys, offsets and weights per case
# ---------------------------------------------------------------------------
_TABLES = {}


def table(din):
    """(NUM_ROWS, row_bytes) uint8 stored rows of dtype din (seeded per dtype)."""
    if din not in _TABLES:
        rng = np.random.default_rng(9000 + din)
        if din in QUANT:
            _TABLES[din] = quant_table(rng, NUM_ROWS, VALUE_COUNT, din)
        else:
            v = rng.normal(0.0, 0.5, size=(NUM_ROWS, VALUE_COUNT))
            _TABLES[din] = (v.astype(np.float32) if din == O.F32 else v.astype(np.float16)).view(np.uint8)
    return _TABLES[din]


def inputs(case, seed):
    """keys, offsets (None for Fixed), bags, weights (None unless weighted)."""
    rng = np.random.default_rng(seed)
    kdt = np.int64 if case["k64"] else np.int32
    keys = rng.integers(0, NUM_ROWS, size=NUM_KEYS).astype(kdt)
    off = None
    bags = NUM_KEYS
    if case["pool"] != O.CONCAT:
        if case["sparse"] == O.CSR:
            # 128 bags over the 1024 keys at random cut points: empty and long bags
            cuts = np.sort(rng.integers(0, NUM_KEYS + 1, size=NUM_KEYS // HOTNESS - 1))
            off = np.concatenate([[0], cuts, [NUM_KEYS]]).astype(kdt)
            bags = off.size - 1
        else:
            bags = NUM_KEYS // HOTNESS
    w = None
    if weighted(case["pool"]):
        w = rng.uniform(0.0, 1.0, size=NUM_KEYS)
        w = w.astype(np.float32) if case["wdt"] == O.F32 else w.astype(np.float16)
    return keys, off, bags, w


def out_array(case, bags):
    """Zeroed host output of the case's layout (rows x values of the output dtype)."""
    return np.zeros((bags, VALUE_COUNT), np.float32 if case["dout"] == O.F32 else np.uint16)


# ---------------------------------------------------------------------------
# references
# ---------------------------------------------------------------------------
def values64(rows_bytes, din, count=VALUE_COUNT):
    """Stored rows -> (n, count) float64 values (dequantized for quant rows)."""
    rows_bytes = np.ascontiguousarray(rows_bytes)
    n = rows_bytes.shape[0]
    if din == O.F32:
        return rows_bytes.view(np.float32).reshape(n, count).astype(np.float64)
    if din == O.F16:
        return rows_bytes.view(np.float16).reshape(n, count).astype(np.float64)
    q = np.ascontiguousarray(rows_bytes[:, :count])
    q = (q.view(np.int8) if din in (O.QI8_F32, O.QI8_F16) else q).astype(np.float64)
    meta = np.ascontiguousarray(rows_bytes[:, count:])
    mt = np.float32 if din in (O.QI8_F32, O.QU8_F32) else np.float16
    m = meta.view(mt).astype(np.float64)
    v = q * m[:, :1]
    if din in (O.QU8_F32, O.QU8_F16):
        v = v + m[:, 1:2]
    return v


def reduce64(case, keys, off, bags, w):
    """Float64 reduction of the case and the magnitude each output element is
    compared against: (ref, mag)."""
    v = values64(table(case["din"])[keys.astype(np.int64)], case["din"])
    pool = case["pool"]
    if pool == O.CONCAT:
        return v, np.abs(v)
    if off is None:
        off = np.arange(0, NUM_KEYS + 1, HOTNESS)
    off = off.astype(np.int64)
    ww = np.ones(NUM_KEYS) if w is None else w.astype(np.float64)
    ref = np.zeros((bags, VALUE_COUNT))
    mag = np.zeros((bags, VALUE_COUNT))
    for b in range(bags):
        s, e = off[b], off[b + 1]
        if e == s:
            continue
        terms = v[s:e] * ww[s:e, None]
        acc, a = terms.sum(axis=0), np.abs(terms).sum(axis=0)
        if pool == O.MEAN:
            acc, a = acc / (e - s), a / (e - s)
        elif pool == O.WMEAN:
            den = ww[s:e].sum()
            if den == 0:
                continue
            acc, a = acc / den, a / abs(den)
        ref[b], mag[b] = acc, a
    return ref, mag


def assert_close64(case, got, ref, mag):
    """Within 1e-5 of the magnitude (fp32 accumulation), plus one fp16 ulp of
    the result for fp16 output.  Rows whose scale is fp16 are dequantized in
    fp32 and rounded to fp16 value by value before they are pooled (the F16
    variants of the reference's dequantize, kernels_common.cuh:174-297), so
    for them each term may also be off by half an fp16 ulp: 2^-11 of the
    magnitude."""
    term = 2.0 ** -11 if case["din"] in (O.QI8_F16, O.QU8_F16) else 0.0
    if case["dout"] == O.F32:
        g = got.astype(np.float64)
        tol = (1e-5 + term) * mag + 1e-30
    else:
        g = got.view(np.float16).astype(np.float64)
        r16 = np.abs(ref).astype(np.float16)
        ulp = np.spacing(np.maximum(r16, np.float16(6.1e-5))).astype(np.float64)
        tol = ulp + (1e-5 + term) * mag
    bad = np.abs(g - ref) > tol
    assert not bad.any(), (f"{int(bad.sum())} elements off, first at {np.argwhere(bad)[0]}: "
                           f"{g[bad][0]} vs {ref[bad][0]}")


def oracle_out(case, keys, off, bags, w, host_order):
    """The oracle's result for the case, in the output array's dtype."""
    tb = table(case["din"])
    pool = case["pool"]
    dout = case["dout"]
    if pool == O.CONCAT:
        if case["din"] == dout:
            return np.ascontiguousarray(tb[keys.astype(np.int64)]).view(out_array(case, 1).dtype)
        if host_order:
            return O.convert_rows_host(tb[keys.astype(np.int64)], case["din"], VALUE_COUNT, dout)
        return O.dequant_rows(tb[keys.astype(np.int64)], case["din"], VALUE_COUNT, dout)
    flat = np.ascontiguousarray(tb).reshape(-1)
    ptrs = O.linear_row_ptrs(keys, flat, tb.shape[1])
    wv = None if w is None else (w.view(np.uint16) if w.dtype == np.float16 else w)
    return O.pool(ptrs, case["din"], VALUE_COUNT, case["sparse"], pool, NUM_KEYS, off, bags,
                  0 if off is not None else HOTNESS, wv, case["wdt"] if w is not None else 0, dout,
                  host_order=host_order, key_bytes=8 if case["k64"] else 4)

"""GPU parity of the dequantizing gather of one-byte row formats (int8 / uint8
/ fp8 values followed by their scale and offset: rows of count + 2..8 bytes,
not 16-byte aligned), the path of find_and_dequant.cuh:41-123 restated over
aligned 16-byte loads realigned across lanes.

Every format and value count 16..256 (1..16 lanes per row), table bases
shifted off 16-byte alignment so that rows start at every offset their
alignment allows, keys outside the table (nothing is written for them), and
layouts the realigned path does not take (metadata wider than the row
alignment, value counts that are not a power of two times 16), all compared
bit for bit with the oracle's dequantization."""
import numpy as np
import pytest

from nve_helpers import oracle_dequant, quant_table, stream_ptr, to_dev, vp
from oracle import oracle as O
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

FORMATS = [(O.QI8_F32, _lib.DT_QI8_F32), (O.QI8_F16, _lib.DT_QI8_F16), (O.QU8_F32, _lib.DT_QU8_F32),
           (O.QU8_F16, _lib.DT_QU8_F16), (O.XI8A_F32, _lib.DT_XI8A_F32),
           (O.XE4M3_F32, _lib.DT_XE4M3_F32)]
ODT = {O.F32: _lib.DT_F32, O.F16: _lib.DT_F16}
SENTINEL = 0xA5


def outputs(odt):
    """The reference's formats dequantize to their metadata precision; the
    two extension formats to fp32 or fp16."""
    return (O.F32, O.F16) if odt in (O.XI8A_F32, O.XE4M3_F32) else (O.native_out(odt),)


CASES = [(f, o) for f in FORMATS for o in outputs(f[0])]


def gather(table_bytes, row_bytes, rows, keys, vdt, count, out_dtype, base_shift=0):
    """nve_amd_find_and_pool Concatenate over `rows` rows of `row_bytes` that
    start `base_shift` bytes into a device buffer; returns the output bytes."""
    flat = np.zeros(base_shift + table_bytes.size + 64, np.uint8)
    flat[base_shift:base_shift + table_bytes.size] = table_bytes.reshape(-1)
    d_flat = to_dev(flat)
    oes = 2 if out_dtype == O.F16 else 4
    n = keys.size
    out = torch.full((max(n, 1), count * oes), SENTINEL, dtype=torch.uint8, device="cuda")
    d_keys = to_dev(keys.astype(np.int64))
    _lib.call("nve_amd_find_and_pool", _lib.KEY_INT64, n, vp(d_keys), d_flat.data_ptr() + base_shift, rows,
              row_bytes, vdt, _lib.POOL_CONCAT, 0, None, 0, 0, None, 0, ODT[out_dtype], vp(out), count * oes,
              0, 0, stream_ptr())
    torch.cuda.synchronize()
    return out.cpu().numpy()[:n]


def check(table, keys, odt, count, out_dtype, got):
    bits = np.uint16 if out_dtype == O.F16 else np.uint32
    inside = (keys >= 0) & (keys < table.shape[0])
    ref = oracle_dequant(table, keys[inside], odt, count, out_dtype)
    assert np.array_equal(got[inside].view(bits).reshape(-1, count), ref.view(bits).reshape(-1, count))
    assert np.all(got[~inside] == SENTINEL)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0][0]}-{c[1]}")
@pytest.mark.parametrize("count", [16, 32, 64, 128, 256])
def test_every_format_and_group_width(case, count):
    (odt, vdt), out_dtype = case
    rng = np.random.default_rng(1000 * odt + count + out_dtype)
    rows = 1500
    table = quant_table(rng, rows, count, odt)
    # a batch that is not a multiple of a wave's keys, with keys past the table
    keys = rng.integers(0, rows, size=1234).astype(np.int64)
    keys[rng.integers(0, keys.size, size=40)] = rows + 7
    got = gather(table, table.shape[1], rows, keys, vdt, count, out_dtype)
    check(table, keys, odt, count, out_dtype, got)


@pytest.mark.parametrize("fmt", FORMATS, ids=lambda f: str(f[0]))
@pytest.mark.parametrize("shift", [2, 4, 8, 12])
def test_table_base_off_alignment(fmt, shift):
    """Rows starting at every offset mod 16 the format's alignment allows; a
    shift finer than the metadata's width takes the general gather."""
    odt, vdt = fmt
    rng = np.random.default_rng(77 + 10 * odt + shift)
    rows, count = 900, 256
    table = quant_table(rng, rows, count, odt)
    keys = rng.integers(0, rows, size=700).astype(np.int64)
    for out_dtype in outputs(odt):
        got = gather(table, table.shape[1], rows, keys, vdt, count, out_dtype, base_shift=shift)
        check(table, keys, odt, count, out_dtype, got)


@pytest.mark.parametrize("fmt", FORMATS, ids=lambda f: str(f[0]))
def test_layouts_outside_the_realigned_path(fmt):
    """Padded rows (row stride 2 bytes past the metadata, so 2-byte aligned)
    and a value count of 48: the general gather, same results."""
    odt, vdt = fmt
    rng = np.random.default_rng(5 + odt)
    rows = 600
    for count, pad in ((256, 2), (48, 0)):
        q = quant_table(rng, rows, count, odt)
        table = np.zeros((rows, q.shape[1] + pad), np.uint8)
        table[:, :q.shape[1]] = q
        keys = rng.integers(0, rows, size=333).astype(np.int64)
        out_dtype = outputs(odt)[0]
        got = gather(table, table.shape[1], rows, keys, vdt, count, out_dtype)
        check(q, keys, odt, count, out_dtype, got)


def test_f16_output_rounds_through_binary32():
    """q = 1, scale = 2^-40, offset = 1 + 2^-11: fma(q, scale, offset) rounds
    to 1 + 2^-11 in binary32, a tie in binary16 that rounds to even, 1.0.  A
    single rounding of the exact value straight to binary16 gives 1 + 2^-10."""
    odt, vdt = O.XI8A_F32, _lib.DT_XI8A_F32
    count, rows = 256, 64
    table = np.zeros((rows, count + 8), np.uint8)
    table[:, :count] = 1
    table[:, count:count + 4] = np.float32(2.0 ** -40).reshape(1).view(np.uint8)
    table[:, count + 4:count + 8] = np.float32(1 + 2.0 ** -11).reshape(1).view(np.uint8)
    keys = np.arange(rows, dtype=np.int64)
    got = gather(table, table.shape[1], rows, keys, vdt, count, O.F16).view(np.float16)
    assert np.all(got == np.float16(1.0))
    check(table, keys, odt, count, O.F16, gather(table, table.shape[1], rows, keys, vdt, count, O.F16))


def test_empty_batch_writes_nothing():
    rng = np.random.default_rng(9)
    table = quant_table(rng, 10, 256, O.XI8A_F32)
    got = gather(table, table.shape[1], 10, np.zeros(0, np.int64), _lib.DT_XI8A_F32, 256, O.F16)
    assert got.shape[0] == 0

"""CPU checks of the .nve table container (pynve.nve.TensorFileFormat), the
format of the reference's src/serialization.cpp:234-300 and
include/serialization.hpp:100-140.

The expected bytes are written out by hand from the format's definition
(little-endian u32 magic 0x4E564500, version 0.2; 32-byte records {key1 =
cols | esize << 16 | rows << 20, name, next-record offset, length}), so a
wrong field order, shift or offset base fails here.  The search cases follow
load_tensor_from_stream: walk records by their offsets, stop silently at the
end, raise on a short record, a size mismatch or a wrong header."""
import io
import struct

import pytest

from pynve import _lib, nve  # noqa: E402

HEADER = bytes.fromhex("0045564e" "00000000" "02000000")


def _fmt():
    return nve.TensorFileFormat()


def test_header_bytes_and_verify():
    f = io.BytesIO()
    _fmt().write_table_file_header(f)
    assert f.getvalue() == HEADER
    assert _fmt().verify_table_header(f)
    assert f.tell() == 12
    for bad in (b"\x01" + HEADER[1:], HEADER[:4] + b"\x01\0\0\0" + HEADER[8:],
                HEADER[:8] + b"\x03\0\0\0", HEADER[:7]):
        assert not _fmt().verify_table_header(io.BytesIO(bad))


def test_header_is_written_at_offset_zero():
    f = io.BytesIO(b"x" * 40)
    f.seek(25)
    _fmt().write_table_file_header(f)
    assert f.getvalue()[:12] == HEADER and f.getvalue()[12:] == b"x" * 28


def test_entry_bytes_closed_form():
    f = io.BytesIO()
    _fmt().write_table_file_header(f)
    data = bytes(range(24))  # 3 rows x 4 cols x 2-byte elements
    _fmt().write_tensor_to_stream(f, 7, 3, 4, 2, [data[:10], data[10:]])
    raw = f.getvalue()
    assert len(raw) == 12 + 32 + 24
    # key1 = 4 | 2 << 16 | 3 << 20 = 0x00320004; next record at 12 + 32 + 24 = 68
    assert raw[12:44] == bytes.fromhex("0400320000000000" "0700000000000000"
                                       "4400000000000000" "1800000000000000")
    assert raw[44:] == data


def test_key_packing_limits():
    k = _fmt().make_key((1 << 44) - 1, (1 << 16) - 1, 15)
    assert k == (1 << 64) - 1
    assert _fmt().make_key(5, 128, 4) == 128 | (4 << 16) | (5 << 20)
    with pytest.raises(_lib.NVEError, match="16 bit row size"):
        _fmt().make_key(1, 1 << 16, 2)
    with pytest.raises(_lib.NVEError, match="44 bit rows"):
        _fmt().make_key(1 << 44, 1, 2)
    with pytest.raises(_lib.NVEError, match="data type"):
        _fmt().make_key(1, 1, 16)


def _file(entries):
    f = io.BytesIO()
    _fmt().write_table_file_header(f)
    for name, rows, cols, esize, data in entries:
        _fmt().write_tensor_to_stream(f, name, rows, cols, esize, [data])
    return f


def test_find_walks_entries_by_offset():
    a, b, c = b"A" * 8, b"B" * 48, b"C" * 6
    f = _file([(1, 2, 2, 2, a), (2 ** 63 + 5, 4, 3, 4, b), (3, 3, 1, 2, c)])
    for name, geo, data in ((1, (2, 2, 2), a), (2 ** 63 + 5, (4, 3, 4), b), (3, (3, 1, 2), c)):
        found = _fmt().find_tensor(f, name, *geo)
        assert found is not None and found[1] == name and found[3] == len(data)
        assert f.read(len(data)) == data
        assert found[0] == _fmt().make_key(*geo)
    # the record offsets chain to the end of the file
    raw = f.getvalue()
    pos = 12
    while pos < len(raw):
        _, _, nxt, length = struct.unpack_from("<QQQQ", raw, pos)
        assert nxt == pos + 32 + length
        pos = nxt
    assert pos == len(raw)


def test_find_missing_name_returns_none():
    f = _file([(1, 1, 4, 2, b"x" * 8)])
    assert _fmt().find_tensor(f, 9, 1, 4, 2) is None
    assert _fmt().find_tensor(_file([]), 1, 1, 4, 2) is None


def test_find_errors():
    f = _file([(1, 1, 4, 2, b"x" * 8)])
    with pytest.raises(_lib.NVEError, match="Incorrect tensor size"):
        _fmt().find_tensor(f, 1, 2, 4, 2)
    with pytest.raises(_lib.NVEError, match="Incorrect file version"):
        _fmt().find_tensor(io.BytesIO(b"\0" * 64), 1, 1, 4, 2)
    raw = f.getvalue()
    with pytest.raises(_lib.NVEError, match="Problem reading table entry"):
        _fmt().find_tensor(io.BytesIO(raw[:12 + 20]), 1, 1, 4, 2)
    with pytest.raises(_lib.NVEError, match="Problem reading tensor"):
        _fmt().find_tensor(io.BytesIO(raw[:-1]), 1, 1, 4, 2)


def test_short_source_and_bad_name_raise():
    f = io.BytesIO()
    _fmt().write_table_file_header(f)
    with pytest.raises(_lib.NVEError, match="gave 4 of 8"):
        _fmt().write_tensor_to_stream(f, 1, 1, 4, 2, [b"1234"])
    with pytest.raises(_lib.InvalidArgument):
        _fmt().write_tensor_to_stream(f, -1, 1, 4, 2, [b"12345678"])


class _Trickle(io.RawIOBase):
    """A stream that moves at most 5 bytes per write / readinto call."""

    def __init__(self):
        self.buf = io.BytesIO()

    def writable(self):
        return True

    def readable(self):
        return True

    def seekable(self):
        return True

    def write(self, b):
        return self.buf.write(bytes(memoryview(b)[:5]))

    def readinto(self, b):
        d = self.buf.read(min(5, len(b)))
        memoryview(b)[:len(d)] = d
        return len(d)

    def seek(self, pos, whence=0):
        return self.buf.seek(pos, whence)

    def tell(self):
        return self.buf.tell()


def test_partial_writes_and_reads_are_completed():
    s = _Trickle()
    _fmt().write_table_file_header(s)
    data = bytes(range(48))
    _fmt().write_tensor_to_stream(s, 11, 2, 6, 4, [data])
    assert s.buf.getvalue() == _file([(11, 2, 6, 4, data)]).getvalue()
    assert _fmt().find_tensor(s, 11, 2, 6, 4) is not None
    out = bytearray(48)
    assert nve._PyStream(s).read_into(out) == 48 and bytes(out) == data


def test_layer_entry_points_reject_other_objects():
    with pytest.raises(TypeError):
        nve.write_tensor_to_stream(object(), io.BytesIO(), 1)
    with pytest.raises(TypeError):
        nve.load_tensor_from_stream(object(), io.BytesIO(), 1)

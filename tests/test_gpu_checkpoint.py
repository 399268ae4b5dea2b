"""GPU checks of table checkpoints in the .nve container: the layer entry
points nve.write_tensor_to_stream / nve.load_tensor_from_stream
(python_binding.cu:83-105, binding_layers.hpp:626-636 and 693-716) and
NVEmbeddingBase.load_from_stream (nve_layers.py:400-401), as the reference's
export path uses them (nve_export.py:270-272 writes, :534 loads).

Round trips are bit-exact: a table written by one layer and loaded into a
fresh layer of the same geometry holds the same bytes and serves the same
lookups; the file's bytes equal the header plus one record plus the table's
bytes; entries of several layers share one file and load by name."""
import io
import struct

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from pynve import _lib, nve  # noqa: E402
from pynve.torch import nve_layers  # noqa: E402

LT = nve_layers.LayerType
CACHE = 16 * 1024 * 1024


def make(layer_type, weight, *, id, bag=False):
    n, d = weight.shape
    kw = dict(weight_init=weight, optimize_for_training=False, id=id)
    if layer_type == LT.LinearUVM:
        kw["gpu_cache_size"] = CACHE
    if bag:
        return nve_layers.NVEmbeddingBag(n, d, weight.dtype, layer_type, "sum", **kw)
    return nve_layers.NVEmbedding(n, d, weight.dtype, layer_type, **kw)


def table(layer):
    return layer.weight.detach()


def rand_table(n, d, dtype, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(n, d, generator=g, dtype=torch.float32).to(dtype).cuda()


def save(*layers):
    f = io.BytesIO()
    nve.TensorFileFormat().write_table_file_header(f)
    for layer in layers:
        nve.write_tensor_to_stream(layer.emb_layer, f, layer.id)
    return f


@pytest.mark.parametrize("src_type", [LT.GPULayer, LT.LinearUVM], ids=["from_gpu", "from_uvm"])
@pytest.mark.parametrize("dst_type", [LT.GPULayer, LT.LinearUVM], ids=["to_gpu", "to_uvm"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_round_trip_bitwise(src_type, dst_type, dtype):
    n, d = 5000, 32
    src = make(src_type, rand_table(n, d, dtype, 1), id=77)
    f = save(src)
    esize = 4 if dtype == torch.float32 else 2
    raw = f.getvalue()
    assert raw[:12] == bytes.fromhex("0045564e0000000002000000")
    key1, name, nxt, length = struct.unpack_from("<QQQQ", raw, 12)
    assert (key1, name, nxt, length) == (d | esize << 16 | n << 20, 77, 44 + n * d * esize,
                                         n * d * esize)
    assert raw[44:] == table(src).cpu().contiguous().view(torch.uint8).numpy().tobytes()

    dst = make(dst_type, rand_table(n, d, dtype, 2), id=77)
    f.seek(0)
    dst.load_from_stream(f)
    torch.cuda.synchronize()
    assert torch.equal(table(dst).cpu(), table(src).cpu())
    keys = torch.randint(0, n, (4096,), dtype=torch.int64, device="cuda")
    with torch.no_grad():
        assert torch.equal(dst(keys), src(keys))


def test_several_layers_in_one_file_load_by_name():
    dtype = torch.float16
    a = make(LT.GPULayer, rand_table(3000, 64, dtype, 3), id=1)
    b = make(LT.LinearUVM, rand_table(2000, 16, dtype, 4), id=2 ** 62 + 9)
    c = make(LT.GPULayer, rand_table(100, 128, dtype, 5), id=3, bag=True)
    f = save(a, b, c)
    for src, seed in ((c, 6), (a, 7), (b, 8)):  # out of file order
        n, d = table(src).shape
        lt = LT.LinearUVM if src is b else LT.GPULayer
        dst = make(lt, rand_table(n, d, dtype, seed), id=src.id, bag=src is c)
        dst.load_from_stream(f)
        torch.cuda.synchronize()
        assert torch.equal(table(dst).cpu(), table(src).cpu())


def test_staged_copy_over_several_chunks():
    # 300000 x 64 fp32 = 76.8 MB: two 64 MiB staging passes each way
    n, d = 300000, 64
    src = make(LT.GPULayer, rand_table(n, d, torch.float32, 9), id=5)
    f = save(src)
    dst = make(LT.GPULayer, torch.zeros(n, d, dtype=torch.float32, device="cuda"), id=5)
    f.seek(0)
    dst.load_from_stream(f)
    torch.cuda.synchronize()
    assert torch.equal(table(dst), table(src))


def test_write_sees_pending_device_updates():
    n, d = 1000, 16
    src = make(LT.GPULayer, rand_table(n, d, torch.float16, 10), id=6)
    keys = torch.arange(0, n, 7, dtype=torch.int64, device="cuda")
    vals = torch.full((keys.numel(), d), 3.0, dtype=torch.float16, device="cuda")
    src.update(keys, vals)  # queued on the current stream, not waited for
    f = save(src)
    expect = table(src).cpu()
    assert torch.all(expect[keys.cpu()] == 3.0)
    assert f.getvalue()[44:] == expect.contiguous().view(torch.uint8).numpy().tobytes()


def test_missing_name_and_errors():
    dtype = torch.float16
    src = make(LT.GPULayer, rand_table(500, 8, dtype, 11), id=10)
    f = save(src)
    # a GPU layer is zero-filled when the name is absent (the reference copies
    # its zero-initialised staging buffer); a LinearUVM table is left as it was
    g = make(LT.GPULayer, rand_table(500, 8, dtype, 12), id=11)
    g.load_from_stream(f)
    torch.cuda.synchronize()
    assert torch.count_nonzero(table(g)) == 0
    w = rand_table(500, 8, dtype, 13)
    u = make(LT.LinearUVM, w, id=11)
    u.load_from_stream(f)
    assert torch.equal(table(u).cpu(), w.cpu())
    # same name, other size
    wrong = make(LT.GPULayer, rand_table(400, 8, dtype, 14), id=10)
    with pytest.raises(_lib.NVEError, match="Incorrect tensor size"):
        wrong.load_from_stream(f)
    # truncated data: the error comes before the table is touched
    keep = rand_table(500, 8, dtype, 15)
    t = make(LT.GPULayer, keep, id=10)
    with pytest.raises(_lib.NVEError, match="Problem reading tensor"):
        t.load_from_stream(io.BytesIO(f.getvalue()[:-2]))
    assert torch.equal(table(t), keep)
    with pytest.raises(_lib.NVEError, match="Incorrect file version"):
        t.load_from_stream(io.BytesIO(b"\0" * 64))


def test_file_on_disk(tmp_path):
    src = make(LT.LinearUVM, rand_table(2048, 32, torch.float32, 16), id=21)
    p = tmp_path / "embeddings.nve"
    with open(p, "wb") as fh:
        nve.TensorFileFormat().write_table_file_header(fh)
        nve.write_tensor_to_stream(src.emb_layer, fh, src.id)
    assert p.stat().st_size == 12 + 32 + 2048 * 32 * 4
    dst = make(LT.LinearUVM, torch.zeros(2048, 32, dtype=torch.float32, device="cuda"), id=21)
    with open(p, "rb") as fh:
        dst.load_from_stream(fh)
    assert torch.equal(table(dst).cpu(), table(src).cpu())

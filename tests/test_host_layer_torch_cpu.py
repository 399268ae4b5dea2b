"""The torch surface of the host layer on the CPU (no GPU):
NVEmbedding / NVEmbeddingBag with LayerType.HostLayer and device='cpu',
through the ops' CPU dispatch.  Compared with torch.nn.Embedding /
torch.nn.EmbeddingBag (the reference's tests/python_binding/
test_host_cpu.py:288-315 holds the same comparison to 1e-6) and bit for bit
with the oracle's CPU HostLayer order."""
import io

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle import oracle as O  # noqa: E402
from pynve import nve  # noqa: E402
from pynve.torch import nve_layers  # noqa: E402

LT = nve_layers.LayerType


def make_bag(rows, dim, dtype, mode, init, **kw):
    return nve_layers.NVEmbeddingBag(rows, dim, dtype, LT.HostLayer, mode, weight_init=init,
                                     optimize_for_training=False, device="cpu", **kw)


@pytest.mark.parametrize("mode", ["sum", "mean"])
@pytest.mark.parametrize("weighted", [False, True])
def test_embedding_bag_matches_torch(mode, weighted):
    g = torch.Generator().manual_seed(3)
    rows, dim, bags = 1000, 32, 64
    init = torch.randn(rows, dim, generator=g)
    lens = torch.randint(1, 12, (bags,), generator=g)
    off = torch.zeros(bags + 1, dtype=torch.int64)
    off[1:] = torch.cumsum(lens, 0)
    keys = torch.randint(0, rows, (int(off[-1]),), generator=g)
    w = torch.rand(keys.numel(), generator=g) if weighted else None
    layer = make_bag(rows, dim, torch.float32, mode, init)
    got = layer(keys, off, w)
    ref_mod = torch.nn.EmbeddingBag(rows, dim, mode=mode, include_last_offset=True, _weight=init)
    want = ref_mod(keys, off, per_sample_weights=w if weighted and mode == "sum" else None)
    if weighted and mode == "mean":  # EmbeddingBag has no weighted mean: sum(w x) / sum(w)
        s = torch.nn.functional.embedding_bag(keys, init, off, mode="sum", per_sample_weights=w,
                                              include_last_offset=True)
        den = torch.stack([w[off[b]:off[b + 1]].sum() for b in range(bags)])
        want = s / den[:, None]
    assert got.dtype == torch.float32 and got.shape == (bags, dim)
    assert torch.allclose(got, want.detach(), rtol=1e-6, atol=1e-6)
    # and bit for bit with the CPU HostLayer order
    tb = init.numpy().view(np.uint8).reshape(-1)
    pool = {("sum", False): O.SUM, ("mean", False): O.MEAN, ("sum", True): O.WSUM, ("mean", True): O.WMEAN}
    ref = O.pool(O.linear_row_ptrs(keys.numpy(), tb, dim * 4), O.F32, dim, O.CSR, pool[(mode, weighted)],
                 keys.numel(), off.numpy(), bags, 0, None if w is None else w.numpy(),
                 O.F32 if weighted else 0, O.F32, host_order=True)
    assert np.array_equal(got.numpy().view(np.uint32), ref.view(np.uint32))


def test_fp16_embedding_concat_and_bag():
    g = torch.Generator().manual_seed(4)
    rows, dim = 500, 24
    init = (torch.randn(rows, dim, generator=g) * 0.1).half()
    keys = torch.randint(0, rows, (90,), generator=g)
    emb = nve_layers.NVEmbedding(rows, dim, torch.float16, LT.HostLayer, weight_init=init,
                                 optimize_for_training=False, device="cpu")
    out = emb(keys)
    assert out.dtype == torch.float16 and torch.equal(out, init[keys])
    bag = make_bag(rows, dim, torch.float16, "concat", init)
    assert torch.equal(bag(keys, torch.tensor([0, 90])), init[keys])
    bag = make_bag(rows, dim, torch.float16, "sum", init)
    off = torch.arange(0, 91, 9)
    got = bag(keys, off)
    want = torch.nn.functional.embedding_bag(keys, init.float(), off, mode="sum", include_last_offset=True)
    assert got.dtype == torch.float16
    assert torch.allclose(got.float(), want, rtol=1e-3, atol=1e-3)


def test_missed_keys_read_the_default_row():
    rows, dim = 10, 4
    init = torch.arange(rows * dim, dtype=torch.float32).view(rows, dim)
    default = torch.full((dim,), -2.0)
    emb = nve_layers.NVEmbedding(rows, dim, torch.float32, LT.HostLayer, weight_init=init,
                                 optimize_for_training=False, device="cpu",
                                 config={"default_embedding": default})
    out = emb(torch.tensor([1, 10, -5, 9]))
    assert torch.equal(out[0], init[1]) and torch.equal(out[3], init[9])
    assert torch.equal(out[1], default) and torch.equal(out[2], default)
    # without a configured default, a host layer reads zeros for a missed key
    emb0 = nve_layers.NVEmbedding(rows, dim, torch.float32, LT.HostLayer, weight_init=init,
                                  optimize_for_training=False, device="cpu")
    assert torch.all(emb0(torch.tensor([123]))[0] == 0)


def test_update_on_a_host_memblock_and_checkpoint_round_trip():
    rows, dim = 16, 8
    host = np.zeros((rows, dim), np.float32)
    block = nve.UserMemBlock(host.ctypes.data, host.nbytes)
    emb = nve_layers.NVEmbedding(rows, dim, torch.float32, LT.HostLayer, storage=block,
                                 optimize_for_training=False, device="cpu", id=77)
    keys = torch.tensor([2, 5])
    vals = torch.ones(2, dim) * torch.tensor([[3.0], [4.0]])
    emb.update(keys, vals)
    assert np.all(host[2] == 3) and np.all(host[5] == 4)
    assert torch.equal(emb(torch.tensor([5, 2])), vals.flip(0))
    # the .nve container round trip of a host table
    buf = io.BytesIO()
    fmt = nve.TensorFileFormat()
    fmt.write_table_file_header(buf)
    nve.write_tensor_to_stream(emb.emb_layer, buf, 77)
    host[:] = 0
    emb.load_from_stream(buf)
    assert np.all(host[2] == 3) and np.all(host[5] == 4)


def test_host_layer_rejects_training():
    with pytest.raises(ValueError):
        nve_layers.NVEmbedding(10, 4, torch.float32, LT.HostLayer, device="cpu")


def test_concurrent_gathers_on_one_layer():
    """test_host_cpu.py:454-497: 8 threads gather disjoint rows of one layer
    200 times each; row i holds the value i, so a lookup that another thread's
    scratch clobbered shows at once.  Each calling thread has its own
    execution context (the module's default row keeps the lookup's hit bits
    in context scratch)."""
    import threading
    rows, dim, nt = 4096, 16, 8
    w = torch.arange(rows, dtype=torch.float32)[:, None].expand(rows, dim).contiguous()
    layer = nve_layers.NVEmbedding(rows, dim, torch.float32, LT.HostLayer, weight_init=w,
                                   optimize_for_training=False, device="cpu")
    errors = []
    barrier = threading.Barrier(nt)

    def worker(tid):
        keys = torch.arange(tid, rows, nt, dtype=torch.int64)
        want = w[keys]
        try:
            barrier.wait()
            for _ in range(200):
                if not torch.equal(layer(keys), want):
                    raise AssertionError(f"thread {tid}: rows of another lookup")
        except Exception as exc:  # noqa: BLE001 - reported by the main thread
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(nt)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


def test_concurrent_gathers_on_distinct_layers():
    """test_host_cpu.py:500-537: 6 threads, each with its own layer whose
    values are offset per layer, so a context shared across layers shows."""
    import threading
    rows, dim, nt = 1024, 8, 6
    ws = [(torch.arange(rows, dtype=torch.float32) + t * rows)[:, None].expand(rows, dim).contiguous()
          for t in range(nt)]
    layers = [nve_layers.NVEmbedding(rows, dim, torch.float32, LT.HostLayer, weight_init=ws[t],
                                     optimize_for_training=False, device="cpu") for t in range(nt)]
    keys = torch.tensor([0, 5, 17, 256, 1023], dtype=torch.int64)
    errors = []
    barrier = threading.Barrier(nt)

    def worker(tid):
        want = ws[tid][keys]
        try:
            barrier.wait()
            for _ in range(200):
                if not torch.equal(layers[tid](keys), want):
                    raise AssertionError(f"thread {tid}: another layer's rows")
        except Exception as exc:  # noqa: BLE001
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(nt)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors


def test_binding_lookups_from_several_threads():
    """The pynve binding itself (nve.HostEmbedding over a caller's memory
    block, lookups with no stream) from 8 threads: each thread gets its own
    execution context (a context is not thread-safe).  With a default row the
    lookup keeps its hit bits in the context's scratch, which threads sharing
    one context overwrite: rows went missing that way."""
    import threading
    rows, dim, nt = 4096, 16, 8
    table = np.repeat(np.arange(rows, dtype=np.float32)[:, None], dim, axis=1)
    mb = nve.UserMemBlock(table.ctypes.data, table.nbytes)
    cfg = nve.EmbedLayerConfig()
    cfg.default_embedding = [0] * (dim * 4)
    layer = nve.HostEmbedding(dim, rows, nve.DataType_t.Float32, mb, config=cfg)
    errors = []
    barrier = threading.Barrier(nt)

    def worker(tid):
        keys = np.arange(tid, rows, nt, dtype=np.int64)
        out = np.zeros((keys.size, dim), np.float32)
        try:
            barrier.wait()
            for _ in range(200):
                out[:] = -1
                layer.lookup(keys.size, keys.ctypes.data, out.ctypes.data, 0)
                if not np.array_equal(out, table[keys]):
                    raise AssertionError(f"thread {tid}: rows of another lookup")
        except Exception as exc:  # noqa: BLE001
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(nt)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors
    layer.release_contexts()


def test_distributed_checkpoint_loads_into_the_layer_weight(tmp_path):
    """test_dcp_load.py:112-141 on one process: a torch.distributed.checkpoint
    of an nn.Embedding's weight is loaded in place into the layer's weight
    (the table the layer reads), and lookups then return those rows."""
    import torch.distributed.checkpoint as dcp
    torch.manual_seed(6)
    ref = torch.nn.Embedding(10, 2)
    dcp.save({"embedding": {"embed.weight": ref.weight.detach()}}, checkpoint_id=str(tmp_path))
    layer = nve_layers.NVEmbedding(10, 2, torch.float32, LT.HostLayer, optimize_for_training=False,
                                   device="cpu")
    dcp.load({"embedding": {"embed.weight": layer.weight}}, checkpoint_id=str(tmp_path))
    assert torch.equal(layer.weight.detach(), ref.weight.detach())
    k = torch.tensor([1, 5, 9, 0])
    assert torch.equal(layer(k), ref(k).detach())

"""GPU parity of the torch surface (pynve.torch.nve_layers over libnve_amd.so):
the cases of the reference's tests/python_binding/test_pytorch.py that the
GPU and LinearUVM layers cover -- lookups bit-exact against torch.nn.Embedding,
pooling against torch.nn.EmbeddingBag (include_last_offset=True) and the
oracle, multi-stream and multi-layer use, managed memory blocks, default row
index routing, and the cache modify calls."""
import numpy as np
import pytest

from nve_helpers import pooled_f16_close, rel_close
from oracle import oracle as O

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from pynve import _lib, nve  # noqa: E402
from pynve.torch import nve_layers  # noqa: E402

LT = nve_layers.LayerType
CACHE = 128 * 1024 * 1024


def make(layer_type, weight, *, bag_mode=None, cache=CACHE, train=False, config=None):
    n, d = weight.shape
    kw = dict(weight_init=weight, optimize_for_training=train, config=config)
    if layer_type == LT.LinearUVM:
        kw["gpu_cache_size"] = cache
    if bag_mode is None:
        return nve_layers.NVEmbedding(n, d, weight.dtype, layer_type, **kw)
    return nve_layers.NVEmbeddingBag(n, d, weight.dtype, layer_type, bag_mode, **kw)


@pytest.mark.parametrize("layer_type", [LT.GPULayer, LT.LinearUVM], ids=["gpu", "uvm"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("train", [False, True])
def test_concat_matches_torch_embedding(layer_type, dtype, train):
    # test_pytorch.py:265-270 (functional): several steps of the same keys
    torch.manual_seed(0)
    ref = torch.nn.Embedding(10000, 2, dtype=dtype, device="cuda")
    layer = make(layer_type, ref.weight.detach(), train=train)
    keys = torch.tensor([5, 4, 3, 100, 1024, 6], dtype=torch.int64, device="cuda")
    with torch.no_grad():
        for _ in range(6):
            out = layer(keys)
            assert out.dtype == dtype and tuple(out.shape) == (6, 2)
            assert torch.equal(out, ref(keys))


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_pooling_matches_torch_embedding_bag(dtype):
    # test_pytorch.py:533-552 (functional_bag, rtol 1e-10)
    torch.manual_seed(1)
    ref = torch.nn.EmbeddingBag(10000, 2, mode="sum", dtype=dtype, include_last_offset=True,
                                device="cuda")
    w = ref.weight.detach()
    uvm = make(LT.LinearUVM, w, bag_mode="sum")
    gpu = make(LT.GPULayer, w, bag_mode="sum")
    keys = torch.tensor([5, 4, 3, 100, 1024, 6], dtype=torch.int64, device="cuda")
    offsets = torch.tensor([0, 3, 6], dtype=torch.int64, device="cuda")
    with torch.no_grad():
        t = ref(keys, offsets)
        for _ in range(6):
            g, u = gpu(keys, offsets), uvm(keys, offsets)
            assert torch.isclose(g, t, rtol=1e-10).all() and torch.isclose(u, t, rtol=1e-10).all()
            assert torch.equal(u, g)


@pytest.mark.parametrize("layer_type", [LT.GPULayer, LT.LinearUVM], ids=["gpu", "uvm"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("mode,weighted", [("sum", False), ("mean", False), ("sum", True),
                                           ("mean", True)])
def test_random_bags_against_oracle(layer_type, dtype, mode, weighted):
    rng = np.random.default_rng(layer_type.value * 8 + (dtype == torch.float16) * 4
                                + (mode == "mean") * 2 + weighted)
    rows, dim, bags = 50000, 64, 300
    w = torch.from_numpy(rng.normal(0, 0.05, size=(rows, dim)).astype(
        np.float32 if dtype == torch.float32 else np.float16))
    layer = make(layer_type, w, bag_mode=mode, cache=4 << 20)
    lens = rng.integers(0, 80, size=bags)
    off = np.zeros(bags + 1, np.int64)
    off[1:] = np.cumsum(lens)
    keys = O.power_law(rng.random(int(off[-1])), 1, rows - 1, 1.05).astype(np.int64)
    wts = rng.uniform(0, 1, size=keys.size).astype(np.float32 if dtype == torch.float32 else np.float16)
    d_keys, d_off = torch.from_numpy(keys).cuda(), torch.from_numpy(off).cuda()
    d_w = torch.from_numpy(wts).cuda() if weighted else None
    odt = O.F32 if dtype == torch.float32 else O.F16
    pooling = {("sum", False): O.SUM, ("mean", False): O.MEAN, ("sum", True): O.WSUM,
               ("mean", True): O.WMEAN}[(mode, weighted)]
    tb = np.ascontiguousarray(w.numpy().view(np.uint8).reshape(rows, -1))
    flat = tb.reshape(-1)  # the row pointers below point into this array
    ref = O.pool(O.linear_row_ptrs(keys, flat, tb.shape[1]), odt,
                 dim, O.CSR, pooling, keys.size, off, bags, 0, wts if weighted else None,
                 odt if weighted else O.F32, odt)
    with torch.no_grad():
        for _ in range(3):  # the UVM layer warms its cache between calls
            out = layer(d_keys, d_off, d_w).cpu().numpy()
            if dtype == torch.float32:
                assert rel_close(out, ref, rtol=1e-5)
            else:
                assert pooled_f16_close(out.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("kernel_mode", [1, 2, 3])
def test_linear_gather_flows(kernel_mode):
    # test_pytorch.py:367-384: every lookup mode of a LinearUVM layer returns torch.nn.Embedding's rows
    torch.manual_seed(10)
    ref = torch.nn.Embedding(200000, 4, device="cuda")
    layer = make(LT.LinearUVM, ref.weight.detach(), cache=1 << 20,
                 config={"kernel_mode": kernel_mode, "kernel_mode_value_1": 256})
    gen = torch.Generator(device="cuda")
    gen.manual_seed(kernel_mode)
    with torch.no_grad():
        for _ in range(5):
            keys = torch.randint(0, 200000, (20000,), generator=gen, device="cuda")
            keys[:5000] = keys[:5000] % 3000
            assert torch.equal(layer(keys), ref(keys))


def test_multi_stream():
    # test_pytorch.py:554-576
    torch.manual_seed(2)
    ref = torch.nn.Embedding(10000, 2, device="cuda")
    layer = make(LT.LinearUVM, ref.weight.detach().cpu())
    key_sets = [[5, 4, 3, 100, 1024, 6], [345, 7, 19, 45, 2837, 34], [134, 295, 20, 1, 76, 207]]
    outs = []
    with torch.no_grad():
        for ks in key_sets:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                k = torch.tensor(ks, dtype=torch.int64, device="cuda")
                outs.append((layer(k), ref(k)))
        torch.cuda.synchronize()
    for a, b in outs:
        assert torch.equal(a, b)
    # one execution context per stream, made by the native ops on first use
    assert nve._native_ops.num_contexts(layer.marker_tensor.data_ptr()) == len(key_sets)


@pytest.mark.parametrize("layer_type", [LT.GPULayer, LT.LinearUVM], ids=["gpu", "uvm"])
def test_multi_thread(layer_type):
    """test_pytorch.py:711-747: threads share one layer, each lookup on a
    stream of its own (a 1 MiB cache for the LinearUVM layer, so its default
    auto-insert runs between lookups); every output equals torch.nn.Embedding."""
    import threading
    torch.manual_seed(4)
    n, nt, iters = 100000, 4, 6
    ref = torch.nn.Embedding(n, 2, device="cuda")
    layer = make(layer_type, ref.weight.detach().cpu(), cache=1 << 20)
    keys = [[torch.randint(0, n, (4096,), device="cuda") for _ in range(iters)] for _ in range(nt)]
    results = [[] for _ in range(nt)]
    errors = []

    def worker(t):
        try:
            with torch.no_grad():
                for k in keys[t]:
                    s = torch.cuda.Stream()
                    s.wait_stream(torch.cuda.default_stream())
                    with torch.cuda.stream(s):
                        results[t].append(layer(k))
                    s.synchronize()
        except Exception as exc:  # noqa: BLE001 - reported by the main thread
            errors.append(exc)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(nt)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    with torch.no_grad():
        for t in range(nt):
            for k, out in zip(keys[t], results[t]):
                assert torch.equal(out, ref(k))


def test_multi_layer_registry():
    # test_pytorch.py:433-448
    torch.manual_seed(3)
    r1 = torch.nn.Embedding(1000, 4, device="cuda")
    r2 = torch.nn.Embedding(1000, 4, device="cuda")
    l1 = make(LT.LinearUVM, r1.weight.detach(), cache=128 * 1024)
    l2 = make(LT.LinearUVM, r2.weight.detach(), cache=128 * 1024)
    keys = torch.arange(1, 11, dtype=torch.int64, device="cuda")
    with torch.no_grad():
        assert torch.equal(l1(keys), r1(keys))
        assert torch.equal(l2(keys), r2(keys))
    marker = l1.marker_tensor.data_ptr()
    assert nve.get_binding(marker) is l1.emb_layer
    del l1
    import gc
    gc.collect()
    with pytest.raises(RuntimeError, match="no binding registered"):
        nve.get_binding(marker)


def test_managed_memblock():
    # test_pytorch.py:386-395
    mb = nve.ManagedMemBlock(2, 100000, nve.DataType_t.Float32, [0])
    layer = nve_layers.NVEmbedding(100000, 2, torch.float32, LT.LinearUVM, storage=mb,
                                   gpu_cache_size=128 * 1024,
                                   weight_init=torch.zeros(100000, 2), optimize_for_training=False)
    keys = torch.arange(1, 11, dtype=torch.int64, device="cuda")
    assert torch.equal(layer(keys), torch.zeros(10, 2, device="cuda"))
    assert layer.memblock_type == nve.MemBlockType.Managed


def test_host_memblock_copy_from():
    rng = np.random.default_rng(4)
    table = rng.normal(size=(5000, 8)).astype(np.float32)
    mb = nve.HostMemBlock(8, 5000, nve.DataType_t.Float32)
    mb.copy_from(table)
    layer = nve_layers.NVEmbedding(5000, 8, torch.float32, LT.LinearUVM, storage=mb,
                                   gpu_cache_size=1 << 20, optimize_for_training=False)
    keys = torch.from_numpy(rng.integers(0, 5000, size=777)).cuda()
    assert np.array_equal(layer(keys).cpu().numpy(), table[keys.cpu().numpy()])
    with pytest.raises(IndexError):
        mb.copy_from(np.zeros(5000 * 8 + 1, np.float32))


MISS_ROWS = 64


def _miss_weight():
    return torch.arange(MISS_ROWS * 4, dtype=torch.float32).reshape(MISS_ROWS, 4)


@pytest.mark.parametrize("layer_type", [LT.GPULayer, LT.LinearUVM], ids=["gpu", "uvm"])
def test_default_row_index_routes_out_of_range_keys(layer_type):
    # test_pytorch.py:948-960
    w = _miss_weight()
    layer = make(layer_type, w, cache=1 << 20, config={"default_row_index": 3})
    assert layer.config.default_row_index == 3
    keys = torch.tensor([7, MISS_ROWS + 5, -3, 10**9], dtype=torch.int64, device="cuda")
    expected = torch.stack([w[7], w[3], w[3], w[3]])
    for _ in range(2):
        assert torch.equal(layer(keys).cpu(), expected)


@pytest.mark.parametrize("layer_type", [LT.GPULayer, LT.LinearUVM], ids=["gpu", "uvm"])
def test_default_row_index_bag_pooled_and_rejected(layer_type):
    # test_pytorch.py:974-991
    w = _miss_weight()
    bag = make(layer_type, w, bag_mode="sum", cache=1 << 20, config={"default_row_index": 3})
    keys = torch.tensor([0, MISS_ROWS + 1, 5, 9], dtype=torch.int64, device="cuda")
    offsets = torch.tensor([0, 2, 4], dtype=torch.int64, device="cuda")
    assert torch.allclose(bag(keys, offsets).cpu(), torch.stack([w[0] + w[3], w[5] + w[9]]))
    with pytest.raises(RuntimeError, match="Default row index"):
        make(layer_type, w, cache=1 << 20, config={"default_row_index": MISS_ROWS})


def test_uvm_insert_erase_clear():
    # cached rows win over the backing table until they are erased / cleared
    # (test_pytorch.py:496-531 pattern, on the one-table LinearUVM layer)
    w = torch.zeros(1 << 16, 2)
    layer = make(LT.LinearUVM, w, cache=1 << 16)
    keys = torch.tensor([1, 2, 3, 4, 5], dtype=torch.int64, device="cuda")
    vals = torch.arange(1, 11, dtype=torch.float32, device="cuda")
    layer.insert(keys, vals, table_id=0)
    torch.cuda.synchronize()
    assert torch.equal(layer(keys), vals.reshape(5, 2))
    layer.erase(keys[:2], table_id=0)
    torch.cuda.synchronize()
    out = layer(keys)
    assert torch.equal(out[:2], torch.zeros(2, 2, device="cuda"))
    assert torch.equal(out[2:], vals.reshape(5, 2)[2:])
    layer.clear()
    torch.cuda.synchronize()
    assert torch.equal(layer(keys), torch.zeros(5, 2, device="cuda"))


def _coalesced(grad):
    g = grad.coalesce()
    return g.indices().cpu(), g.values().float().cpu()


@pytest.mark.parametrize("layer_type", [LT.GPULayer, LT.LinearUVM], ids=["gpu", "uvm"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_embedding_backward_matches_torch(layer_type, dtype):
    # NVEmbeddingOpTraining.backward (nve_ops.py:108-127): the sparse table
    # gradient equals torch.nn.Embedding(sparse=True)'s; 2-D keys with repeats
    # (the op returns one row per key, [keys.numel(), dim])
    torch.manual_seed(5)
    rows, dim = 1000, 16
    ref = torch.nn.Embedding(rows, dim, sparse=True, device="cuda")
    layer = make(layer_type, ref.weight.detach().to(dtype), train=True)
    keys = torch.randint(0, 200, (64, 5), device="cuda")
    g_out = torch.randn(64 * 5, dim, device="cuda").to(dtype)
    (layer(keys) * g_out).sum().backward()
    (ref(keys).reshape(-1, dim) * g_out.float()).sum().backward()
    gi, gv = _coalesced(layer.weight.grad)
    ri, rv = _coalesced(ref.weight.grad)
    assert torch.equal(gi, ri)
    tol = 1e-5 if dtype == torch.float32 else 2.0 ** -10  # fp16: one rounding of an fp32 sum
    assert torch.allclose(gv, rv, rtol=tol, atol=tol * rv.abs().max().item())
    assert layer.weight.grad.dtype == dtype


@pytest.mark.parametrize("mode,weighted", [("sum", False), ("mean", False), ("sum", True)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
def test_embedding_bag_backward_matches_torch(mode, weighted, dtype):
    # NVEmbeddingBagOpTraining.backward (nve_ops.py:186-226) against
    # torch.nn.EmbeddingBag(sparse=True, include_last_offset=True), empty bags included
    torch.manual_seed(7)
    rows, dim, bags = 5000, 32, 300
    ref = torch.nn.EmbeddingBag(rows, dim, mode=mode, sparse=True, include_last_offset=True, device="cuda")
    layer = make(LT.GPULayer, ref.weight.detach().to(dtype), bag_mode=mode, train=True)
    lens = torch.randint(0, 40, (bags,))
    lens[::11] = 0
    offsets = torch.zeros(bags + 1, dtype=torch.int64)
    offsets[1:] = torch.cumsum(lens, 0)
    n = int(offsets[-1])
    keys = (torch.from_numpy(np.random.default_rng(3).zipf(1.2, size=n)) % rows).to(torch.int64).cuda()
    offsets = offsets.cuda()
    psw = torch.rand(n, device="cuda").to(dtype) if weighted else None
    g_out = torch.randn(bags, dim, device="cuda").to(dtype)
    (layer(keys, offsets, psw) * g_out).sum().backward()
    (ref(keys, offsets, per_sample_weights=None if psw is None else psw.float()) * g_out.float()).sum().backward()
    gi, gv = _coalesced(layer.weight.grad)
    ri, rv = _coalesced(ref.weight.grad)
    assert torch.equal(gi, ri)
    tol = 1e-5 if dtype == torch.float32 else 2.0 ** -10
    assert torch.allclose(gv, rv, rtol=tol, atol=tol * rv.abs().max().item())


def test_sgd_steps_match_torch_embedding_bag():
    # a sparse-gradient training loop: SGD applies the gradient through
    # CachedTable.add_ (nve_tensors.py:64-80) into the layer's table
    torch.manual_seed(11)
    rows, dim, bags, hot = 2000, 16, 64, 8
    ref = torch.nn.EmbeddingBag(rows, dim, mode="sum", sparse=True, include_last_offset=True, device="cuda")
    layer = make(LT.GPULayer, ref.weight.detach().clone(), bag_mode="sum", train=True)
    opt_ref = torch.optim.SGD(ref.parameters(), lr=0.05, foreach=False)
    opt = torch.optim.SGD([layer.weight], lr=0.05, foreach=False)
    offsets = torch.arange(0, bags * hot + 1, hot, device="cuda")
    for step in range(4):
        keys = torch.randint(0, 300, (bags * hot,), device="cuda")
        target = torch.randn(bags, dim, device="cuda")
        for model, o in ((layer, opt), (ref, opt_ref)):
            o.zero_grad()
            ((model(keys, offsets) - target) ** 2).sum().backward()
            o.step()
    torch.cuda.synchronize()
    probe = torch.arange(0, 300, device="cuda")
    one = torch.arange(0, 301, device="cuda")
    with torch.no_grad():
        assert torch.allclose(layer(probe, one), ref(probe, one), rtol=1e-5, atol=1e-5)


def test_inference_layer_has_no_gradient_path():
    # optimize_for_training=False: the op does not take the weight, so the
    # output is not part of an autograd graph (nve_ops.py:65-86)
    w = torch.randn(100, 4)
    keys = torch.tensor([1, 2, 3], dtype=torch.int64, device="cuda")
    infer = make(LT.GPULayer, w, train=False)
    out = infer(keys)
    assert not out.requires_grad
    assert torch.equal(out, w[keys.cpu()].cuda())


@pytest.mark.parametrize("layer_type", [LT.GPULayer, LT.LinearUVM], ids=["gpu", "uvm"])
def test_layer_update_and_sparse_add(layer_type):
    # NVEmbeddingBase.update (nve_layers.py:356-367) and CachedTable.add_ (nve_tensors.py:64-80):
    # rows change in the table and in the GPU cache; dyadic values keep the sums exact
    rng = np.random.default_rng(9)
    rows, dim = 2000, 16
    w = torch.from_numpy((rng.integers(-8, 9, size=(rows, dim)) / 64.0).astype(np.float32))
    layer = make(layer_type, w, cache=1 << 20)
    keys = torch.tensor([3, 17, 1999, 256], dtype=torch.int64, device="cuda")
    with torch.no_grad():
        layer(keys)  # (UVM: the lookup may start caching these rows)
        new = torch.full((4, dim), 0.5, device="cuda")
        layer.update(keys, new)
        torch.cuda.synchronize()
        assert torch.equal(layer(keys), new)
        grad = torch.sparse_coo_tensor(torch.tensor([[3, 3, 5]]), torch.full((3, dim), 0.25),
                                       (rows, dim)).cuda()
        layer.weight.add_(grad, alpha=-1.0)
        out = layer(torch.tensor([3, 5, 17], dtype=torch.int64, device="cuda"))
        exp = torch.stack([new[0] - 0.5, w[5].cuda() - 0.25, new[1]])
        assert torch.equal(out, exp)


def test_direct_binding_calls():
    # pynve.nve bindings with raw pointers (binding_layers.hpp:86-129)
    rng = np.random.default_rng(6)
    table = torch.from_numpy(rng.normal(size=(4096, 16)).astype(np.float16)).cuda()
    mb = nve.UserMemBlock(table.data_ptr(), table.nbytes)
    b = nve.GPUEmbedding(16, 4096, nve.DataType_t.Float16, mb, 0, nve.EmbedLayerConfig())
    assert b.get_embedding_dim() == 16 and b.get_data_type() == nve.DataType_t.Float16
    keys = torch.from_numpy(rng.integers(0, 4096, size=1000)).cuda()
    out = torch.empty(1000, 16, dtype=torch.float16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    b.lookup(1000, keys.data_ptr(), out.data_ptr(), s)
    torch.cuda.synchronize()
    assert torch.equal(out, table[keys])
    off = torch.tensor([0, 400, 400, 1000], dtype=torch.int64, device="cuda")
    pooled = torch.empty(3, 16, dtype=torch.float16, device="cuda")
    b.lookup_with_pooling(1000, keys.data_ptr(), pooled.data_ptr(), int(nve.PoolingType_t.Sum),
                          4, off.data_ptr(), 0, 0, s)
    torch.cuda.synchronize()
    ref = torch.nn.functional.embedding_bag(keys, table.float(), off, mode="sum",
                                            include_last_offset=True)
    assert torch.allclose(pooled.float(), ref, rtol=2e-3, atol=2e-3)
    assert torch.equal(pooled[1], torch.zeros(16, dtype=torch.float16, device="cuda"))
    with pytest.raises(_lib.InvalidArgument):
        # GPU layers take weights of the table's dtype only (gpu_embedding_layer.cu:410-413)
        wts = torch.ones(1000, device="cuda")
        b.lookup_with_pooling(1000, keys.data_ptr(), pooled.data_ptr(),
                              int(nve.PoolingType_t.WeightedSum), 4, off.data_ptr(),
                              int(nve.DataType_t.Float32), wts.data_ptr(), s)


@pytest.mark.parametrize("layer_type", [LT.GPULayer, LT.LinearUVM], ids=["gpu", "uvm"])
def test_distributed_checkpoint_loads_into_the_layer_weight(layer_type, tmp_path):
    """test_dcp_load.py:112-141 on one process: a torch.distributed.checkpoint
    of an nn.Embedding's weight loads in place into the layer's weight, and
    lookups then return the loaded rows."""
    import torch.distributed.checkpoint as dcp
    torch.manual_seed(7)
    ref = torch.nn.Embedding(1000, 8)
    dcp.save({"embedding": {"embed.weight": ref.weight.detach()}}, checkpoint_id=str(tmp_path))
    layer = make(layer_type, torch.zeros(1000, 8))
    dcp.load({"embedding": {"embed.weight": layer.weight}}, checkpoint_id=str(tmp_path))
    assert torch.equal(layer.weight.detach().cpu(), ref.weight.detach())
    k = torch.randint(0, 1000, (256,), device="cuda")
    with torch.no_grad():
        assert torch.equal(layer(k).cpu(), ref(k.cpu()))

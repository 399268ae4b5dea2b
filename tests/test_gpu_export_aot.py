"""GPU checks of the AOTInductor path (pynve.torch.nve_export.export_aot /
load_aot / rebind_markers and the C++ nve::LayerDirectory of
include/nve_loader.hpp), following the reference's
tests/python_binding/test_nve_export.py AOT cases and its C++ inference test
(tests/python_binding/export_inference_test.cpp):

* a model with a GPU-table NVEmbedding and a LinearUVM NVEmbeddingBag (fp16,
  in a submodule) plus dense ops is packaged, then loaded in this process, in a
  fresh Python process and in a fresh C++ process (tests/cpp/
  aoti_loader_check.cpp); every output equals the eager output bit for bit;
* dynamic batch sizes, two packages whose layers share an id, a host layer
  bound to the GPU, and rebinding after the package's marker was replaced."""
import os
import subprocess
import sys

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from pynve.torch import nve_export as E  # noqa: E402
from pynve.torch import nve_layers  # noqa: E402

LT = nve_layers.LayerType
DEV = torch.device("cuda")
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CPP_CHECK = os.path.join(ROOT, "nv-embedding-cache_amd", "aoti_loader_check")


class Tower(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.bag = nve_layers.NVEmbeddingBag(3000, 16, torch.float16, LT.LinearUVM, "sum",
                                             gpu_cache_size=1 << 20, optimize_for_training=False, device=DEV)
        self.bag.weight.data.copy_(torch.randn(3000, 16, device=DEV).half())


class Model(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.emb = nve_layers.NVEmbedding(5000, 16, torch.float32, LT.GPULayer, optimize_for_training=False,
                                          device=DEV)
        self.emb.weight.data.copy_(torch.randn(5000, 16, device=DEV))
        self.tower = Tower()
        torch.cuda.synchronize()

    def forward(self, keys, bag_keys, offsets):
        rows = self.emb(keys)
        pooled = self.tower.bag(bag_keys, offsets)
        return rows * 2.0, pooled.float() + 1.0


def inputs(seed=0, n=64, bags=8):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    keys = torch.randint(0, 5000, (n,), device=DEV, generator=g)
    bag_keys = torch.randint(0, 3000, (bags * 6,), device=DEV, generator=g)
    offsets = torch.arange(0, bags * 6 + 1, 6, device=DEV)
    return keys, bag_keys, offsets


def same(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def write_io(io_dir, ins, outs):
    """The tensors as raw files plus io.txt, as aoti_loader_check reads them."""
    names = {torch.int64: "int64", torch.float32: "float32", torch.float16: "float16"}
    os.makedirs(io_dir, exist_ok=True)
    lines = []
    for kind, ts in (("in", ins), ("out", outs)):
        for i, t in enumerate(ts):
            f = f"{kind}{i}.bin"
            t.detach().contiguous().cpu().numpy().tofile(os.path.join(io_dir, f))
            lines.append(" ".join([kind, f, names[t.dtype]] + [str(d) for d in t.shape]))
    with open(os.path.join(io_dir, "io.txt"), "w") as fh:
        fh.write("\n".join(lines) + "\n")


def test_package_loads_in_process_and_in_fresh_python_and_cpp_processes(tmp_path):
    model = Model()
    ins = inputs()
    expected = model(*ins)
    save = str(tmp_path / "pkg")
    print("[aoti] export_aot", flush=True)
    E.export_aot(model, ins, save)
    assert os.path.exists(os.path.join(save, "model.pt2"))
    loader, layers = E.load_aot(save)
    got = loader.run(list(ins))
    assert len(got) == 2 and all(same(g, e) for g, e in zip(got, expected))
    del loader, layers

    io_dir = str(tmp_path / "io")
    write_io(io_dir, ins, expected)
    # a fresh Python process: load_aot and compare
    script = (
        "import os, sys, numpy as np, torch\n"
        f"sys.path[:0] = [{ROOT!r}, {os.path.join(ROOT, 'nv-embedding-cache_amd')!r}]\n"
        "from pynve.torch import nve_export as E\n"
        "save, io = sys.argv[1], sys.argv[2]\n"
        "specs = [l.split() for l in open(os.path.join(io, 'io.txt')) if l.strip()]\n"
        "dt = {'int64': np.int64, 'float32': np.float32, 'float16': np.float16}\n"
        "load = lambda s: torch.from_numpy(np.fromfile(os.path.join(io, s[1]), dt[s[2]]).reshape(\n"
        "    [int(d) for d in s[3:]]))\n"
        "ins = [load(s).cuda() for s in specs if s[0] == 'in']\n"
        "outs = [load(s) for s in specs if s[0] == 'out']\n"
        "loader, layers = E.load_aot(save)\n"
        "got = [g.cpu() for g in loader.run(ins)]\n"
        "ok = len(got) == len(outs) and all(torch.equal(g.view(torch.uint8), o.view(torch.uint8))\n"
        "                                   for g, o in zip(got, outs))\n"
        "print('ok' if ok else 'FAIL')\n")
    print("[aoti] fresh python process", flush=True)
    r = subprocess.run([sys.executable, "-c", script, save, io_dir], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr[-2000:]
    # a fresh C++ process through nve::LayerDirectory
    assert os.path.exists(CPP_CHECK), "build the C++ loader check first (make -C nv-embedding-cache_amd)"
    print("[aoti] fresh C++ process", flush=True)
    r = subprocess.run([CPP_CHECK, save, io_dir, str(torch.cuda.current_device())], capture_output=True, text=True,
                       timeout=300)
    assert r.returncode == 0 and r.stdout.startswith("ok"), r.stdout + r.stderr[-2000:]


def test_dynamic_batch(tmp_path):
    model = Model()
    ins = inputs()
    sc = torch.export.ShapesCollection()
    sc[ins[0]] = {0: torch.export.Dim.AUTO(min=1, max=4096)}
    ds = sc.dynamic_shapes(model, ins)
    E.export_aot(model, ins, str(tmp_path), dynamic_shapes=ds)
    loader, layers = E.load_aot(str(tmp_path))
    for n in (64, 5, 1000):
        k = inputs(seed=n, n=n)
        got = loader.run(list(k))
        exp = model(*k)
        assert got[0].shape == (n, 16) and all(same(g, e) for g, e in zip(got, exp))


class One(torch.nn.Module):
    def __init__(self, layer_id, base):
        super().__init__()
        self.emb = nve_layers.NVEmbedding(256, 4, torch.float32, LT.GPULayer, optimize_for_training=False,
                                          device=DEV, id=layer_id)
        self.emb.weight.data.copy_((torch.arange(256, dtype=torch.float32, device=DEV) + base)[:, None].expand(256, 4))
        torch.cuda.synchronize()

    def forward(self, keys):
        return self.emb(keys)


def test_two_packages_with_one_layer_id(tmp_path):
    keys = torch.tensor([0, 1, 5, 10], device=DEV)
    a, b = One(0, 0.0), One(0, 1000.0)
    ea, eb = a(keys), b(keys)
    E.export_aot(a, (keys,), str(tmp_path / "a"))
    E.export_aot(b, (keys,), str(tmp_path / "b"))
    la, layers_a = E.load_aot(str(tmp_path / "a"))
    lb, layers_b = E.load_aot(str(tmp_path / "b"))
    assert same(la.run([keys])[0], ea) and same(lb.run([keys])[0], eb)
    assert not torch.equal(ea, eb)


def test_rebind_markers_after_the_marker_was_replaced(tmp_path):
    """The package's marker constant decides which layer its op reaches: set to
    another package's (registered) marker, package a returns b's rows, until
    rebind_markers points it at a's own layer again."""
    keys = torch.tensor([3, 7, 200], device=DEV)
    a, b = One(11, 5.0), One(12, 900.0)
    ea, eb = a(keys), b(keys)
    E.export_aot(a, (keys,), str(tmp_path / "a"))
    E.export_aot(b, (keys,), str(tmp_path / "b"))
    la, layers_a = E.load_aot(str(tmp_path / "a"))
    lb, layers_b = E.load_aot(str(tmp_path / "b"))
    assert same(la.run([keys])[0], ea)
    la.load_constants({"emb.marker_tensor": layers_b[0].marker_tensor}, False, False, True)
    assert same(la.run([keys])[0], eb)
    E.rebind_markers(la, layers_a)
    E.rebind_markers(la, layers_a)  # idempotent
    assert same(la.run([keys])[0], ea) and same(lb.run([keys])[0], eb)


def test_host_layer_on_the_gpu(tmp_path):
    w = torch.arange(512, dtype=torch.float32)[:, None].expand(512, 8).contiguous()

    class M(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.emb = nve_layers.NVEmbedding(512, 8, torch.float32, layer_type=LT.HostLayer, weight_init=w,
                                              optimize_for_training=False, device=DEV)
            self.bag = nve_layers.NVEmbeddingBag(512, 8, torch.float32, layer_type=LT.HostLayer, mode="sum",
                                                 weight_init=w, optimize_for_training=False, device=DEV)

        def forward(self, keys, offsets):
            return self.emb(keys), self.bag(keys, offsets)

    keys = torch.tensor([0, 5, 17, 256, 511], device=DEV)
    offsets = torch.tensor([0, 2, 5], device=DEV)
    model = M()
    expected = model(keys, offsets)
    E.export_aot(model, (keys, offsets), str(tmp_path))
    del model
    loader, layers = E.load_aot(str(tmp_path))
    assert [l.layer_type for l in layers] == [LT.HostLayer, LT.HostLayer]
    got = loader.run([keys, offsets])
    assert all(g.device.type == "cuda" for g in got)
    assert all(same(g, e) for g, e in zip(got, expected))

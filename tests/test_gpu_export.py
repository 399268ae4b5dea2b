"""GPU checks of saving and reloading models with NVE layers
(pynve.torch.nve_export), the cases of the reference's
tests/python_binding/test_nve_export.py that GPU and LinearUVM layers cover:
export / load reproduces the eager outputs bit-for-bit (GPU and cached layers,
NVEmbedding and NVEmbeddingBag), the marker buffer survives and is re-pointed
at the live layer, two models with one layer id stay apart, schema-2 metadata
with resources, shared memory blocks, User-block resolution, config round
trip, registry reuse and key remapping, schema-1 loading, geometry errors."""
import json
import os
import shutil

import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from pynve import nve  # noqa: E402
from pynve.torch import nve_export as E  # noqa: E402
from pynve.torch import nve_layers  # noqa: E402

LT = nve_layers.LayerType
DEV = torch.device("cuda")
NUM_EMB, EMB_SIZE, CACHE = 1024, 8, 4 * 1024 * 1024


def _emb(layer_type=LT.LinearUVM, id=None, base=None, dtype=torch.float32):
    kw = dict(optimize_for_training=False, device=DEV, id=id)
    if layer_type == LT.LinearUVM:
        kw["gpu_cache_size"] = CACHE
    m = nve_layers.NVEmbedding(NUM_EMB, EMB_SIZE, dtype, layer_type, **kw)
    w = (torch.randn(NUM_EMB, EMB_SIZE, device=DEV) if base is None else
         (torch.arange(NUM_EMB, dtype=torch.float32, device=DEV) + base)[:, None]
         .expand(NUM_EMB, EMB_SIZE)).to(dtype)
    m.weight.data.copy_(w)
    torch.cuda.synchronize()
    return m


class One(torch.nn.Module):
    def __init__(self, emb):
        super().__init__()
        self.emb = emb

    def forward(self, keys):
        return self.emb(keys)


class Two(torch.nn.Module):
    def __init__(self, a, b):
        super().__init__()
        self.emb_a, self.emb_b = a, b

    def forward(self, keys):
        return self.emb_a(keys) + self.emb_b(keys)


class BagModel(torch.nn.Module):
    def __init__(self, layer_type):
        super().__init__()
        kw = dict(optimize_for_training=False, device=DEV)
        if layer_type == LT.LinearUVM:
            kw["gpu_cache_size"] = CACHE
        self.tower = torch.nn.Module()
        self.tower.bag = nve_layers.NVEmbeddingBag(NUM_EMB, 16, torch.float16, layer_type, "sum",
                                                   **kw)
        self.tower.bag.weight.data.copy_(torch.randn(NUM_EMB, 16, device=DEV).half())
        torch.cuda.synchronize()

    def forward(self, keys, offsets):
        return self.tower.bag(keys, offsets)


@pytest.mark.parametrize("layer_type", [LT.LinearUVM, LT.GPULayer], ids=["uvm", "gpu"])
def test_export_and_load(tmp_path, layer_type):
    model = One(_emb(layer_type))
    keys = torch.randint(0, NUM_EMB, (32,), device=DEV, dtype=torch.int64)
    expected = model(keys)
    E.export(model, (keys,), str(tmp_path))
    assert os.path.exists(tmp_path / "model.pt2")
    meta = json.load(open(tmp_path / "metadata.json"))
    assert meta["version"] == 2 and len(meta["layers"]) == 1
    l0 = meta["layers"][0]
    assert (l0["num_embeddings"], l0["embedding_size"], l0["layer_type"]) == (
        NUM_EMB, EMB_SIZE, layer_type.name)
    assert l0["storage_ref"] in meta["resources"]["memblocks"]
    # an auto-allocated GPU table is a User block, rebuilt as Linear
    want = "Linear" if layer_type == LT.GPULayer else "Managed"
    assert meta["resources"]["memblocks"][l0["storage_ref"]]["type"] == want
    assert os.listdir(tmp_path / "weights") == [l0["storage_ref"] + ".nve"]
    loaded, layers = E.load(str(tmp_path))
    assert loaded.get_submodule("emb").marker_tensor.data_ptr() == layers[0].marker_tensor.data_ptr()
    assert torch.equal(loaded(keys), expected)
    keys2 = torch.randint(0, NUM_EMB, (32,), device=DEV, dtype=torch.int64)
    assert torch.equal(loaded(keys2), model(keys2))


@pytest.mark.parametrize("layer_type", [LT.LinearUVM, LT.GPULayer], ids=["uvm", "gpu"])
def test_export_and_load_bag_in_submodule(tmp_path, layer_type):
    model = BagModel(layer_type)
    keys = torch.randint(0, NUM_EMB, (40,), device=DEV, dtype=torch.int64)
    offsets = torch.tensor([0, 3, 3, 17, 40], device=DEV, dtype=torch.int64)
    expected = model(keys, offsets)
    E.export(model, (keys, offsets), str(tmp_path))
    meta = json.load(open(tmp_path / "metadata.json"))
    assert meta["layers"][0]["module_path"] == "tower.bag"
    assert meta["layers"][0]["is_bag"] and meta["layers"][0]["mode"] == "sum"
    loaded, layers = E.load(str(tmp_path))
    assert torch.equal(loaded(keys, offsets), expected)


def test_marker_buffer_survives_export(tmp_path):
    model = One(_emb())
    keys = torch.tensor([0, 1], device=DEV, dtype=torch.int64)
    E.export(model, (keys,), str(tmp_path))
    mod = torch.export.load(str(tmp_path / "model.pt2")).module()
    bufs = dict(mod.named_buffers())
    assert "emb.marker_tensor" in bufs
    assert bufs["emb.marker_tensor"].item() == model.emb.id


def test_two_models_sharing_a_layer_id(tmp_path):
    keys = torch.tensor([0, 1, 5, 10], device=DEV, dtype=torch.int64)
    a, b = One(_emb(id=0, base=0.0)), One(_emb(id=0, base=1000.0))
    ea, eb = a(keys), b(keys)
    E.export(a, (keys,), str(tmp_path / "a"))
    E.export(b, (keys,), str(tmp_path / "b"))
    la, layers_a = E.load(str(tmp_path / "a"))
    lb, layers_b = E.load(str(tmp_path / "b"))
    assert layers_a[0].marker_tensor.data_ptr() != layers_b[0].marker_tensor.data_ptr()
    assert torch.equal(la(keys), ea) and torch.equal(lb(keys), eb)
    assert not torch.equal(ea, eb)


def test_shared_memblock_within_model(tmp_path):
    mb = nve.ManagedMemBlock(EMB_SIZE, 512, nve.DataType_t.Float32, [torch.cuda.current_device()])
    mk = lambda: nve_layers.NVEmbedding(512, EMB_SIZE, torch.float32, LT.LinearUVM,  # noqa: E731
                                        gpu_cache_size=1 << 20, storage=mb,
                                        optimize_for_training=False, device=DEV)
    a, b = mk(), mk()
    a.weight.data.copy_(torch.randn(512, EMB_SIZE))
    model = Two(a, b)
    keys = torch.arange(0, 512, 3, device=DEV, dtype=torch.int64)
    expected = model(keys)
    E.save_nve(model, str(tmp_path))
    meta = json.load(open(tmp_path / "metadata.json"))
    refs = [l["storage_ref"] for l in meta["layers"]]
    assert refs[0] == refs[1]
    assert len(os.listdir(tmp_path / "weights")) == 1
    layers = E.load_nve_layers(str(tmp_path))
    assert len(layers) == 2 and layers[0].storage is layers[1].storage
    assert torch.equal(layers[0](keys) + layers[1](keys), expected)


def test_collect_resources_resolves_user_blocks():
    model = One(_emb(LT.GPULayer))
    assert model.emb.memblock_type == nve.MemBlockType.User
    res, _, refs = E._collect_resources(model)
    assert res["memblocks"][refs["emb"]]["type"] == "Linear"
    t = torch.empty(NUM_EMB, EMB_SIZE, dtype=torch.float32, device=DEV)
    shared = nve.UserMemBlock(t.data_ptr(), t.nbytes)
    mk = lambda: nve_layers.NVEmbedding(NUM_EMB, EMB_SIZE, torch.float32, LT.GPULayer,  # noqa: E731
                                        storage=shared, device=DEV)
    res2, _, refs2 = E._collect_resources(Two(mk(), mk()))
    assert refs2["emb_a"] == refs2["emb_b"]
    assert res2["memblocks"][refs2["emb_a"]]["type"] == "Linear"


def test_build_memblock_from_descriptor():
    cfg = {"row_elements": 8, "num_rows": 64, "dtype": "float32"}
    for kind in ("Linear", "Managed", "Host"):
        blk = E._build_memblock_from_descriptor({**cfg, "type": kind}, 0, "cuda")
        assert blk.get_type() == nve.MemBlockType[kind]
        assert blk.get_size_in_bytes() == 8 * 64 * 4


def test_registry_reuse_and_resource_remap(tmp_path):
    mb = nve.ManagedMemBlock(EMB_SIZE, 256, nve.DataType_t.Float32, [torch.cuda.current_device()])
    model = torch.nn.Module()
    model.emb = nve_layers.NVEmbedding(256, EMB_SIZE, torch.float32, LT.LinearUVM,
                                       gpu_cache_size=1 << 19, storage=mb,
                                       optimize_for_training=False, device=DEV)
    E.save_nve(model, str(tmp_path))
    meta = json.load(open(tmp_path / "metadata.json"))
    key = meta["layers"][0]["storage_ref"]
    registry = {}
    la = E.load_nve_layers(str(tmp_path), registry=registry)
    lb = E.load_nve_layers(str(tmp_path), registry=registry)
    assert la[0].storage is lb[0].storage is registry[key]
    fake = "mb-9999999999"
    meta["layers"][0]["storage_ref"] = fake
    meta["resources"]["memblocks"][fake] = meta["resources"]["memblocks"].pop(key)
    shutil.copy(tmp_path / "weights" / (key + ".nve"), tmp_path / "weights" / (fake + ".nve"))
    json.dump(meta, open(tmp_path / "metadata.json", "w"))
    lc = E.load_nve_layers(str(tmp_path), registry=registry, resource_remap={fake: key})
    assert lc[0].storage is la[0].storage


def test_embed_config_roundtrip(tmp_path):
    config = {"kernel_mode": 2, "logging_interval": 100, "kernel_mode_value_1": 7,
              "kernel_mode_value_2": 9, "max_modify_size": 1024, "default_row_index": 3,
              "default_embedding": []}
    emb = nve_layers.NVEmbedding(256, EMB_SIZE, torch.float32, LT.LinearUVM,
                                 gpu_cache_size=1 << 19, optimize_for_training=False, device=DEV,
                                 config=config)
    bag = nve_layers.NVEmbeddingBag(256, EMB_SIZE, torch.float32, LT.LinearUVM, "sum",
                                    gpu_cache_size=1 << 19, optimize_for_training=False,
                                    device=DEV, config=config)
    E.save_nve(Two(emb, bag), str(tmp_path))
    meta = json.load(open(tmp_path / "metadata.json"))
    assert all(l["config"] == config for l in meta["layers"])
    layers = E.load_nve_layers(str(tmp_path))
    assert len(layers) == 2
    for layer in layers:
        for k, v in config.items():
            assert getattr(layer.config, k) == v


def test_schema1_load(tmp_path):
    model = torch.nn.Module()
    model.emb = _emb()
    keys = torch.arange(16, dtype=torch.int64, device=DEV)
    expected = model.emb(keys)
    E.save_nve(model, str(tmp_path))
    meta = json.load(open(tmp_path / "metadata.json"))
    l0 = meta["layers"][0]
    v1 = {k: v for k, v in l0.items() if k != "storage_ref"}
    v1["memblock_type"] = meta["resources"]["memblocks"][l0["storage_ref"]]["type"]
    shutil.copy(tmp_path / "weights" / (l0["storage_ref"] + ".nve"), tmp_path / "weights" / "emb.nve")
    json.dump([v1], open(tmp_path / "metadata.json", "w"))
    del model
    layers = E.load_nve_layers(str(tmp_path))
    assert len(layers) == 1 and torch.equal(layers[0](keys), expected)


def test_geometry_mismatch_raises(tmp_path):
    E.save_nve(One(_emb()), str(tmp_path))
    meta = json.load(open(tmp_path / "metadata.json"))
    meta["resources"]["memblocks"][meta["layers"][0]["storage_ref"]]["num_rows"] = 9999
    json.dump(meta, open(tmp_path / "metadata.json", "w"))
    with pytest.raises(ValueError, match="num_rows"):
        E.load_nve_layers(str(tmp_path))

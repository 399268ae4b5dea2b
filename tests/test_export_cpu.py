"""CPU checks of pynve.torch.nve_export's metadata logic (no layer is built):
the User-block type resolution, the memory-block descriptor, descriptor
rebuilding errors and the schema-version gate, following the reference's
tests/python_binding/test_nve_export.py:640-703, 835-850 and 1032-1047."""
import json
import os

import pytest

torch = pytest.importorskip("torch")

from pynve import _lib, nve  # noqa: E402
from pynve.torch import nve_export as E  # noqa: E402
from pynve.torch.nve_layers import LayerType  # noqa: E402

G, U, H = LayerType.GPULayer, LayerType.LinearUVM, LayerType.HostLayer
MB = nve.MemBlockType


class _Stub:
    def __init__(self, layer_type, memblock_type):
        self.layer_type, self.memblock_type = layer_type, memblock_type
        self.id, self.embedding_size, self.num_embeddings = 0, 8, 1024
        self.data_type = torch.float32


def test_gcd_memblock_type():
    assert E._gcd_memblock_type({G}) == "Linear"
    assert E._gcd_memblock_type({U}) == "Managed"
    assert E._gcd_memblock_type({H}) == "Host"
    assert E._gcd_memblock_type({G, U}) == "Linear"
    assert E._gcd_memblock_type({H, U}) == "Managed"
    with pytest.warns(UserWarning, match="GPULayer and HostLayer"):
        assert E._gcd_memblock_type({G, H}) == "Managed"
    with pytest.warns(UserWarning, match="GPULayer and HostLayer"):
        assert E._gcd_memblock_type({G, H, U}) == "Managed"
    with pytest.raises(ValueError):
        E._gcd_memblock_type({LayerType.Hierarchical})


def test_descriptor_records_actual_type_and_rejects_mpi():
    for mb in (MB.NVL, MB.Managed, MB.Host, MB.Linear, MB.User):
        d = E._memblock_resource_descriptor(_Stub(U, mb))
        assert d == {"type": mb.name, "row_elements": 8, "num_rows": 1024, "dtype": "float32"}
    with pytest.raises(ValueError, match="Cannot serialize memblock of type"):
        E._memblock_resource_descriptor(_Stub(G, MB.MPI))


def test_build_memblock_unsupported_types():
    cfg = {"type": "MPI", "row_elements": 8, "num_rows": 64, "dtype": "float32"}
    with pytest.raises(ValueError, match="Cannot reconstruct memblock of type"):
        E._build_memblock_from_descriptor(cfg, 0, "cuda")
    with pytest.raises(_lib.NotImplementedInBuild):
        E._build_memblock_from_descriptor({**cfg, "type": "NVL"}, 0, "cuda")


def _write_meta(tmp_path, doc):
    with open(os.path.join(tmp_path, "metadata.json"), "w") as f:
        json.dump(doc, f)
    return str(tmp_path)


def test_future_version_raises(tmp_path):
    d = _write_meta(tmp_path, {"version": 102, "resources": {}, "layers": []})
    with pytest.raises(RuntimeError, match="schema version"):
        E.load_nve_layers(d, device=torch.device("cpu"))


def _entry(layer_type, ref="mb-1"):
    return {"id": 1, "module_path": "emb", "num_embeddings": 16, "embedding_size": 4,
            "dtype": "float32", "layer_type": layer_type, "gpu_cache_size": 1 << 20,
            "host_cache_size": 0, "optimize_for_training": False, "is_bag": False, "mode": None,
            "storage_ref": ref, "config": None}


def test_device_and_reference_errors(tmp_path):
    res = {"remote_ps": {}, "memblocks": {}}
    d = _write_meta(tmp_path, {"version": 2, "resources": res, "layers": [_entry("GPULayer")]})
    with pytest.raises(ValueError, match="requires a CUDA device"):
        E.load_nve_layers(d, device=torch.device("cpu"))
    d = _write_meta(tmp_path, {"version": 2, "resources": res,
                               "layers": [_entry("HostLayer", ref=None)]})
    with pytest.raises(ValueError, match="has no 'storage_ref'"):
        E.load_nve_layers(d, device=torch.device("cpu"))
    d = _write_meta(tmp_path, {"version": 2, "resources": res, "layers": [_entry("HostLayer")]})
    with pytest.raises(ValueError, match="not found in resources.memblocks"):
        E.load_nve_layers(d, device=torch.device("cpu"))


class _FakeLoader:
    """The two methods of AOTIModelPackageLoader that rebind_markers uses."""

    def __init__(self, fqns):
        self.fqns, self.calls = list(fqns), []

    def get_constant_fqns(self):
        return self.fqns

    def load_constants(self, mapping, use_inactive, check_full_update, user_managed):
        self.calls.append((dict(mapping), use_inactive, check_full_update, user_managed))


class _Layer:
    def __init__(self, path, marker):
        self._export_module_path, self.marker_tensor = path, marker


def test_rebind_markers_points_both_buffers_at_the_live_markers():
    m1, m2 = torch.tensor([7]), torch.tensor([9])
    layers = [_Layer("", m1), _Layer("tower.bag", m2)]
    fake = _FakeLoader(["marker_tensor", "tower.bag.marker_tensor", "dense.weight"])
    E.rebind_markers(fake, layers)
    # each marker, no copy, into the active and the inactive buffer, user-managed
    assert [(list(c[0]), c[1], c[2], c[3]) for c in fake.calls] == [
        (["marker_tensor"], False, False, True), (["marker_tensor"], True, False, True),
        (["tower.bag.marker_tensor"], False, False, True), (["tower.bag.marker_tensor"], True, False, True)]
    assert fake.calls[0][0]["marker_tensor"] is m1 and fake.calls[3][0]["tower.bag.marker_tensor"] is m2
    # a package whose marker was folded away cannot be rebound
    with pytest.raises(RuntimeError, match="no replaceable constant 'tower.bag.marker_tensor'"):
        E.rebind_markers(_FakeLoader(["marker_tensor"]), layers)


def test_export_aot_keeps_markers_replaceable(tmp_path, monkeypatch):
    """export_aot turns runtime constant folding on unless the caller says
    otherwise, and packages the exported program as save_dir/model.pt2."""
    seen = {}
    monkeypatch.setattr(E, "save_nve", lambda model, save_dir, ps_data_paths=None: seen.setdefault("saved", save_dir))
    monkeypatch.setattr(E, "HAS_TORCH_OPS", True)
    monkeypatch.setattr(E, "_require_torch_ops", lambda name: None)
    monkeypatch.setattr(torch.export, "export", lambda m, a, dynamic_shapes=None: ("program", m, a, dynamic_shapes))
    monkeypatch.setattr(torch._inductor, "aoti_compile_and_package",
                        lambda prog, package_path, inductor_configs: seen.update(
                            prog=prog, path=package_path, cfg=inductor_configs))
    model = object()
    E.export_aot(model, (1,), str(tmp_path))
    assert seen["saved"] == str(tmp_path) and seen["path"] == os.path.join(str(tmp_path), "model.pt2")
    assert seen["prog"] == ("program", model, (1,), None)
    assert seen["cfg"] == {"aot_inductor.use_runtime_constant_folding": True}
    E.export_aot(model, (1,), str(tmp_path), inductor_configs={"max_autotune": True,
                                                              "aot_inductor.use_runtime_constant_folding": False})
    assert seen["cfg"] == {"max_autotune": True, "aot_inductor.use_runtime_constant_folding": False}

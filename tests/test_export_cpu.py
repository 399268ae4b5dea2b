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


def test_aot_entry_points_say_not_in_build():
    with pytest.raises(_lib.NotImplementedInBuild):
        E.export_aot(None, (), "/nonexistent")
    with pytest.raises(_lib.NotImplementedInBuild):
        E.load_aot("/nonexistent")

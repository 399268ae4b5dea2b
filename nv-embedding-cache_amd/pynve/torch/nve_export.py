"""Saving and reloading models with NVE layers (python/pynve/torch/nve_export.py).

A save directory holds, as the reference writes it (nve_export.py:16-40):

    save_dir/metadata.json      schema 2: {"version": 2, "resources":
                                {"remote_ps": {}, "memblocks": {key: descriptor}},
                                "layers": [per-layer entry, ...]}
    save_dir/weights/<key>.nve  one .nve table file per storage resource
    save_dir/model.pt2          torch.export program (export) or AOTInductor
                                package (export_aot)

A memory-block descriptor is {"type", "row_elements", "num_rows", "dtype"};
a layer entry is {"id", "module_path", "num_embeddings", "embedding_size",
"dtype", "layer_type", "gpu_cache_size", "host_cache_size",
"optimize_for_training", "is_bag", "mode", "storage_ref", "config"}.  Schema-1
files (a bare list of layer entries, weights named after the module path) load
too.  The graph dispatches through each layer's marker tensor, so loading
rebuilds the layers first and then points the loaded graph's marker buffers at
the new layers' markers (nve_export.py:700-738).

Parameter-server storage (Hierarchical layers), NVL / MPI memory blocks and
the host layer are not part of this build: exporting or loading them raises
NotImplementedInBuild.
"""
import builtins
import json
import os
import warnings

import torch

from .. import _lib
from .. import nve as _nve_mod
from . import HAS_TORCH_OPS
from .nve_layers import (LayerType, NVEmbedding, NVEmbeddingBag, NVEmbeddingBase,
                         torch_type_to_nve_type)

METADATA_SCHEMA_VERSION = 2
_MB = _nve_mod.MemBlockType


def _require_torch_ops(func_name):
    if not HAS_TORCH_OPS:
        raise RuntimeError(f"{func_name} needs the nve_ops custom ops (pynve.torch)")


def _dtype_str(data_type):
    return str(data_type).split(".", 1)[-1]


def _parse_dtype(dtype_str):
    return getattr(torch, dtype_str.split(".", 1)[-1])


def _nve_modules(model):
    return [(name, m) for name, m in model.named_modules() if isinstance(m, NVEmbeddingBase)]


def _gcd_memblock_type(layer_types):
    """The block type to rebuild a caller-owned (User) block as, from the
    layer types sharing it (nve_export.py:72-113): device-only users get a
    Linear block, users that need host access a Managed one, host-only users a
    Host block; a block used by both a GPU layer and a host layer becomes
    Managed with a warning."""
    G, U, H = LayerType.GPULayer, LayerType.LinearUVM, LayerType.HostLayer
    types = frozenset(layer_types)
    if types in (frozenset({G}), frozenset({G, U})):
        return _MB.Linear.name
    if types == frozenset({H}):
        return _MB.Host.name
    if types in (frozenset({U}), frozenset({U, H})):
        return _MB.Managed.name
    if types in (frozenset({G, H}), frozenset({G, U, H})):
        warnings.warn(f"UserMemBlock shared by both GPULayer and HostLayer "
                      f"({sorted(t.name for t in types)}); promoting to Managed", stacklevel=2)
        return _MB.Managed.name
    raise ValueError(f"Unexpected layer types combination: {set(types)}")


def _memblock_resource_descriptor(module):
    """Descriptor of a layer's memory block (nve_export.py:116-139): its own
    type and the layer's geometry, no device ids."""
    if module.memblock_type not in (_MB.User, _MB.NVL, _MB.Host, _MB.Linear, _MB.Managed):
        raise ValueError(f"Cannot serialize memblock of type {module.memblock_type.name!r}; "
                         "supported types are NVL, Host, Linear, Managed")
    return {"type": module.memblock_type.name, "row_elements": module.embedding_size,
            "num_rows": module.num_embeddings, "dtype": _dtype_str(module.data_type)}


def _collect_resources(model, *, ps_data_paths=None):
    """(resources, {id(storage): key}, {module path: key}) of a model
    (nve_export.py:142-198).  Keys are "mb-<id>" for memory blocks and
    "ps-<id>" for parameter servers, so layers sharing a block share a key."""
    resources = {"remote_ps": {}, "memblocks": {}}
    obj_to_key, refs, user_types = {}, {}, {}
    for name, module in _nve_modules(model):
        storage = getattr(module, "storage", None)
        if storage is None:
            continue
        oid = builtins.id(storage)
        if isinstance(storage, _nve_mod.MemBlock):
            if oid not in obj_to_key:
                obj_to_key[oid] = f"mb-{oid}"
                resources["memblocks"][obj_to_key[oid]] = _memblock_resource_descriptor(module)
            if module.memblock_type == _MB.User:
                user_types.setdefault(obj_to_key[oid], set()).add(module.layer_type)
        else:
            if not hasattr(storage, "export_config"):
                raise ValueError(f"Layer '{name}' has a storage object with no export_config() "
                                 "method")
            if oid not in obj_to_key:
                obj_to_key[oid] = f"ps-{oid}"
                resources["remote_ps"][obj_to_key[oid]] = storage.export_config()
            if ps_data_paths and name in ps_data_paths:
                keys_path, values_path = ps_data_paths[name]
                resources["remote_ps"][obj_to_key[oid]]["remote_ps_data"] = {
                    "keys": keys_path, "values": values_path}
        refs[name] = obj_to_key[oid]
    for key, types in user_types.items():
        resources["memblocks"][key]["type"] = _gcd_memblock_type(types)
    return resources, obj_to_key, refs


def _export_metadata(model, save_dir, *, ps_data_paths=None):
    resources, obj_to_key, refs = _collect_resources(model, ps_data_paths=ps_data_paths)
    layers = [{
        "id": m.id,
        "module_path": name,
        "num_embeddings": m.num_embeddings,
        "embedding_size": m.embedding_size,
        "dtype": _dtype_str(m.data_type),
        "layer_type": m.layer_type.name,
        "gpu_cache_size": m.gpu_cache_size,
        "host_cache_size": m.host_cache_size,
        "optimize_for_training": m.optimize_for_training,
        "is_bag": isinstance(m, NVEmbeddingBag),
        "mode": getattr(m, "mode", None),
        "storage_ref": refs.get(name),
        "config": json.loads(m.config.to_json()),
    } for name, m in _nve_modules(model)]
    doc = {"version": METADATA_SCHEMA_VERSION, "resources": resources, "layers": layers}
    with open(os.path.join(save_dir, "metadata.json"), "w") as f:
        json.dump(doc, f, indent=2)
    return doc, obj_to_key


def _export_weights(model, save_dir, obj_to_key=None):
    """One .nve file per memory block, written by the first layer that uses it,
    its entry named by that layer's id (nve_export.py:238-276)."""
    weights_dir = os.path.join(save_dir, "weights")
    os.makedirs(weights_dir, exist_ok=True)
    written = set()
    for name, module in _nve_modules(model):
        mb = getattr(module, "storage", None)
        if not isinstance(mb, _nve_mod.MemBlock):
            continue
        key = obj_to_key.get(builtins.id(mb)) if obj_to_key is not None else None
        filename = (key or name.replace(".", "_")) + ".nve"
        if filename in written:
            continue
        written.add(filename)
        with open(os.path.join(weights_dir, filename), "wb") as f:
            _nve_mod.TensorFileFormat().write_table_file_header(f)
            _nve_mod.write_tensor_to_stream(module.emb_layer, f, module.id)


def save_nve(model, save_dir, *, ps_data_paths=None):
    """metadata.json and weights/ of every NVE layer of `model`."""
    os.makedirs(save_dir, exist_ok=True)
    _, obj_to_key = _export_metadata(model, save_dir, ps_data_paths=ps_data_paths)
    _export_weights(model, save_dir, obj_to_key=obj_to_key)


def export(model, example_inputs, save_dir, *, dynamic_shapes=None, ps_data_paths=None):
    """save_nve plus the torch.export program of `model` as model.pt2."""
    _require_torch_ops("export")
    save_nve(model, save_dir, ps_data_paths=ps_data_paths)
    exported = torch.export.export(model, example_inputs, dynamic_shapes=dynamic_shapes)
    torch.export.save(exported, os.path.join(save_dir, "model.pt2"))


# The package must keep each layer's marker as a constant that can be replaced
# after loading (AOTInductor otherwise folds a buffer into the compiled code and
# leaves nothing to point at the rebuilt layer): runtime constant folding keeps
# constants in the package's constant table.
_AOT_KEEP_CONSTANTS = {"aot_inductor.use_runtime_constant_folding": True}


def export_aot(model, example_inputs, save_dir, *, dynamic_shapes=None, inductor_configs=None,
               ps_data_paths=None):
    """save_nve plus an AOTInductor package of `model` as model.pt2
    (nve_export.py:321-360), loadable by `load_aot` here or by a C++ host
    through torch::inductor::AOTIModelPackageLoader and nve::LayerDirectory
    (include/nve_loader.hpp).  `inductor_configs` entries override the
    defaults, the constant-folding switch included (a package built without it
    cannot be pointed at new layers)."""
    _require_torch_ops("export_aot")
    save_nve(model, save_dir, ps_data_paths=ps_data_paths)
    configs = {**_AOT_KEEP_CONSTANTS, **(inductor_configs or {})}
    program = torch.export.export(model, example_inputs, dynamic_shapes=dynamic_shapes)
    torch._inductor.aoti_compile_and_package(program, package_path=os.path.join(save_dir, "model.pt2"),
                                             inductor_configs=configs)


def _device_index(device):
    if device is None:
        return torch.cuda.current_device()
    device = torch.device(device)
    if device.type == "cpu":
        return -1
    return device.index if device.index is not None else torch.cuda.current_device()


def load_aot(save_dir, *, gpu_cache_size_override=None, device=None):
    """(loader, layers) of an `export_aot` directory (nve_export.py:741-800):
    the layers rebuilt with their weights, and an AOTIModelPackageLoader whose
    marker constants are the new layers' markers, so `loader.run(inputs)`
    reaches them.  The loader holds the markers without owning them: keep
    `layers` alive while the loader runs."""
    _require_torch_ops("load_aot")
    from torch._C._aoti import AOTIModelPackageLoader

    index = _device_index(device)
    layers = load_nve_layers(save_dir, gpu_cache_size_override=gpu_cache_size_override,
                             device=torch.device("cpu") if index < 0 else torch.device("cuda", index))
    loader = AOTIModelPackageLoader(os.path.join(save_dir, "model.pt2"), "model", False, 1, index)
    rebind_markers(loader, layers)
    return loader, layers


def rebind_markers(loader, layers):
    """Point each layer's marker constant of `loader` at the layer's
    marker_tensor, in both of the package's constant buffers and without a
    copy (nve_export.py:801; idempotent).  load_aot calls it; call it again
    after the package's constants were replaced (a constant-buffer swap copies
    the markers, and the ops know only the registered tensors)."""
    known = set(loader.get_constant_fqns())
    for layer in layers:
        fqn = _marker_fqn(layer._export_module_path)
        if fqn not in known:
            raise RuntimeError(f"the package has no replaceable constant '{fqn}' (it holds {sorted(known)}): "
                               "it was not built by export_aot, which keeps runtime constant folding on")
        for inactive in (False, True):
            loader.load_constants({fqn: layer.marker_tensor}, inactive, False, True)


def _build_ps_from_config(ps_config):
    raise _lib.NotImplementedInBuild(_lib.NOT_IMPLEMENTED,
                                     "parameter-server storage (Hierarchical layers) is not part of "
                                     "this build")


def _build_memblock_from_descriptor(mb_cfg, device_index, device_type, nvl_devices_override=None):
    """A new memory block for a descriptor (nve_export.py:384-415)."""
    kind = mb_cfg["type"]
    rows, width = mb_cfg["num_rows"], mb_cfg["row_elements"]
    dt = torch_type_to_nve_type(_parse_dtype(mb_cfg["dtype"]))
    if kind == _MB.NVL.name:
        return _nve_mod.NVLMemBlock(width, rows, dt, nvl_devices_override or [])
    if kind == _MB.Host.name or device_type == "cpu":
        return _nve_mod.HostMemBlock(width, rows, dt)
    if kind == _MB.Linear.name:
        gpus = _nve_mod.resolve_memblock_devices(_MB.Linear, device_index, [])
        if not gpus:
            raise RuntimeError("Unable to resolve gpu_ids check machine configuration")
        return _nve_mod.LinearMemBlock(width, rows, dt, gpus[0])
    if kind == _MB.Managed.name:
        return _nve_mod.ManagedMemBlock(width, rows, dt,
                                        _nve_mod.resolve_memblock_devices(_MB.Managed, device_index,
                                                                          []))
    raise ValueError(f"Cannot reconstruct memblock of type {kind!r}; supported types are NVL, "
                     "Host, Linear, Managed")


def _make_layer(num_emb, emb_size, data_type, layer_type, gpu_cache_size, host_cache_size,
                optimize_for_training, device, layer_id, mode, is_bag, *, storage=None,
                config=None):
    kw = dict(optimize_for_training=optimize_for_training, device=device, id=layer_id,
              config=config)
    if layer_type in (LayerType.LinearUVM, LayerType.Hierarchical):
        kw["gpu_cache_size"] = gpu_cache_size
    if layer_type == LayerType.Hierarchical:
        kw["host_cache_size"] = host_cache_size
    if storage is not None:
        kw["storage"] = storage
    if is_bag:
        return NVEmbeddingBag(num_emb, emb_size, data_type, layer_type, mode, **kw)
    return NVEmbedding(num_emb, emb_size, data_type, layer_type, **kw)


def _entry_fields(entry, gpu_cache_size_override):
    return dict(
        num_emb=entry["num_embeddings"], emb_size=entry["embedding_size"],
        data_type=_parse_dtype(entry["dtype"]), layer_type=LayerType[entry["layer_type"]],
        gpu_cache_size=(entry["gpu_cache_size"] if gpu_cache_size_override is None
                        else gpu_cache_size_override),
        host_cache_size=entry.get("host_cache_size", 0),
        optimize_for_training=entry["optimize_for_training"], device=None,
        layer_id=entry["id"], mode=entry.get("mode"), is_bag=entry.get("is_bag", False))


def _check_device(layer_type, device, module_path):
    if device.type == "cpu" and layer_type != LayerType.HostLayer:
        raise ValueError(f"load_nve_layers: layer '{module_path}' is {layer_type.name}, which "
                         "requires a CUDA device, but device='cpu' was requested.")


def _load_weights(layer, path):
    with open(path, "rb") as f:
        layer.load_from_stream(f)


def load_nve_layers(save_dir, *, gpu_cache_size_override=None, device=None, registry=None,
                    resource_remap=None, nvl_devices_override=None):
    """Rebuild the NVE layers of a save directory with their weights
    (nve_export.py:418-672); returns them in file order, each with
    `_export_module_path` set.  `registry` ({resource key: storage}) carries
    built storage across calls so that exports of one process share it;
    `resource_remap` renames keys before the registry is consulted."""
    _require_torch_ops("load_nve_layers")
    if device is None:
        device = (torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available()
                  else torch.device("cpu"))
    elif device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    device_index = device.index if device.type == "cuda" else -1
    with open(os.path.join(save_dir, "metadata.json")) as f:
        doc = json.load(f)
    weights_dir = os.path.join(save_dir, "weights")

    if isinstance(doc, list):  # schema 1
        layers = []
        for entry in doc:
            fields = _entry_fields(entry, gpu_cache_size_override)
            fields["device"] = device
            _check_device(fields["layer_type"], device, entry["module_path"])
            lt = fields["layer_type"]
            if lt == LayerType.Hierarchical:
                layer = _make_layer(**fields, storage=_build_ps_from_config(
                    entry.get("remote_ps_config")), config=entry.get("config"))
            elif lt in (LayerType.LinearUVM, LayerType.GPULayer, LayerType.HostLayer):
                storage = None
                if lt == LayerType.HostLayer:
                    dt = torch_type_to_nve_type(fields["data_type"])
                    storage = (_nve_mod.HostMemBlock(fields["emb_size"], fields["num_emb"], dt)
                               if device.type == "cpu" else
                               _nve_mod.ManagedMemBlock(fields["emb_size"], fields["num_emb"], dt,
                                                        [device_index]))
                fields["host_cache_size"] = 0
                layer = _make_layer(**fields, storage=storage, config=entry.get("config"))
                _load_weights(layer, os.path.join(
                    weights_dir, entry["module_path"].replace(".", "_") + ".nve"))
            else:
                raise NotImplementedError(f"load_nve_layers: layer_type '{lt.name}' not yet "
                                          "supported")
            layer._export_module_path = entry["module_path"]
            layers.append(layer)
        return layers

    version = doc.get("version", 1)
    if version > METADATA_SCHEMA_VERSION:
        raise RuntimeError(f"metadata.json was exported with schema version {version}, but this "
                           f"runtime supports up to version {METADATA_SCHEMA_VERSION}")
    registry = {} if registry is None else registry
    remap = resource_remap or {}
    resources = doc.get("resources", {})
    mb_res = resources.get("memblocks", {})
    ps_res = resources.get("remote_ps", {})

    def check_geometry(key, num_emb, emb_size):
        cfg = mb_res.get(key)
        if not cfg:
            return
        if cfg["row_elements"] != emb_size:
            raise ValueError(f"Resource '{key}' row_elements={cfg['row_elements']} != layer "
                             f"embedding_size={emb_size}")
        if cfg["num_rows"] != num_emb:
            raise ValueError(f"Resource '{key}' num_rows={cfg['num_rows']} != layer "
                             f"num_embeddings={num_emb}")

    layers = []
    for entry in doc["layers"]:
        path = entry["module_path"]
        fields = _entry_fields(entry, gpu_cache_size_override)
        fields["device"] = device
        lt = fields["layer_type"]
        _check_device(lt, device, path)
        ref = entry.get("storage_ref")
        if lt == LayerType.Hierarchical:
            if not ref:
                raise ValueError(f"Hierarchical layer '{path}' is missing 'storage_ref'.")
            key = remap.get(ref, ref)
            if key not in registry:
                if key not in ps_res:
                    raise ValueError(f"storage_ref '{key}' not found in resources.remote_ps.")
                registry[key] = _build_ps_from_config(ps_res[key])
            layer = _make_layer(**fields, storage=registry[key], config=entry.get("config"))
        elif lt in (LayerType.LinearUVM, LayerType.GPULayer, LayerType.HostLayer):
            if not ref:
                raise ValueError(f"v2 metadata: layer '{path}' has no 'storage_ref'. Every layer "
                                 "in a v2 export must reference a resource.")
            key = remap.get(ref, ref)
            fresh = key not in registry
            if fresh and key not in mb_res:
                raise ValueError(f"storage_ref '{key}' not found in resources.memblocks.")
            check_geometry(key, fields["num_emb"], fields["emb_size"])
            if fresh:
                registry[key] = _build_memblock_from_descriptor(mb_res[key], device_index,
                                                                device.type, nvl_devices_override)
            fields["host_cache_size"] = 0
            layer = _make_layer(**fields, storage=registry[key], config=entry.get("config"))
            if fresh:  # a registry hit is already filled
                _load_weights(layer, os.path.join(weights_dir, ref + ".nve"))
        else:
            raise NotImplementedError(f"load_nve_layers: layer_type '{lt.name}' not yet supported")
        layer._export_module_path = path
        layers.append(layer)
    return layers


def _marker_fqn(module_path):
    return f"{module_path}.marker_tensor" if module_path else "marker_tensor"


def load(save_dir, *, gpu_cache_size_override=None, device=None):
    """(module, layers) of an `export` directory (nve_export.py:700-738): the
    layers rebuilt with their weights, and the loaded program's module with
    each layer's marker buffer replaced by the live layer's marker tensor, so
    the ops find the new layers.  Keep `layers` alive while using `module`."""
    layers = load_nve_layers(save_dir, gpu_cache_size_override=gpu_cache_size_override,
                             device=device)
    module = torch.export.load(os.path.join(save_dir, "model.pt2")).module()
    for layer in layers:
        path = layer._export_module_path
        sub = module.get_submodule(path) if path else module
        sub.marker_tensor = layer.marker_tensor
    return module, layers

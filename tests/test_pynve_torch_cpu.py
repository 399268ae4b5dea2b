"""CPU checks of the Python surface (pynve.nve, pynve.torch): enums, config
plumbing, forward-input validation, constructor validation that precedes any
device work, op schemas and their shape inference.  Mirrors the validation
cases of the reference's tests/python_binding/test_pytorch.py."""
import json

import pytest

torch = pytest.importorskip("torch")

from pynve import _lib, nve  # noqa: E402
from pynve.torch import nve_layers, nve_ops  # noqa: E402


def test_enum_values_match_the_c_abi():
    assert int(nve.DataType_t.Float32) == _lib.DT_F32
    assert int(nve.DataType_t.Float16) == _lib.DT_F16
    assert int(nve.PoolingType_t.Concatenate) == _lib.POOL_CONCAT
    assert int(nve.PoolingType_t.WeightedMean) == _lib.POOL_WMEAN
    assert [m.name for m in nve.MemBlockType] == ["Linear", "NVL", "MPI", "Managed", "User", "Host"]
    assert [m.value for m in nve_layers.LayerType] == [1, 2, 3, 4]


def test_embed_layer_config_defaults_and_json():
    c = nve.EmbedLayerConfig()
    d = json.loads(c.to_json())
    assert d == {"logging_interval": -1, "kernel_mode": 0, "kernel_mode_value_1": 0,
                 "kernel_mode_value_2": 0, "max_modify_size": 0, "default_row_index": -1,
                 "default_embedding": []}
    c2 = nve_layers.config_to_nve_config({"kernel_mode": 3, "default_row_index": 5,
                                          "default_embedding": torch.ones(2, dtype=torch.float16)})
    assert c2.kernel_mode == 3 and c2.default_row_index == 5
    assert c2.default_embedding == [0, 60, 0, 60]  # 1.0 in fp16 = 0x3c00, little endian


def test_pooling_type_from_mode():
    assert nve_ops.pooling_type_from_mode("sum", False) == nve.PoolingType_t.Sum
    assert nve_ops.pooling_type_from_mode("sum", True) == nve.PoolingType_t.WeightedSum
    assert nve_ops.pooling_type_from_mode("mean", False) == nve.PoolingType_t.Mean
    assert nve_ops.pooling_type_from_mode("mean", True) == nve.PoolingType_t.WeightedMean
    for bad in ("max", "concat", "SUM"):
        with pytest.raises(ValueError):
            nve_ops.pooling_type_from_mode(bad, False)


def test_forward_input_checks():
    k = torch.arange(6, dtype=torch.int64)
    off = torch.tensor([0, 3, 6])
    nve_layers._check_forward_inputs(k, off, torch.ones(6))
    with pytest.raises(TypeError):  # int32 keys
        nve_layers._check_forward_inputs(k.int())
    with pytest.raises(ValueError):  # a strided view
        nve_layers._check_forward_inputs(torch.arange(12)[::2])
    with pytest.raises(TypeError):  # int32 offsets
        nve_layers._check_forward_inputs(k, off.int())
    with pytest.raises(ValueError):  # fewer than num_bags + 1 >= 2 offsets
        nve_layers._check_forward_inputs(k, torch.tensor([0]))
    with pytest.raises(TypeError):  # float64 weights
        nve_layers._check_forward_inputs(k, off, torch.ones(6, dtype=torch.float64))
    with pytest.raises(ValueError):  # not one weight per key
        nve_layers._check_forward_inputs(k, off, torch.ones(5))


def test_constructor_validation_before_device_work():
    LT = nve_layers.LayerType
    cases = [
        dict(args=(10, 4, torch.float32, LT.GPULayer, "max"), bag=True),  # no 'max' kernel
        dict(args=(10, 4, torch.float32, LT.GPULayer), kw=dict(device="cpu")),  # GPU layer on the host
        dict(args=(10, 4, torch.bfloat16, LT.GPULayer)),  # not a table dtype
        dict(args=(10, 4, torch.float32, LT.GPULayer), kw=dict(config={"default_embedding": torch.zeros(4)})),
        dict(args=(10, 4, torch.float32, LT.GPULayer),
             kw=dict(config={"default_embedding": torch.zeros(2, dtype=torch.float64)})),
        dict(args=(10, 4, torch.float32, LT.GPULayer), kw=dict(config={"default_embedding": torch.zeros(3)})),
        dict(args=(10, 4, torch.float32, LT.HostLayer), kw=dict(device="cpu")),  # trainable host layer
        dict(args=(10, 4, torch.float32, LT.HostLayer),
             kw=dict(device="cpu", optimize_for_training=False, storage="not a block")),
    ]
    for c in cases:
        cls = nve_layers.NVEmbeddingBag if c.get("bag") else nve_layers.NVEmbedding
        with pytest.raises(ValueError):
            cls(*c["args"], **c.get("kw", {}))
    with pytest.raises(NotImplementedError):
        nve_layers.NVEmbedding(10, 4, torch.float32, LT.Hierarchical, gpu_cache_size=1 << 20, device="cuda:0")


def test_ops_are_registered_with_the_reference_schemas():
    s1 = str(torch.ops.nve_ops.embedding_lookup.default._schema)
    s2 = str(torch.ops.nve_ops.embedding_lookup_with_pooling.default._schema)
    assert s1 == "nve_ops::embedding_lookup(Tensor marker, Tensor keys, int embedding_size, int dtype) -> Tensor"
    assert s2 == ("nve_ops::embedding_lookup_with_pooling(Tensor marker, Tensor keys, Tensor offsets, "
                  "Tensor? weights, int pooling_type, int embedding_size, int dtype) -> Tensor")


def test_fake_kernels_infer_shape_and_dtype():
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        marker = torch.empty(1, dtype=torch.int64)
        keys = torch.empty(37, dtype=torch.int64)
        off = torch.empty(9, dtype=torch.int64)
        out = torch.ops.nve_ops.embedding_lookup(marker, keys, 24, int(nve.DataType_t.Float16))
        assert tuple(out.shape) == (37, 24) and out.dtype == torch.float16
        out = torch.ops.nve_ops.embedding_lookup_with_pooling(marker, keys, off, None, 1, 16,
                                                              int(nve.DataType_t.Float32))
        assert tuple(out.shape) == (8, 16) and out.dtype == torch.float32


def test_cpu_ops_need_a_registered_layer():
    with pytest.raises(RuntimeError):
        torch.ops.nve_ops.embedding_lookup(torch.zeros(1, dtype=torch.int64),
                                           torch.zeros(3, dtype=torch.int64), 4, 1)


def test_registry():
    with pytest.raises(RuntimeError, match="no binding registered"):
        nve.get_binding(0xdead0)
    sentinel = object()
    nve.register_for_torch(0xbeef0, sentinel)
    assert nve.get_binding(0xbeef0) is sentinel
    nve.unregister_from_torch(0xbeef0)
    with pytest.raises(RuntimeError):
        nve.get_binding(0xbeef0)


def test_unbuilt_layers_and_memblocks_raise():
    for cls in (nve.HierarchicalEmbedding, nve.NVLMemBlock, nve.MPIMemBlock):
        with pytest.raises(NotImplementedError, match="not part of this build"):
            cls()


def test_user_memblock():
    mb = nve.UserMemBlock(0x1000, 64)
    assert mb.get_type() == nve.MemBlockType.User
    assert mb.get_ptr() == 0x1000 and mb.get_size_in_bytes() == 64
    assert nve.dtype_size(nve.DataType_t.Float16) == 2


def test_cached_table_binding_is_required_and_stays_out_of_pickles():
    import io
    import pickle

    from pynve.torch.nve_tensors import CachedTable

    class Binding:  # stands for a native layer binding: not picklable
        def __reduce__(self):
            raise TypeError("native handle")

    with pytest.raises(TypeError):
        CachedTable(torch.zeros(2, 3))  # cache= is a required keyword
    with pytest.raises(_lib.InvalidArgument):
        CachedTable(torch.zeros(2, 3), cache=None)
    b = Binding()
    w = CachedTable(torch.arange(6.0).reshape(2, 3), cache=b)
    assert isinstance(w, torch.nn.Parameter) and w.requires_grad and w.emb_layer is b
    assert w.__getstate__()["emb_layer"] is None
    buf = io.BytesIO()
    torch.save({"w": w}, buf)  # would raise if the binding were pickled
    assert w.emb_layer is b  # the live parameter keeps its binding
    buf.seek(0)
    back = torch.load(buf, weights_only=False)["w"]  # written by this test itself
    assert torch.equal(back.detach(), w.detach())
    with pytest.raises(TypeError):
        pickle.dumps(b)
    with pytest.raises(_lib.InvalidArgument):
        w.add_(torch.ones(2, 3))  # dense updates are not row updates

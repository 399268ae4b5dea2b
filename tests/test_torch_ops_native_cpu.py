"""The nve_ops torch library is native (libnve_torch_ops.so, the reference's
torch_binding.cpp:85-92 with its implementations in nve_torch_ops.cu:67-146 and
nve_torch_ops_cpu.cpp:59-133): the dispatcher's kernels for both keys are C++,
the library exports its registry, and a lookup through the op reaches the C
ABI (hit rates logged at the perf level every logging_interval lookups, as
binding_layers.hpp:370-387 does).  Host layers only: no GPU needed."""
import ctypes
import os
import subprocess
import sys

import pytest

torch = pytest.importorskip("torch")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
OPS = os.path.join(ROOT, "nv-embedding-cache_amd", "libnve_torch_ops.so")


def test_library_exports_its_registry():
    lib = ctypes.CDLL(OPS)
    for name in ("nve_torch_ops_register", "nve_torch_ops_unregister", "nve_torch_ops_release_layer",
                 "nve_torch_ops_num_contexts"):
        assert hasattr(lib, name), name


def test_ops_have_native_kernels_for_both_keys():
    import pynve.torch  # noqa: F401  (loads the library)
    for op in ("embedding_lookup", "embedding_lookup_with_pooling"):
        dump = torch._C._dispatch_dump(f"nve_ops::{op}")
        for key in ("CPU", "CUDA"):
            line = [s for s in dump.splitlines() if s.startswith(f"{key}:")]
            assert line, (op, key, dump)
            assert "nve_torch_ops.cpp" in line[0], (op, key, line[0])  # registered from C++, not Python


def test_register_rejects_bad_arguments():
    lib = ctypes.CDLL(OPS)
    reg = lib.nve_torch_ops_register
    reg.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
                    ctypes.c_int64]
    reg.restype = ctypes.c_int32
    assert reg(None, 0x1000, 64, 1, None, -1) != 0      # no marker
    assert reg(0x2000, None, 64, 1, None, -1) != 0      # no layer
    assert reg(0x2000, 0x1000, 0, 1, None, -1) != 0     # no row
    assert reg(0x2000, 0x1000, 64, 7, None, -1) != 0    # rows neither float32 nor float16
    assert lib.nve_torch_ops_unregister(ctypes.c_void_p(0x2000)) == 0  # unknown marker: nothing to do


SNIPPET = r"""
import sys, torch
sys.path.insert(0, {pkg!r})
from pynve.torch import nve_layers
LT = nve_layers.LayerType
init = torch.arange(40 * 4, dtype=torch.float32).reshape(40, 4)
bag = nve_layers.NVEmbeddingBag(40, 4, torch.float32, LT.HostLayer, "sum", weight_init=init,
                                optimize_for_training=False, device="cpu",
                                config={{"logging_interval": 2}})
keys = torch.tensor([1, 2, 3, 39], dtype=torch.int64)
off = torch.tensor([0, 2, 4], dtype=torch.int64)
for _ in range(3):
    out = bag(keys, off)
assert torch.equal(out, torch.stack([init[1] + init[2], init[3] + init[39]]))
print("OK", flush=True)
"""


def test_op_lookups_log_hit_rates_at_perf_level():
    env = dict(os.environ, NVE_LOG_LEVEL="PERF")
    code = SNIPPET.format(pkg=os.path.join(ROOT, "nv-embedding-cache_amd"))
    p = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, env=env, timeout=300)
    assert p.returncode == 0, p.stderr
    lines = [s for s in p.stdout.splitlines() if "Hit rates:" in s]
    assert len(lines) == 2 and all("][P] Hit rates: " in s for s in lines), p.stdout  # lookups 0 and 2 of 3
    assert "OK" in p.stdout


def _host_bag():
    from pynve.torch import nve_layers
    init = torch.arange(40 * 4, dtype=torch.float32).reshape(40, 4)
    return nve_layers.NVEmbeddingBag(40, 4, torch.float32, nve_layers.LayerType.HostLayer, "sum",
                                     weight_init=init, optimize_for_training=False, device="cpu"), init


def test_op_checks_and_status_mapping():
    """The C++ ops check their tensors (nve_torch_ops_checks.hpp:27-45 in the
    reference) and map the C ABI's status to Python exceptions: an invalid
    argument is a ValueError, any other failure a RuntimeError."""
    bag, init = _host_bag()
    m = bag.marker_tensor
    keys = torch.tensor([1, 2, 3, 39], dtype=torch.int64)
    off = torch.tensor([0, 2, 4], dtype=torch.int64)
    op = torch.ops.nve_ops.embedding_lookup_with_pooling
    out = op(m, keys, off, None, 1, 4, 1)
    assert torch.equal(out, torch.stack([init[1] + init[2], init[3] + init[39]]))
    with pytest.raises(RuntimeError, match="int64"):
        op(m, keys.int(), off, None, 1, 4, 1)
    with pytest.raises(RuntimeError, match="contiguous"):
        op(m, torch.arange(8, dtype=torch.int64)[::2], off, None, 1, 4, 1)
    with pytest.raises(RuntimeError, match="num_bags"):
        op(m, keys, off[:1], None, 1, 4, 1)
    with pytest.raises(RuntimeError, match="float32 or float16"):
        op(m, keys, off, torch.ones(4, dtype=torch.float64), 3, 4, 1)
    with pytest.raises(RuntimeError, match="one per key"):
        op(m, keys, off, torch.ones(3), 3, 4, 1)
    with pytest.raises(ValueError, match="invalid argument"):  # the C ABI rejects the pooling type
        op(m, keys, off, None, 77, 4, 1)
    # weighted sum through the op, weights of the table's dtype
    w = torch.tensor([1.0, 0.5, 2.0, 0.25])
    out = op(m, keys, off, w, 3, 4, 1)
    assert torch.equal(out, torch.stack([init[1] + 0.5 * init[2], 2.0 * init[3] + 0.25 * init[39]]))
    rows = torch.ops.nve_ops.embedding_lookup(m, keys, 4, 1)
    assert torch.equal(rows, init[keys])


def test_unregistered_marker_after_the_layer_is_gone():
    import gc
    bag, _ = _host_bag()
    m = bag.marker_tensor
    keys = torch.tensor([1], dtype=torch.int64)
    assert torch.ops.nve_ops.embedding_lookup(m, keys, 4, 1).shape == (1, 4)
    marker_copy = m.clone()  # a tensor at another address was never registered
    with pytest.raises(RuntimeError, match="no binding registered"):
        torch.ops.nve_ops.embedding_lookup(marker_copy, keys, 4, 1)
    del bag
    gc.collect()
    with pytest.raises(RuntimeError, match="no binding registered"):
        torch.ops.nve_ops.embedding_lookup(m, keys, 4, 1)

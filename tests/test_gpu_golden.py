"""The HIP library against the committed golden fixtures
(tests/golden/fixtures.npz; tests/test_golden_cpu.py pins them with numpy):
pooled find-and-pool over a linear table (find_and_pool.cuh:103-132), dedup
(deduper.cuh:136-221) and pooling backprop (gradient_calculator.cuh:238-301),
through the C ABI.  Dyadic data makes every sum exact, so the bar is bit
equality; mean pooling (a quotient) is held to 1e-5 relative."""
import numpy as np
import pytest

from nve_helpers import rel_close, to_dev
from oracle import oracle as O
from pynve import _lib
from test_gpu_backprop import gpu_backprop
from test_gpu_dedup import gpu_dedup
from test_gpu_find_and_pool import CDT, fap
from test_golden_cpu import cases, get

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", cases("pool_"))
def test_pool_fixture(name):
    vdt, odt, sparse, pooling, rows, dim, bags, hot = (int(x) for x in get(name, "params"))
    want = get(name, "out_bits")
    tb, keys, off, w = get(name, "table"), get(name, "keys"), get(name, "offsets"), get(name, "weights")
    oes = 2 if odt == O.F16 else 4
    out = torch.zeros((bags, dim * oes), dtype=torch.uint8, device="cuda")
    fap(to_dev(keys), keys.size, to_dev(tb.reshape(-1)), rows, tb.shape[1], CDT[vdt], pooling,
        _lib.SPARSE_CSR if sparse == O.CSR else _lib.SPARSE_FIXED, None if off is None else to_dev(off),
        0 if off is None else off.size, hot, None if w is None else to_dev(w),
        0 if w is None else _lib.DT_F32, CDT[odt], out, dim * oes,
        key_type=_lib.KEY_INT32 if keys.dtype == np.int32 else _lib.KEY_INT64)
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16 if odt == O.F16 else np.float32).reshape(bags, dim)
    if pooling == O.MEAN:
        assert rel_close(got, want.view(np.float32), 1e-5)
    else:
        assert np.array_equal(got.view(want.dtype), want)


@pytest.mark.parametrize("name", cases("dedup_"))
def test_dedup_fixture(name):
    u, uq, ct, inv, off = gpu_dedup(get(name, "keys"))
    assert u == get(name, "unique").size
    assert np.array_equal(uq, get(name, "unique"))
    assert np.array_equal(ct, get(name, "counts"))
    assert np.array_equal(inv, get(name, "inverse"))
    assert np.array_equal(off, get(name, "offsets"))


@pytest.mark.parametrize("name", cases("bwd_"))
def test_backprop_fixture(name):
    sparse, gdt, bags, hot, dim = (int(x) for x in get(name, "params"))
    uq, grad = gpu_backprop(get(name, "keys"), O.SUM, sparse, get(name, "offsets"), hot, None, O.F32,
                            get(name, "grads_in_bits"), gdt, dim)
    assert np.array_equal(uq, get(name, "unique"))
    assert np.array_equal(grad, get(name, "grad_bits"))

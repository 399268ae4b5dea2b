"""The allocation-free entry point nve_amd_dedup_gather_noalloc against the
entry it varies, nve_amd_dedup_gather (caller workspace), through the C ABI:
two calls in a row on the same GPU scratch, the second with a smaller batch,
each bit-identical to the workspace variant's output and to the rows
themselves; batches above the maximum are rejected before any GPU work."""
import ctypes

import numpy as np
import pytest

from nve_helpers import stream_ptr, vp
from pynve import _lib

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def with_workspace(keys, table, rows, width):
    n = keys.numel()
    wsb = ctypes.c_uint64()
    _lib.call("nve_amd_dedup_workspace_size", n, ctypes.byref(wsb))
    ws = torch.empty(int(wsb.value), dtype=torch.uint8, device="cuda")
    out = torch.full((n, width // 2), -7.0, dtype=torch.float16, device="cuda")
    _lib.call("nve_amd_dedup_gather", _lib.KEY_INT64, n, vp(keys), vp(table), rows, width, vp(out), width, vp(ws),
              wsb.value, stream_ptr())
    torch.cuda.synchronize()
    return out


def no_alloc(keys, table, rows, width):
    n = keys.numel()
    out = torch.full((n, width // 2), -7.0, dtype=torch.float16, device="cuda")
    _lib.call("nve_amd_dedup_gather_noalloc", _lib.KEY_INT64, n, vp(keys), vp(table), rows, width, vp(out), width,
              stream_ptr())
    torch.cuda.synchronize()
    return out


def test_two_calls_match_the_workspace_entry():
    rows, dim = 300_000, 128
    width = dim * 2
    g = torch.Generator(device="cuda")
    g.manual_seed(17)
    table = torch.randn((rows, dim), device="cuda", generator=g).half()
    # a large Zipf-like batch (many repeats, keys outside the table), then a smaller one
    big = (torch.randint(0, rows, (262144,), device="cuda", generator=g) ** 2 // rows).to(torch.int64)
    big[::97] = rows + 5  # outside the table: output rows stay as they were
    small = torch.randint(0, 1000, (5000,), device="cuda", generator=g, dtype=torch.int64)
    for keys in (big, small):
        print(f"[no_alloc] {keys.numel()} keys", flush=True)
        got = no_alloc(keys, table, rows, width)
        ref = with_workspace(keys, table, rows, width)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
        inside = keys < rows
        assert torch.equal(got[inside].view(torch.int16), table[keys[inside]].view(torch.int16))
        assert torch.all(got[~inside] == -7.0)


def test_rejects_batches_above_the_maximum():
    keys = torch.zeros(262145, dtype=torch.int64, device="cuda")
    table = torch.zeros((10, 8), dtype=torch.float16, device="cuda")
    out = torch.zeros((262145, 8), dtype=torch.float16, device="cuda")
    with pytest.raises(_lib.InvalidArgument):
        _lib.call("nve_amd_dedup_gather_noalloc", _lib.KEY_INT64, keys.numel(), vp(keys), vp(table), 10, 16,
                  vp(out), 16, stream_ptr())


def test_calls_on_two_streams_are_ordered():
    """Two calls issued back to back on two streams, with no synchronization
    between them, share the GPU's scratch array: the library orders the second
    after the first, so both match the workspace entry.  Then a third call on
    the first stream, again without a sync, ordered after the second."""
    rows, dim = 200_000, 64
    width = dim * 2
    g = torch.Generator(device="cuda")
    g.manual_seed(23)
    table = torch.randn((rows, dim), device="cuda", generator=g).half()
    batches = [(torch.randint(0, rows, (n,), device="cuda", generator=g) ** 2 // rows).to(torch.int64)
               for n in (262144, 200000, 150000)]
    refs = [with_workspace(k, table, rows, width) for k in batches]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [torch.full((k.numel(), dim), -7.0, dtype=torch.float16, device="cuda") for k in batches]
    torch.cuda.synchronize()
    print("[no_alloc] three calls on two streams", flush=True)
    for k, o, s in zip(batches, outs, (s1, s2, s1)):
        _lib.call("nve_amd_dedup_gather_noalloc", _lib.KEY_INT64, k.numel(), vp(k), vp(table), rows, width, vp(o),
                  width, ctypes.c_void_p(s.cuda_stream))
    torch.cuda.synchronize()
    for o, r in zip(outs, refs):
        assert torch.equal(o.view(torch.int16), r.view(torch.int16))

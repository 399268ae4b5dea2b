"""Shared helpers of the parity tests: table builders, device plumbing, and
oracle wrappers.  The oracle (oracle/) is the checker; the code under test is
libnve_amd.so, reached through its C ABI."""
import ctypes

import numpy as np

from oracle import oracle as O

try:
    import torch
except ImportError:  # pragma: no cover
    torch = None


def vp(t):
    """ctypes void* of a torch tensor (device or host) or None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_ptr():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def to_dev(a):
    """numpy array -> torch cuda tensor with the same bytes."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint64:
        a = a.view(np.int64)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    return torch.from_numpy(a.copy()).cuda()


def from_dev(t, np_dtype):
    return t.cpu().numpy().view(np_dtype)


# ---------------------------------------------------------------------------
# tables
# ---------------------------------------------------------------------------
def dyadic(rng, shape):
    """Values nom / 2^e, nom in [-8, 8], e in [3, 9]: the fixture of the
    reference's kernel tests (tests/kernels/kernel_test_common.cuh AllocateTable),
    so fp32 sums of up to thousands of them are exact in any order."""
    nom = rng.integers(-8, 9, size=shape).astype(np.float64)
    e = rng.integers(3, 10, size=shape).astype(np.float64)
    return nom / np.exp2(e)


def float_table(rng, rows, dim, dtype, dyadic_values=True):
    """Returns the table as raw bytes (rows, row_bytes) uint8."""
    v = dyadic(rng, (rows, dim)) if dyadic_values else rng.normal(0, 0.02, size=(rows, dim))
    if dtype == O.F32:
        return v.astype(np.float32).view(np.uint8).reshape(rows, dim * 4)
    return v.astype(np.float16).view(np.uint8).reshape(rows, dim * 2)


def quant_table(rng, rows, count, dtype):
    """Rowwise-quantized rows: values then scale (and offset), as stored bytes."""
    meta = O.meta_bytes(dtype)
    out = np.zeros((rows, count + meta), np.uint8)
    if dtype in (O.QI8_F32, O.QI8_F16, O.XI8A_F32):
        q = rng.integers(-127, 128, size=(rows, count)).astype(np.int8).view(np.uint8)
    elif dtype == O.XE4M3_F32:
        q = rng.integers(0, 256, size=(rows, count)).astype(np.uint8)
        q[(q & 0x7F) == 0x7F] = 0x3C  # no NaN codes in table data
    else:
        q = rng.integers(0, 256, size=(rows, count)).astype(np.uint8)
    out[:, :count] = q
    scale = np.exp(rng.uniform(np.log(1e-3), np.log(1e-1), size=rows))
    offset = rng.normal(0, 0.01, size=rows)
    if dtype in (O.QI8_F32, O.XE4M3_F32):
        out[:, count:count + 4] = scale.astype(np.float32).view(np.uint8).reshape(rows, 4)
    elif dtype in (O.QU8_F32, O.XI8A_F32):
        out[:, count:count + 4] = scale.astype(np.float32).view(np.uint8).reshape(rows, 4)
        out[:, count + 4:count + 8] = offset.astype(np.float32).view(np.uint8).reshape(rows, 4)
    elif dtype == O.QI8_F16:
        out[:, count:count + 2] = scale.astype(np.float16).view(np.uint8).reshape(rows, 2)
    elif dtype == O.QU8_F16:
        out[:, count:count + 2] = scale.astype(np.float16).view(np.uint8).reshape(rows, 2)
        out[:, count + 2:count + 4] = offset.astype(np.float16).view(np.uint8).reshape(rows, 2)
    return out


def csr_offsets(rng, bags, max_len, dtype=np.int64, allow_empty=True):
    lens = rng.integers(0 if allow_empty else 1, max_len + 1, size=bags)
    off = np.zeros(bags + 1, dtype)
    off[1:] = np.cumsum(lens)
    return off


def oracle_pool(table_bytes, keys, dtype, count, sparse, pooling, offsets, bags, hotness,
                weights, weight_dtype, out_dtype, host_order=False):
    tb = np.ascontiguousarray(table_bytes).reshape(-1)
    row_bytes = table_bytes.shape[1]
    ptrs = O.linear_row_ptrs(keys, tb, row_bytes)
    return O.pool(ptrs, dtype, count, sparse, pooling, keys.size, offsets, bags, hotness, weights,
                  weight_dtype, out_dtype, host_order=host_order,
                  key_bytes=np.dtype(keys.dtype).itemsize)


def oracle_dequant(table_bytes, keys, dtype, count, out_dtype):
    rows = np.ascontiguousarray(table_bytes[keys.astype(np.int64)])
    return O.dequant_rows(rows, dtype, count, out_dtype)


def rel_close(got, ref, rtol=1e-5, atol_scale=None):
    """|got - ref| <= rtol * max(|ref|, scale) elementwise, scale defaulting to
    the row's max |ref| (pooled sums of mixed-sign values can land near 0)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    if atol_scale is None:
        atol_scale = np.max(np.abs(ref), axis=-1, keepdims=True) if ref.ndim else abs(ref)
    return np.all(np.abs(got - ref) <= rtol * np.maximum(np.abs(ref), atol_scale) + 1e-30)


def f16_ulp_close(got_bits, ref_bits, ulps=1):
    """fp16 results within `ulps` units in the last place (as ordered integers)."""
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    return np.all(np.abs(ordered(got_bits) - ordered(ref_bits)) <= ulps)


def pooled_f16_close(got_bits, ref_bits, rtol=1e-5):
    """fp16 pooled outputs: each element within 1 fp16 ulp of the oracle, or
    within rtol of the row's largest magnitude (fp32 accumulation order may
    differ from the oracle's near zero, where an fp16 ulp is tiny)."""
    def ordered(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, 0x8000 - (b & 0x7FFF), 0x8000 + b)
    ulp_ok = np.abs(ordered(got_bits) - ordered(ref_bits)) <= 1
    g = got_bits.view(np.float16).astype(np.float64)
    r = ref_bits.view(np.float16).astype(np.float64)
    scale = np.max(np.abs(r), axis=-1, keepdims=True)
    return bool(np.all(ulp_ok | (np.abs(g - r) <= rtol * scale)))


_hip = None


def hip_memcpy(dst, src, nbytes):
    """hipMemcpy(dst, src, n, hipMemcpyDefault) on raw addresses (test plumbing)."""
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.restype = ctypes.c_int
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    rc = _hip.hipMemcpy(ctypes.c_void_p(dst), ctypes.c_void_p(src), nbytes, 4)
    assert rc == 0, f"hipMemcpy failed: {rc}"
    # from pageable memory hipMemcpy may return once the source is staged, before
    # the device has the bytes; kernels on other streams must not start earlier
    assert _hip.hipDeviceSynchronize() == 0

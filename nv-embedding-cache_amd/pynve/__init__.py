"""pynve for MI355X: Python surface of the HIP lookup library (libnve_amd.so).

Mirrors the reference's `pynve` package (python/pynve/): `pynve.nve` exposes
the layer bindings that take raw device pointers and a stream, and
`pynve.torch.nve_layers` the torch modules.  Both call the C ABI of
libnve_amd.so; there is no CPU fallback -- loading fails loudly when the
library has not been built.
"""
from . import _lib  # noqa: F401

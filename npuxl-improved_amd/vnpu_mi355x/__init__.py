"""Python side of the MI355X vnpu backend.

The product is the C-ABI shared library ``lib/libvnpu.so`` (HIP, gfx950);
this package only binds that ABI with ctypes (``abi``), drives it
(``runtime.Session``) and generates the benchmark's seeded synthetic inputs
(``synth``).
"""
from . import abi
from .runtime import BACKEND_LIB, Buffer, Session, VnpuError, load_backend, load_library

__all__ = ["abi", "BACKEND_LIB", "Buffer", "Session", "VnpuError", "load_backend", "load_library"]

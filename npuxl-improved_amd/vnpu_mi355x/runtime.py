"""Thin Python driver for any library that exports the vnpu C ABI.

``Session`` opens a device and a stream through ``vnpu_device_create`` /
``vnpu_stream_create`` and moves numpy arrays in and out with
``vnpu_buffer_alloc`` / ``vnpu_buffer_copy``.  Against this repository's
``libvnpu.so`` the buffers are HBM; against the reference build
(``libvnpu_ref.so``) the very same calls use host memory - which is what lets
one harness drive both backends with identical inputs.

The MI355X backend fails loudly: ``load_backend`` raises if the shared
library is missing, and ``Session`` raises if no GPU device can be created.
There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from . import abi

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
BACKEND_LIB = os.path.join(ROOT, "lib", "libvnpu.so")


class VnpuError(RuntimeError):
    def __init__(self, what: str, status: int):
        super().__init__(f"{what} failed with status {status}")
        self.status = status


def load_library(path: str) -> C.CDLL:
    if not os.path.exists(path):
        raise FileNotFoundError(f"vnpu library not built: {path}")
    lib = C.CDLL(path, mode=C.RTLD_LOCAL)
    return abi.bind(lib)


def load_backend() -> C.CDLL:
    """The MI355X backend (HIP); raises if it has not been built."""
    return load_library(BACKEND_LIB)


@dataclass
class Buffer:
    handle: C.c_void_p
    ptr: int
    nbytes: int


class Session:
    """One device + one stream on a vnpu library."""

    def __init__(self, lib: C.CDLL | str | None = None, config: abi.Config | None = None):
        if lib is None:
            lib = load_backend()
        elif isinstance(lib, str):
            lib = load_library(lib)
        self.lib = lib
        self.dev = C.c_void_p()
        rc = lib.vnpu_device_create(C.byref(config) if config is not None else None, C.byref(self.dev))
        if rc != abi.OK:
            raise VnpuError("vnpu_device_create", rc)
        self.stream = C.c_void_p()
        rc = lib.vnpu_stream_create(self.dev, 0, C.byref(self.stream))
        if rc != abi.OK:
            lib.vnpu_device_destroy(self.dev)
            raise VnpuError("vnpu_stream_create", rc)
        self._buffers: list[Buffer] = []
        self._packed: list[C.c_void_p] = []

    # -- lifecycle -----------------------------------------------------
    def close(self) -> None:
        if self.dev is None:
            return
        self.lib.vnpu_stream_sync(self.stream)
        for w in self._packed:
            self.lib.vnpu_packed_weights_destroy(w)
        for b in self._buffers:
            self.lib.vnpu_buffer_free(b.handle)
        self._packed.clear()
        self._buffers.clear()
        self.lib.vnpu_stream_destroy(self.stream)
        self.lib.vnpu_device_destroy(self.dev)
        self.dev = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> abi.DeviceInfo:
        info = abi.DeviceInfo()
        self.check("vnpu_device_get_info", self.lib.vnpu_device_get_info(self.dev, C.byref(info)))
        return info

    def status(self) -> abi.DeviceStatus:
        st = abi.DeviceStatus()
        self.check("vnpu_device_get_status", self.lib.vnpu_device_get_status(self.dev, C.byref(st)))
        return st

    @staticmethod
    def check(what: str, rc: int) -> None:
        if rc != abi.OK:
            raise VnpuError(what, rc)

    # -- memory --------------------------------------------------------
    def alloc(self, nbytes: int) -> Buffer:
        h = C.c_void_p()
        self.check("vnpu_buffer_alloc", self.lib.vnpu_buffer_alloc(self.dev, max(1, int(nbytes)), C.byref(h)))
        ptr = self.lib.vnpu_buffer_host_ptr(h)
        b = Buffer(h, int(ptr), int(nbytes))
        self._buffers.append(b)
        return b

    def free(self, b: Buffer) -> None:
        self.lib.vnpu_buffer_free(b.handle)
        self._buffers = [x for x in self._buffers if x is not b]

    def upload(self, arr: np.ndarray) -> Buffer:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes)
        if arr.nbytes:
            self.check("vnpu_buffer_copy", self.lib.vnpu_buffer_copy(
                self.stream, C.c_void_p(b.ptr), arr.ctypes.data_as(C.c_void_p), arr.nbytes, abi.COPY_H2D))
        return b

    def write(self, b: Buffer, arr: np.ndarray, offset: int = 0) -> None:
        arr = np.ascontiguousarray(arr)
        assert offset + arr.nbytes <= b.nbytes
        self.check("vnpu_buffer_copy", self.lib.vnpu_buffer_copy(
            self.stream, C.c_void_p(b.ptr + offset), arr.ctypes.data_as(C.c_void_p), arr.nbytes, abi.COPY_H2D))

    def download(self, b: Buffer | int, dtype, shape, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        ptr = b.ptr if isinstance(b, Buffer) else int(b)
        if out.nbytes:
            self.check("vnpu_buffer_copy", self.lib.vnpu_buffer_copy(
                self.stream, out.ctypes.data_as(C.c_void_p), C.c_void_p(ptr + offset), out.nbytes, abi.COPY_D2H))
        return out

    # -- commands ------------------------------------------------------
    @staticmethod
    def command(opcode: int, flags: int = 0, id: int = 0, **fields) -> abi.Command:
        cmd = abi.Command()
        cmd.opcode = opcode
        cmd.flags = flags
        cmd.id = id
        if opcode in abi.OP_FIELD:
            name, _ = abi.OP_FIELD[opcode]
            args = getattr(cmd.args, name)
            for k, v in fields.items():
                if isinstance(v, Buffer):
                    v = v.ptr
                setattr(args, k, v)
        return cmd

    def submit(self, cmds, event: C.c_void_p | None = None) -> int:
        arr = (abi.Command * len(cmds))(*cmds)
        return self.lib.vnpu_stream_submit(self.stream, arr, len(cmds), event)

    def sync(self) -> int:
        return self.lib.vnpu_stream_sync(self.stream)

    def run(self, opcode: int, flags: int = 0, **fields) -> None:
        """Submit one command and synchronize; raise on any failure."""
        self.check("vnpu_stream_submit", self.submit([self.command(opcode, flags, **fields)]))
        self.check("vnpu_stream_sync", self.sync())

    def pack(self, B: Buffer | np.ndarray, K: int, N: int, scales=None, ldb: int = 0,
             trans_b: int = 0, tile_mask=None, mask_ld: int = 0) -> C.c_void_p:
        """PACK_WEIGHTS_I8; with tile_mask (uint8 [ceil(K/64), >= ceil(N/64)],
        or a device Buffer with mask_ld), vnpu_pack_weights_i8_masked: the
        64 x 64 weight tiles whose byte is zero are packed as zeros."""
        if isinstance(B, np.ndarray):
            B = np.ascontiguousarray(B, dtype=np.int8)
            bptr = B.ctypes.data_as(C.c_void_p)
        else:
            bptr = C.c_void_p(B.ptr)
        if scales is None:
            sptr = None
        elif isinstance(scales, Buffer):
            sptr = C.c_void_p(scales.ptr)
        else:
            scales = np.ascontiguousarray(scales, dtype=np.float32)
            sptr = scales.ctypes.data_as(C.c_void_p)
        w = C.c_void_p()
        if tile_mask is None:
            self.check("vnpu_pack_weights_i8", self.lib.vnpu_pack_weights_i8(
                self.dev, bptr, sptr, K, N, ldb, trans_b, C.byref(w)))
        else:
            if isinstance(tile_mask, Buffer):
                mptr = C.c_void_p(tile_mask.ptr)
            else:
                tile_mask = np.ascontiguousarray(tile_mask, dtype=np.uint8)
                mask_ld = mask_ld or tile_mask.shape[1]
                mptr = tile_mask.ctypes.data_as(C.c_void_p)
            self.check("vnpu_pack_weights_i8_masked", self.lib.vnpu_pack_weights_i8_masked(
                self.dev, bptr, sptr, K, N, ldb, trans_b, mptr, mask_ld, C.byref(w)))
        self._packed.append(w)
        return w

    def unpack_info(self, w: C.c_void_p):
        K, N, nbytes = C.c_uint32(), C.c_uint32(), C.c_uint64()
        sc, cs = C.POINTER(C.c_float)(), C.POINTER(C.c_int32)()
        self.check("vnpu_packed_weights_info", self.lib.vnpu_packed_weights_info(
            w, C.byref(K), C.byref(N), C.byref(nbytes), C.byref(sc), C.byref(cs)))
        n = N.value
        return (K.value, n, nbytes.value, np.ctypeslib.as_array(sc, (n,)).copy(),
                np.ctypeslib.as_array(cs, (n,)).copy())

    def release_packed(self, w: C.c_void_p) -> None:
        self.lib.vnpu_packed_weights_destroy(w)
        self._packed = [x for x in self._packed if x is not w]

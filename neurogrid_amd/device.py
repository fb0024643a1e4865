"""Raw device buffers over the C ABI, for tests, smoke and bench.

A :class:`DeviceBuffer` is memory from ``cuda_malloc`` that numpy arrays are
copied into and out of bit for bit (through the int8 copy entry points, which
move raw bytes). 16-bit floats travel as ``uint16`` bit patterns so that the
exact fp16/bf16 values reach the kernels unchanged.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from ._lib import load


class DeviceError(RuntimeError):
    pass


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise DeviceError(f"{what} returned {rc}")


class DeviceBuffer:
    def __init__(self, nbytes: int):
        self.lib = load()
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(self.lib.cuda_malloc(C.byref(p), max(self.nbytes, 1)), f"cuda_malloc({self.nbytes})")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        if a.nbytes > self.nbytes:
            raise DeviceError(f"upload of {a.nbytes} bytes into a {self.nbytes}-byte buffer")
        if a.nbytes:
            check(self.lib.cuda_copy_int8_to_device(C.c_void_p(self.ptr), a.ctypes.data, a.nbytes), "upload")

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise DeviceError(f"download of {out.nbytes} bytes from a {self.nbytes}-byte buffer")
        if out.nbytes:
            check(self.lib.cuda_sync_device(), "cuda_sync_device")
            check(self.lib.cuda_copy_int8_to_host(out.ctypes.data, C.c_void_p(self.ptr), out.nbytes), "download")
        return out

    @property
    def vp(self) -> C.c_void_p:
        return C.c_void_p(self.ptr)

    @property
    def ip(self):
        return C.cast(C.c_void_p(self.ptr), C.POINTER(C.c_int))

    def offset(self, nbytes: int) -> C.c_void_p:
        return C.c_void_p(self.ptr + nbytes)

    def free(self) -> None:
        if self.ptr is not None:
            self.lib.cuda_free(C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync() -> None:
    check(load().cuda_sync_device(), "cuda_sync_device")

"""Helpers for the GPU parity tests: move numpy arrays through the C ABI and
compare with the oracle to the stated bars (bit-exact for integer/byte work
and exactly-rounded ops; |d| <= 1e-2 or |d| <= 2 ulp for transcendental ones).
"""
from __future__ import annotations

import ctypes as C
import sys

import numpy as np

from neurogrid_amd.device import DeviceBuffer, sync


def banner(msg: str) -> None:
    """Name the case before a GPU step, so a crash can be attributed."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def dev(a: np.ndarray) -> DeviceBuffer:
    return DeviceBuffer.from_array(np.ascontiguousarray(a))


def empty(nbytes: int) -> DeviceBuffer:
    return DeviceBuffer(nbytes)


def get(buf: DeviceBuffer, dtype, shape) -> np.ndarray:
    return buf.download(dtype, shape)


def ok(rc: int, what: str = "call") -> None:
    assert rc == 0, f"{what} returned {rc}"


def f32(bits: np.ndarray, dtype: str) -> np.ndarray:
    bits = np.asarray(bits, np.uint16)
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def ulp(ref: np.ndarray, dtype: str) -> np.ndarray:
    v = np.abs(np.asarray(ref, np.float64))
    if dtype == "bf16":
        return 2.0 ** (np.floor(np.log2(np.maximum(v, 2.0 ** -126))) - 7)
    return 2.0 ** (np.floor(np.log2(np.maximum(v, 2.0 ** -14))) - 10)


def assert_close16(got_bits, ref_bits, dtype: str, what: str = "") -> float:
    """|d| <= 1e-2 or |d| <= 2 ulp(ref); NaN only where the oracle has NaN.
    Returns the fraction of bit-identical elements."""
    g = f32(got_bits, dtype).astype(np.float64)
    r = f32(ref_bits, dtype).astype(np.float64)
    nan_r = np.isnan(r)
    assert (np.isnan(g) == nan_r).all(), f"{what}: NaN pattern differs"
    g, r = g[~nan_r], r[~nan_r]
    inf = np.isinf(r)
    assert (g[inf] == r[inf]).all(), f"{what}: inf differs"
    d = np.abs(g[~inf] - r[~inf])
    bad = ~((d <= 1e-2) | (d <= 2 * ulp(r[~inf], dtype)))
    assert not bad.any(), f"{what}: {bad.sum()} elements outside tolerance, max |d| {d.max()}"
    return float((np.asarray(got_bits) == np.asarray(ref_bits)).mean())


def assert_bits_equal(got, ref, what: str = "") -> None:
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    neq = got != ref
    if neq.any():
        idx = np.argwhere(neq)[:5]
        raise AssertionError(f"{what}: {neq.sum()} of {neq.size} differ; first at {idx.tolist()}: "
                             f"got {got[tuple(idx[0])]} want {ref[tuple(idx[0])]}")


__all__ = ["banner", "dev", "empty", "get", "ok", "f32", "ulp", "assert_close16", "assert_bits_equal", "sync", "C",
           "HipRuntime"]


class HipRuntime:
    """The few HIP runtime calls the graph-capture test needs (ctypes)."""

    def __init__(self):
        vp = C.c_void_p
        self.h = C.CDLL("libamdhip64.so")
        self.h.hipStreamBeginCapture.argtypes = [vp, C.c_int]
        self.h.hipStreamEndCapture.argtypes = [vp, C.POINTER(vp)]
        self.h.hipGraphInstantiate.argtypes = [C.POINTER(vp), vp, vp, vp, C.c_size_t]
        self.h.hipGraphLaunch.argtypes = [vp, vp]
        self.h.hipGraphExecDestroy.argtypes = [vp]
        self.h.hipGraphDestroy.argtypes = [vp]
        self.h.hipStreamSynchronize.argtypes = [vp]
        self.h.hipStreamDestroy.argtypes = [vp]

    def check(self, rc, what):
        assert rc == 0, f"{what} failed with hipError {rc}"

    def stream(self):
        s = C.c_void_p()
        self.check(self.h.hipStreamCreate(C.byref(s)), "hipStreamCreate")
        return s

    def capture(self, stream, fn):
        """Capture the launches `fn` makes on `stream` (relaxed mode); returns (graph, exec)."""
        self.check(self.h.hipStreamBeginCapture(stream, 2), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = C.c_void_p()
            rc = self.h.hipStreamEndCapture(stream, C.byref(g))
        self.check(rc, "hipStreamEndCapture")
        ex = C.c_void_p()
        self.check(self.h.hipGraphInstantiate(C.byref(ex), g, None, None, 0), "hipGraphInstantiate")
        return g, ex

    def launch(self, ex, stream):
        self.check(self.h.hipGraphLaunch(ex, stream), "hipGraphLaunch")
        self.check(self.h.hipStreamSynchronize(stream), "hipStreamSynchronize")

    def destroy(self, g, ex):
        self.h.hipGraphExecDestroy(ex)
        self.h.hipGraphDestroy(g)

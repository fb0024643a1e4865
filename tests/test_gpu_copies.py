"""The dtype-converting copies of memory.h (memory.cu:145-213): fp32 on the
host, fp16 on the device (dtype code 1).

Up to 64 K elements the library converts on the host; larger copies go
through a device buffer in chunks of 4 M elements and convert on the device.
Both halves must give the same bits, checked against closed forms:
- host -> device: round to nearest even (numpy's float32 -> float16 cast, a
  correctly rounded IEEE conversion), NaN as sign | 0x7e00;
- device -> host: exact (numpy's float16 -> float32 cast), a NaN's payload
  kept as is: sign | 0x7f800000 | (mantissa << 13), quiet bit not forced.
Sizes cover the switch-over (65 536 host, 65 537 device) and more than one
chunk (4 M + 4 099).
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import assert_bits_equal, banner, empty, get, ok

# numpy's float32 -> float16 casts of values beyond the fp16 range give inf,
# the expected result, and warn about it.
pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore:overflow encountered in cast:RuntimeWarning")]

RNG = np.random.Generator(np.random.PCG64(77))
SIZES = [1000, 65536, 65537, 1 << 20, (1 << 22) + 4099]


def f32_inputs(n):
    """Midpoints between neighbouring fp16 values (ties), specials, NaN
    payloads, the overflow and underflow edges, then random values."""
    finite = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    mids = (finite[:-1] + finite[1:]) / np.float32(2)
    nan_bits = np.array([0x7F800001, 0x7FC00000, 0xFFC12345, 0x7FBFFFFF, 0xFF800001, 0x7FFFFFFF], np.uint32)
    edges = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.996, 65520.0, -65520.0, 2.0 ** -25,
                      np.nextafter(np.float32(2.0 ** -25), np.float32(1)), 2.0 ** -24, 3.0e38], np.float32)
    pool = np.concatenate([mids, -mids, nan_bits.view(np.float32), edges])
    rest = (RNG.standard_normal(n) * np.float32(100)).astype(np.float32)
    x = np.concatenate([pool, rest])[:n] if n >= pool.size else pool[RNG.choice(pool.size, n, replace=False)]
    return np.ascontiguousarray(x[RNG.permutation(n)])


def want_f16(x):
    bits = x.view(np.uint32)
    out = x.astype(np.float16).view(np.uint16).copy()
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    out[nan] = ((bits[nan] >> 16) & 0x8000) | 0x7E00
    return out


def want_f32_bits(h):
    h = h.astype(np.uint32)
    out = h.astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32).copy()
    nan = ((h & 0x7C00) == 0x7C00) & ((h & 0x3FF) != 0)
    out[nan] = ((h[nan] & 0x8000) << 16) | 0x7F800000 | ((h[nan] & 0x3FF) << 13)
    return out


@pytest.mark.parametrize("n", SIZES)
def test_copy_to_device_fp32_to_fp16(lib, n):
    banner(f"cuda_copy_to_device dtype 1 n={n}")
    x = f32_inputs(n)
    d = empty(2 * n)
    ok(lib.cuda_copy_to_device(d.vp, x.ctypes.data, n, 1), "cuda_copy_to_device")
    assert_bits_equal(get(d, np.uint16, (n,)), want_f16(x), "fp16 bits")


@pytest.mark.parametrize("n", SIZES)
def test_copy_to_host_fp16_to_fp32(lib, n):
    banner(f"cuda_copy_to_host dtype 1 n={n}")
    h = np.resize(np.arange(65536, dtype=np.uint32).astype(np.uint16), n)   # every pattern, repeated
    h = h[RNG.permutation(n)]
    d = empty(2 * n)
    ok(lib.cuda_copy_int8_to_device(d.vp, h.ctypes.data, 2 * n), "upload")
    out = np.empty(n, np.float32)
    ok(lib.cuda_copy_to_host(out.ctypes.data, d.vp, n, 1), "cuda_copy_to_host")
    assert_bits_equal(out.view(np.uint32), want_f32_bits(h), "fp32 bits")


def test_copy_round_trip_large(lib):
    """Through the device and back: every fp16 value survives unchanged."""
    banner("copy round trip 3 M")
    n = 3 * (1 << 20) + 5
    h = np.resize(np.arange(0x7C00, dtype=np.uint16), n)
    x = h.view(np.float16).astype(np.float32)
    x[1::2] *= -1
    d = empty(2 * n)
    ok(lib.cuda_copy_to_device(d.vp, x.ctypes.data, n, 1), "to device")
    back = np.empty(n, np.float32)
    ok(lib.cuda_copy_to_host(back.ctypes.data, d.vp, n, 1), "to host")
    assert_bits_equal(back.view(np.uint32), x.view(np.uint32), "round trip")

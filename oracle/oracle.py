"""numpy front end of the CPU oracle (oracle/ng_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker. The gfx950 product path never
imports it.

16-bit tensors are passed as ``uint16`` bit patterns; ``dtype`` selects
binary16 ("f16") or bfloat16 ("bf16") interpretation.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libng_oracle.so"

_u16p = C.POINTER(C.c_uint16)
_i8p = C.POINTER(C.c_int8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int)
_i, _f, _sz = C.c_int, C.c_float, C.c_size_t

_SIGS = {
    "ora_f16_to_f32": (C.c_float, [C.c_uint16]),
    "ora_f32_to_f16": (C.c_uint16, [C.c_float]),
    "ora_bf16_to_f32": (C.c_float, [C.c_uint16]),
    "ora_f32_to_bf16": (C.c_uint16, [C.c_float]),
    "ora_set_threads": (None, [_i]),
    "ora_get_threads": (_i, []),
    "ora_set_exact_only": (None, [_i]),
    "ora_sumsq": (C.c_float, [_f32p, _i]),
    "ora_rmsnorm": (None, [_u16p, _u16p, _u16p, _i, _i, _f, _i]),
    "ora_add_rmsnorm": (None, [_u16p, _u16p, _u16p, _u16p, _u16p, _i, _i, _f, _i]),
    "ora_rmsnorm_quant": (None, [_i8p, _f32p, _u16p, _u16p, _i, _i, _f]),
    "ora_add_rmsnorm_quant": (None, [_i8p, _f32p, _u16p, _u16p, _u16p, _u16p, _i, _i, _f]),
    "ora_quant_rows": (None, [_i8p, _f32p, _u16p, _i, _i]),
    "ora_quant_tensor": (None, [_i8p, _f32p, _u16p, _sz]),
    "ora_quant_cols": (None, [_i8p, _f32p, _u16p, _i, _i]),
    "ora_dequant": (None, [_u16p, _i8p, _f32p, _i, _i, _i]),
    "ora_elementwise": (None, [_u16p, _u16p, _u16p, _f, _sz, _i, _i]),
    "ora_rope_inv_freq": (None, [_f32p, _i, _f]),
    "ora_rope": (None, [_u16p, _u16p, _i32p, _i, _i, _i, _i, _f, _i]),
    "ora_gather": (None, [_u16p, _u16p, _i32p, _i, _i]),
    "ora_softmax": (None, [_u16p, _u16p, _i, _i]),
    "ora_rmsnorm_f32": (None, [_f32p, _f32p, _f32p, _i, _i, _f]),
    "ora_elementwise_f32": (None, [_f32p, _f32p, _f32p, _f, _sz, _i]),
    "ora_rope_f32": (None, [_f32p, _f32p, _i32p, _i, _i, _i, _i, _f]),
    "ora_gather_bytes": (None, [C.c_void_p, C.c_void_p, _i32p, _i, _sz]),
    "ora_bf16_to_f16_trunc": (None, [_u16p, _u16p, _sz]),
}

OPS = {"add": 0, "mul": 1, "silu": 2, "silu_mul": 3, "scale": 4}
DTYPES = {"f16": 0, "bf16": 1}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(t)


def _u16(a) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype in (np.float16,):
        a = a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a


# ------------------------------------------------------------------ conversions

def f32_to_bf16_bits(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    lower = b & 0xFFFF
    upper = (b >> 16).astype(np.uint32)
    up = (lower > 0x8000) | ((lower == 0x8000) & ((upper & 1) == 1))
    out = (upper + up.astype(np.uint32)) & 0xFFFF
    out = np.where(nan, (b >> 16) | 0x40, out)
    return out.astype(np.uint16)


def bf16_bits_to_f32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def f16_bits_to_f32(h) -> np.ndarray:
    return np.ascontiguousarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_f32(h, dtype: str) -> np.ndarray:
    return bf16_bits_to_f32(h) if dtype == "bf16" else f16_bits_to_f32(h)


def from_f32(x, dtype: str) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    if dtype == "bf16":
        return f32_to_bf16_bits(x)
    return x.astype(np.float16).view(np.uint16)


# ------------------------------------------------------------------ controls

def set_threads(n: int) -> None:
    lib().ora_set_threads(int(n))


def get_threads() -> int:
    return lib().ora_get_threads()


def set_exact_only(on: bool) -> None:
    lib().ora_set_exact_only(1 if on else 0)


def sumsq(v) -> float:
    v = np.ascontiguousarray(v, dtype=np.float32)
    return float(np.float32(lib().ora_sumsq(_p(v, _f32p), v.size)))


# ------------------------------------------------------------------ kernels

def rmsnorm(x, w, eps: float, dtype: str = "f16") -> np.ndarray:
    x, w = _u16(x), _u16(w)
    H = x.shape[-1]
    T = x.size // H
    y = np.empty_like(x)
    lib().ora_rmsnorm(_p(y, _u16p), _p(x, _u16p), _p(w, _u16p), T, H, eps, DTYPES[dtype])
    return y


def add_rmsnorm(x, res, w, eps: float, dtype: str = "f16"):
    x, res, w = _u16(x), _u16(res), _u16(w)
    H = x.shape[-1]
    T = x.size // H
    y = np.empty_like(x)
    ro = np.empty_like(x)
    lib().ora_add_rmsnorm(_p(y, _u16p), _p(ro, _u16p), _p(x, _u16p), _p(res, _u16p), _p(w, _u16p), T, H, eps,
                          DTYPES[dtype])
    return y, ro


def rmsnorm_quant(x, w, eps: float):
    x, w = _u16(x), _u16(w)
    H = x.shape[-1]
    T = x.size // H
    q = np.empty(x.shape, np.int8)
    s = np.empty(T, np.float32)
    lib().ora_rmsnorm_quant(_p(q, _i8p), _p(s, _f32p), _p(x, _u16p), _p(w, _u16p), T, H, eps)
    return q, s


def add_rmsnorm_quant(x, res, w, eps: float):
    x, res, w = _u16(x), _u16(res), _u16(w)
    H = x.shape[-1]
    T = x.size // H
    q = np.empty(x.shape, np.int8)
    s = np.empty(T, np.float32)
    ro = np.empty_like(x)
    lib().ora_add_rmsnorm_quant(_p(q, _i8p), _p(s, _f32p), _p(ro, _u16p), _p(x, _u16p), _p(res, _u16p),
                                _p(w, _u16p), T, H, eps)
    return q, s, ro


def quant_rows(x):
    x = _u16(x)
    cols = x.shape[-1]
    rows = x.size // cols
    q = np.empty(x.shape, np.int8)
    s = np.empty(rows, np.float32)
    lib().ora_quant_rows(_p(q, _i8p), _p(s, _f32p), _p(x, _u16p), rows, cols)
    return q, s


def quant_tensor(x):
    x = _u16(x)
    q = np.empty(x.shape, np.int8)
    s = np.empty(1, np.float32)
    lib().ora_quant_tensor(_p(q, _i8p), _p(s, _f32p), _p(x, _u16p), x.size)
    return q, s


def quant_cols(x):
    x = _u16(x)
    K, N = x.shape
    q = np.empty(x.shape, np.int8)
    s = np.empty(N, np.float32)
    lib().ora_quant_cols(_p(q, _i8p), _p(s, _f32p), _p(x, _u16p), K, N)
    return q, s


def dequant(q, scales, mode: str):
    q = np.ascontiguousarray(q, dtype=np.int8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    if mode == "tensor":
        rows, cols = 1, q.size
    else:
        rows, cols = q.shape
    out = np.empty(q.shape, np.uint16)
    lib().ora_dequant(_p(out, _u16p), _p(q, _i8p), _p(scales, _f32p), rows, cols,
                      {"row": 0, "col": 1, "tensor": 2}[mode])
    return out


def bf16_to_f16_trunc(h) -> np.ndarray:
    """bf16 bits -> fp16 bits with the model loader's truncating rule
    (pkg/model/loader.go:23-85)."""
    h = _u16(h)
    out = np.empty_like(h)
    lib().ora_bf16_to_f16_trunc(_p(out, _u16p), _p(h, _u16p), h.size)
    return out


def gemm_int8(a, q, scale, transpose_b: bool) -> np.ndarray:
    """C = A @ (B * scale) as the reference composes it (gpu/cuda/matmul.cu:189-244).

    The int8 weights are first dequantized to fp16 by dequantize_and_copy
    (matmul.cu:169-186: fp16(float(q) * scale), scale per row of B when
    transpose_b, per column otherwise; the same rule as ``dequant``), then
    multiplied with the fp16 activations (cuda_gemm_fp16, matmul.cu:75-156).
    a: fp16 bits [M, K]; q: int8 [N, K] if transpose_b else [K, N]; scale:
    fp32 [N]. Returns the product of the two fp16 operands in float64, not
    rounded: the reference's own GEMM rounding belongs to cuBLAS and is not
    specified, so tests bound the distance to this value.
    """
    x = f16_bits_to_f32(_u16(a)).astype(np.float64)
    w = f16_bits_to_f32(dequant(q, scale, "row" if transpose_b else "col")).astype(np.float64)
    return x @ (w.T if transpose_b else w)


def gemm_fp16(a, b, transpose_a: bool, transpose_b: bool) -> np.ndarray:
    """C = op(A) @ op(B) of fp16 operands (gpu/cuda/matmul.cu:75-156), in
    float64, not rounded. A is [M, K] ([K, M] if transpose_a), B is [K, N]
    ([N, K] if transpose_b)."""
    x = f16_bits_to_f32(_u16(a)).astype(np.float64)
    w = f16_bits_to_f32(_u16(b)).astype(np.float64)
    return (x.T if transpose_a else x) @ (w.T if transpose_b else w)


def elementwise(op: str, a, b=None, s: float = 0.0, dtype: str = "f16") -> np.ndarray:
    a = _u16(a)
    b = _u16(b) if b is not None else a
    out = np.empty_like(a)
    lib().ora_elementwise(_p(out, _u16p), _p(a, _u16p), _p(b, _u16p), s, a.size, OPS[op], DTYPES[dtype])
    return out


def rope_inv_freq(D: int, theta: float) -> np.ndarray:
    inv = np.empty(D // 2, np.float32)
    lib().ora_rope_inv_freq(_p(inv, _f32p), D, theta)
    return inv


def rope(x, pos, style: int, theta: float, dtype: str = "f16") -> np.ndarray:
    """x [..., nh, D] with tokens = prod(leading dims); pos int32 [tokens]."""
    x = _u16(x)
    D = x.shape[-1]
    nh = x.shape[-2]
    T = x.size // (nh * D)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    assert pos.size == T
    out = np.empty_like(x)
    lib().ora_rope(_p(out, _u16p), _p(x, _u16p), _p(pos, _i32p), T, nh, D, style, theta, DTYPES[dtype])
    return out


def gather(table, ids) -> np.ndarray:
    table = _u16(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    V, H = table.shape
    assert ids.min(initial=0) >= 0 and ids.max(initial=0) < V
    out = np.empty((ids.size, H), np.uint16)
    lib().ora_gather(_p(out, _u16p), _p(table, _u16p), _p(ids, _i32p), ids.size, H)
    return out


def softmax(x) -> np.ndarray:
    x = _u16(x)
    R, Cc = x.shape
    out = np.empty_like(x)
    lib().ora_softmax(_p(out, _u16p), _p(x, _u16p), R, Cc)
    return out


# ------------------------------------------------------------------ fp32 storage

def rmsnorm_f32(x, w, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    H = x.shape[-1]
    y = np.empty_like(x)
    lib().ora_rmsnorm_f32(_p(y, _f32p), _p(x, _f32p), _p(w, _f32p), x.size // H, H, eps)
    return y


def elementwise_f32(op: str, a, b=None, s: float = 0.0) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32) if b is not None else a
    out = np.empty_like(a)
    lib().ora_elementwise_f32(_p(out, _f32p), _p(a, _f32p), _p(b, _f32p), s, a.size, OPS[op])
    return out


def rope_f32(x, pos, style: int, theta: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    D, nh = x.shape[-1], x.shape[-2]
    T = x.size // (nh * D)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    assert pos.size == T
    out = np.empty_like(x)
    lib().ora_rope_f32(_p(out, _f32p), _p(x, _f32p), _p(pos, _i32p), T, nh, D, style, theta)
    return out


def gather_rows(table, ids) -> np.ndarray:
    """Bit copy of table rows (any dtype)."""
    table = np.ascontiguousarray(table)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    V = table.shape[0]
    assert ids.min(initial=0) >= 0 and ids.max(initial=0) < V
    out = np.empty((ids.size,) + table.shape[1:], table.dtype)
    row_bytes = table.strides[0]
    lib().ora_gather_bytes(out.ctypes.data, table.ctypes.data, _p(ids, _i32p), ids.size, row_bytes)
    return out

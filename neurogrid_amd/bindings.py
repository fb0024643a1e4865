"""Host-side mirror of the reference's Go bindings for the per-layer kernels.

The reference's Go host calls ``libgpu_engine.so`` through cgo wrappers in
``gpu/bindings/gpu.go``. Go is not available here, so this module restates
those wrappers over the same C ABI with ctypes: same names, same argument
meaning and shape derivations, same error text (a Go ``error`` becomes a
raised :class:`GPUError`). The Go side stays unchanged in a real deployment:
its cgo wrappers link this library in place of the CUDA build.

Reference wrappers restated here (gpu/bindings/gpu.go):
  InitGPU :73, ShutdownGPU :82, GetDeviceCount :87, SetDevice :97,
  GetDeviceInfo :106, SyncDevice :121, GetMemoryUsed :130,
  AllocateTensor :140, FreeTensor :162, CopyToDevice :171, CopyToHost :192,
  CopyToDeviceINT8 :213, CopyToHostINT8 :236, RMSNorm :256, SiLU :282,
  Add :299, RoPE :317, GEMMFP16 :357, GEMMINT8 :395, QuantizePerTensor :427,
  DequantizePerTensor :445, QuantizeWeights :463, GatherEmbeddings :1277.
Tensor and Dtype restate pkg/types/tensor.go:11-104.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from enum import IntEnum

import numpy as np

from ._lib import DeviceInfo as _DeviceInfo
from ._lib import load


class GPUError(RuntimeError):
    """An error the Go wrapper would have returned."""


class Dtype(IntEnum):
    """pkg/types/tensor.go:11-16; the value is also the copy-function dtype code."""

    FP32 = 0
    FP16 = 1
    INT8 = 2

    def byte_size(self) -> int:  # tensor.go:33-44
        return {Dtype.FP32: 4, Dtype.FP16: 2, Dtype.INT8: 1}[self]


@dataclass
class Tensor:
    """pkg/types/tensor.go:47-104: a device buffer plus shape and dtype."""

    shape: list[int]
    dtype: Dtype
    device: int = 0
    data: int | None = field(default=None)

    def num_elements(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def byte_size(self) -> int:
        return self.num_elements() * self.dtype.byte_size()

    def validate(self) -> None:
        if len(self.shape) == 0:
            raise GPUError("tensor shape cannot be empty")
        for i, d in enumerate(self.shape):
            if d <= 0:
                raise GPUError(f"tensor dimension {i} must be positive, got {d}")


def NewTensor(shape, dtype: Dtype, device: int = 0) -> Tensor:
    return Tensor(list(shape), Dtype(dtype), device)


@dataclass
class DeviceInfo:
    Name: str
    Major: int
    Minor: int
    TotalMemory: int


def _lib():
    return load()


def _ptr(t: Tensor) -> C.c_void_p:
    return C.c_void_p(t.data)


# Where a Go wrapper would index past a short shape (a panic) or hand the
# kernel a tensor smaller than the call touches (a device access past the
# allocation), these wrappers raise before any call into the library, with
# the text of the C++ wrappers (neurogrid_amd/host/neurogrid_gpu.cpp).
def _rank(what: str, t: Tensor, rank: int) -> None:
    if len(t.shape) < rank:
        raise GPUError(f"{what}: tensor has {len(t.shape)} dimensions, needs at least {rank}")


def _need(what: str, operand: str, have: int, need: int) -> None:
    if have < need:
        raise GPUError(f"{what}: {operand} has {have} elements, the call needs {need}")


# ---------------------------------------------------------------- device management

def HasCUDA() -> bool:
    try:
        return GetDeviceCount() > 0
    except GPUError:
        return False


def InitGPU(device_id: int = 0) -> None:
    r = _lib().cuda_init(device_id)
    if r != 0:
        raise GPUError(f"CUDA init failed with code {r}")


def ShutdownGPU() -> None:
    _lib().cuda_shutdown()


def GetDeviceCount() -> int:
    n = C.c_int(0)
    r = _lib().cuda_get_device_count(C.byref(n))
    if r != 0:
        raise GPUError(f"failed to get device count: {r}")
    return n.value


def SetDevice(device_id: int) -> None:
    r = _lib().cuda_set_device(device_id)
    if r != 0:
        raise GPUError(f"failed to set device {device_id}: code {r}")


def GetDeviceInfo() -> DeviceInfo:
    info = _DeviceInfo()
    r = _lib().cuda_get_device_info(C.byref(info))
    if r != 0:
        raise GPUError(f"failed to get device info: {r}")
    return DeviceInfo(info.name.decode(), info.major, info.minor, info.total_memory)


def SyncDevice() -> None:
    r = _lib().cuda_sync_device()
    if r != 0:
        raise GPUError(f"device sync failed: {r}")


def GetMemoryUsed() -> int:
    used = C.c_size_t(0)
    r = _lib().cuda_get_memory_used(C.byref(used))
    if r != 0:
        raise GPUError(f"failed to get memory usage: {r}")
    return used.value


# ---------------------------------------------------------------- tensors

def AllocateTensor(t: Tensor | None) -> None:
    if t is None:
        raise GPUError("tensor is nil")
    t.validate()
    if t.device < 0 or t.device > 7:
        raise GPUError(f"invalid device ID: {t.device}")
    p = C.c_void_p()
    size = t.byte_size()
    r = _lib().cuda_malloc(C.byref(p), size)
    if r != 0:
        raise GPUError(f"CUDA malloc failed: {r} (size={size})")
    t.data = p.value


def FreeTensor(t: Tensor | None) -> None:
    if t is None or t.data is None:
        return
    _lib().cuda_free(C.c_void_p(t.data))
    t.data = None


def CopyToDevice(t: Tensor, data) -> None:
    """fp32 host data -> tensor (converted to fp16 on the way when t is FP16)."""
    if t is None or t.data is None:
        raise GPUError("tensor not allocated")
    a = np.ascontiguousarray(data, dtype=np.float32)
    if a.size < t.num_elements():
        raise GPUError(f"data size {a.size} < tensor size {t.num_elements()}")
    r = _lib().cuda_copy_to_device(_ptr(t), a.ctypes.data, t.num_elements(), int(t.dtype))
    if r != 0:
        raise GPUError(f"copy to device failed: {r}")


def CopyToHost(data: np.ndarray, t: Tensor) -> None:
    """tensor -> fp32 host array (fp16 widened exactly)."""
    if t is None or t.data is None:
        raise GPUError("tensor not allocated")
    if data.dtype != np.float32 or not data.flags.c_contiguous:
        raise GPUError("host buffer must be a contiguous float32 array")
    if data.size < t.num_elements():
        raise GPUError(f"buffer size {data.size} < tensor size {t.num_elements()}")
    r = _lib().cuda_copy_to_host(data.ctypes.data, _ptr(t), t.num_elements(), int(t.dtype))
    if r != 0:
        raise GPUError(f"copy to host failed: {r}")


def CopyToDeviceINT8(t: Tensor, data) -> None:
    if t is None or t.data is None:
        raise GPUError("tensor not allocated")
    if t.dtype != Dtype.INT8:
        raise GPUError("tensor dtype must be INT8")
    a = np.ascontiguousarray(data, dtype=np.int8)
    if a.size < t.num_elements():
        raise GPUError(f"data size {a.size} < tensor size {t.num_elements()}")
    r = _lib().cuda_copy_int8_to_device(_ptr(t), a.ctypes.data, t.num_elements())
    if r != 0:
        raise GPUError(f"copy INT8 to device failed: {r}")


def CopyToHostINT8(data: np.ndarray, t: Tensor) -> None:
    if t is None or t.data is None:
        raise GPUError("tensor not allocated")
    if t.dtype != Dtype.INT8:
        raise GPUError("tensor dtype must be INT8")
    if data.dtype != np.int8 or not data.flags.c_contiguous:
        raise GPUError("host buffer must be a contiguous int8 array")
    if data.size < t.num_elements():
        raise GPUError(f"buffer size {data.size} < tensor size {t.num_elements()}")
    r = _lib().cuda_copy_int8_to_host(data.ctypes.data, _ptr(t), t.num_elements())
    if r != 0:
        raise GPUError(f"copy INT8 to host failed: {r}")


# ---------------------------------------------------------------- kernels

def RMSNorm(output: Tensor, input: Tensor, weight: Tensor, eps: float) -> None:
    """gpu.go:256-279: numTokens = numel / shape[-1]."""
    if output is None or input is None or weight is None:
        raise GPUError("nil tensor")
    if output.data is None or input.data is None or weight.data is None:
        raise GPUError("tensor not allocated")
    _rank("RMSNorm", input, 1)
    hidden = input.shape[-1]
    if hidden <= 0:
        raise GPUError(f"RMSNorm: hidden size {hidden} must be positive")
    tokens = input.num_elements() // hidden
    _need("RMSNorm", "weight", weight.num_elements(), hidden)
    _need("RMSNorm", "output", output.num_elements(), input.num_elements())
    r = _lib().cuda_rmsnorm(_ptr(output), _ptr(input), _ptr(weight), tokens, hidden, C.c_float(eps))
    if r != 0:
        raise GPUError(f"RMSNorm failed: {r}")


def SiLU(output: Tensor, input: Tensor) -> None:
    if output is None or input is None:
        raise GPUError("nil tensor")
    _need("SiLU", "output", output.num_elements(), input.num_elements())
    r = _lib().cuda_silu(_ptr(output), _ptr(input), input.num_elements())
    if r != 0:
        raise GPUError(f"SiLU failed: {r}")


def Add(c: Tensor, a: Tensor, b: Tensor) -> None:
    if c is None or a is None or b is None:
        raise GPUError("nil tensor")
    _need("Add", "b", b.num_elements(), a.num_elements())
    _need("Add", "c", c.num_elements(), a.num_elements())
    r = _lib().cuda_add(_ptr(c), _ptr(a), _ptr(b), a.num_elements())
    if r != 0:
        raise GPUError(f"Add failed: {r}")


def RoPE(output: Tensor, input: Tensor, positions, head_dim: int) -> None:
    """gpu.go:317-357: [batch, seq, heads, head_dim]; host positions are copied
    into a temporary device buffer for the call, then cuda_rope (split-half,
    theta 10000) runs."""
    if output is None or input is None:
        raise GPUError("nil tensor")
    if len(input.shape) < 4:
        raise GPUError("input must have 4 dimensions: [batch, seq, heads, head_dim]")
    batch, seq, heads = input.shape[0], input.shape[1], input.shape[2]
    pos = np.ascontiguousarray(positions, dtype=np.int32)
    touched = batch * seq * heads * head_dim
    _need("RoPE", "positions", pos.size, batch * seq)
    _need("RoPE", "input", input.num_elements(), touched)
    _need("RoPE", "output", output.num_elements(), touched)
    lib = _lib()
    dpos = C.c_void_p()
    if lib.cuda_malloc(C.byref(dpos), pos.nbytes) != 0:
        raise GPUError("failed to allocate positions on GPU")
    try:
        if lib.cuda_copy_int8_to_device(dpos, pos.ctypes.data, pos.nbytes) != 0:
            raise GPUError("failed to copy positions to GPU")
        r = lib.cuda_rope(_ptr(output), _ptr(input), C.cast(dpos, C.POINTER(C.c_int)), batch, seq, heads, head_dim)
        if r != 0:
            raise GPUError(f"RoPE failed: {r}")
        # The Go wrapper frees the positions with a deferred cudaFree, which
        # waits for the kernel; synchronise before freeing likewise.
        lib.cuda_sync_device()
    finally:
        lib.cuda_free(dpos)


def GEMMFP16(c: Tensor, a: Tensor, b: Tensor, transposeA: bool, transposeB: bool) -> None:
    """gpu.go:357-391: M, K from a's shape (swapped when transposeA), N from b's."""
    if c is None or a is None or b is None:
        raise GPUError("nil tensor")
    _rank("GEMM FP16", a, 2)
    _rank("GEMM FP16", b, 2)
    M, K = (a.shape[1], a.shape[0]) if transposeA else (a.shape[0], a.shape[1])
    N = b.shape[0] if transposeB else b.shape[1]
    _need("GEMM FP16", "a", a.num_elements(), M * K)
    _need("GEMM FP16", "b", b.num_elements(), K * N)
    _need("GEMM FP16", "c", c.num_elements(), M * N)
    r = _lib().cuda_gemm_fp16(_ptr(c), _ptr(a), _ptr(b), M, K, N, bool(transposeA), bool(transposeB))
    if r != 0:
        raise GPUError(f"GEMM FP16 failed: {r}")


def GEMMINT8(c: Tensor, a: Tensor, b: Tensor, scale: Tensor, transposeB: bool) -> None:
    """gpu.go:395-424: M, K from a; N = b.shape[0] when transposeB (B [N, K]), else b.shape[1]."""
    if c is None or a is None or b is None or scale is None:
        raise GPUError("nil tensor")
    _rank("GEMM INT8", a, 2)
    _rank("GEMM INT8", b, 2)
    M, K = a.shape[0], a.shape[1]
    N = b.shape[0] if transposeB else b.shape[1]
    _need("GEMM INT8", "b", b.num_elements(), K * N)
    _need("GEMM INT8", "c", c.num_elements(), M * N)
    _need("GEMM INT8", "scale", scale.num_elements(), N)
    r = _lib().cuda_gemm_int8(_ptr(c), _ptr(a), _ptr(b), _ptr(scale), M, K, N, bool(transposeB))
    if r != 0:
        raise GPUError(f"GEMM INT8 failed: {r}")


def QuantizePerTensor(output: Tensor, scale: Tensor, input: Tensor) -> None:
    if output is None or scale is None or input is None:
        raise GPUError("nil tensor")
    _need("quantize", "output", output.num_elements(), input.num_elements())
    r = _lib().cuda_quantize_per_tensor(_ptr(output), _ptr(scale), _ptr(input), input.num_elements())
    if r != 0:
        raise GPUError(f"quantize failed: {r}")


def DequantizePerTensor(output: Tensor, input: Tensor, scale: Tensor) -> None:
    if output is None or input is None or scale is None:
        raise GPUError("nil tensor")
    _need("dequantize", "output", output.num_elements(), input.num_elements())
    r = _lib().cuda_dequantize_per_tensor(_ptr(output), _ptr(input), _ptr(scale), input.num_elements())
    if r != 0:
        raise GPUError(f"dequantize failed: {r}")


def QuantizeWeights(output: Tensor, scales: Tensor, input: Tensor) -> None:
    """gpu.go:463-482: per-column, K = shape[0], N = shape[1]."""
    if output is None or scales is None or input is None:
        raise GPUError("nil tensor")
    _rank("quantize weights", input, 2)
    K, N = input.shape[0], input.shape[1]
    _need("quantize weights", "output", output.num_elements(), input.num_elements())
    _need("quantize weights", "scales", scales.num_elements(), N)
    r = _lib().cuda_quantize_weights(_ptr(output), _ptr(scales), _ptr(input), K, N)
    if r != 0:
        raise GPUError(f"quantize weights failed: {r}")


def GatherEmbeddings(output: int, embed_table: int, d_token_ids: int, hidden_size: int, num_tokens: int) -> None:
    """gpu.go:1277-1285: raw device pointers."""
    r = _lib().cuda_gather_embeddings(
        C.c_void_p(output), C.c_void_p(embed_table), C.cast(C.c_void_p(d_token_ids), C.POINTER(C.c_int)),
        hidden_size, num_tokens)
    if r != 0:
        raise GPUError(f"gather embeddings failed: {r}")

"""Host-side logic of the Python bindings mirror (neurogrid_amd.bindings,
restating gpu/bindings/gpu.go): shape rules and the errors raised before any
call into the library. No GPU: every case here fails its checks before the
library would be touched, and tensors carry a stand-in address that nothing
dereferences."""
from __future__ import annotations

import pytest

from neurogrid_amd import bindings as B


def t(shape, dtype=B.Dtype.FP16):
    x = B.NewTensor(shape, dtype)
    x.data = 0x1000   # a stand-in: the calls below fail before using it
    return x


def test_tensor_rules():
    x = B.NewTensor([2, 3, 4], B.Dtype.FP16)
    assert x.num_elements() == 24 and x.byte_size() == 48
    assert B.NewTensor([5], B.Dtype.INT8).byte_size() == 5
    assert B.NewTensor([5], B.Dtype.FP32).byte_size() == 20
    with pytest.raises(B.GPUError, match="tensor shape cannot be empty"):
        B.NewTensor([], B.Dtype.FP16).validate()
    with pytest.raises(B.GPUError, match="tensor dimension 1 must be positive, got 0"):
        B.NewTensor([3, 0], B.Dtype.FP16).validate()


def test_nil_and_unallocated():
    with pytest.raises(B.GPUError, match="nil tensor"):
        B.SiLU(None, t([4]))
    with pytest.raises(B.GPUError, match="tensor not allocated"):
        B.RMSNorm(t([4]), B.NewTensor([4], B.Dtype.FP16), t([4]), 1e-6)
    with pytest.raises(B.GPUError, match="tensor not allocated"):
        B.CopyToDevice(B.NewTensor([4], B.Dtype.FP16), [0.0] * 4)
    with pytest.raises(B.GPUError, match="tensor is nil"):
        B.AllocateTensor(None)
    with pytest.raises(B.GPUError, match="invalid device ID: 9"):
        B.AllocateTensor(B.NewTensor([4], B.Dtype.FP16, 9))


def test_short_shapes():
    with pytest.raises(B.GPUError, match="input must have 4 dimensions"):
        B.RoPE(t([4]), t([4]), [0], 128)
    with pytest.raises(B.GPUError, match="GEMM INT8: tensor has 1 dimensions, needs at least 2"):
        B.GEMMINT8(t([2, 4]), t([8]), t([4, 4], B.Dtype.INT8), t([4], B.Dtype.FP32), True)
    with pytest.raises(B.GPUError, match="GEMM FP16: tensor has 1 dimensions, needs at least 2"):
        B.GEMMFP16(t([2, 4]), t([2, 4]), t([8]), False, False)
    with pytest.raises(B.GPUError, match="quantize weights: tensor has 1 dimensions"):
        B.QuantizeWeights(t([4], B.Dtype.INT8), t([4], B.Dtype.FP32), t([4]))


def test_operands_smaller_than_the_call():
    q = t([1, 2, 4, 64])                                  # 512 elements, 2 tokens
    with pytest.raises(B.GPUError, match="RoPE: positions has 1 elements, the call needs 2"):
        B.RoPE(q, q, [0], 64)
    with pytest.raises(B.GPUError, match="RoPE: input has 512 elements, the call needs 1024"):
        B.RoPE(q, q, [0, 1], 128)
    with pytest.raises(B.GPUError, match="SiLU: output has 4 elements, the call needs 1024"):
        B.SiLU(t([4]), t([1024]))
    with pytest.raises(B.GPUError, match="Add: b has 4 elements, the call needs 1024"):
        B.Add(t([1024]), t([1024]), t([4]))
    with pytest.raises(B.GPUError, match="RMSNorm: weight has 4 elements, the call needs 1024"):
        B.RMSNorm(t([1024]), t([1024]), t([4]), 1e-6)
    with pytest.raises(B.GPUError, match="GEMM INT8: b has 512 elements, the call needs 1024"):
        B.GEMMINT8(t([2, 16]), t([2, 64]), t([16, 32], B.Dtype.INT8), t([16], B.Dtype.FP32), True)
    with pytest.raises(B.GPUError, match="GEMM INT8: scale has 8 elements, the call needs 16"):
        B.GEMMINT8(t([2, 16]), t([2, 64]), t([16, 64], B.Dtype.INT8), t([8], B.Dtype.FP32), True)
    with pytest.raises(B.GPUError, match="GEMM FP16: c has 4 elements, the call needs 8"):
        B.GEMMFP16(t([4]), t([2, 4]), t([4, 4]), False, False)
    with pytest.raises(B.GPUError, match="quantize: output has 2 elements, the call needs 4"):
        B.QuantizePerTensor(t([2], B.Dtype.INT8), t([1], B.Dtype.FP32), t([4]))
    with pytest.raises(B.GPUError, match="quantize weights: scales has 2 elements, the call needs 4"):
        B.QuantizeWeights(t([8, 4], B.Dtype.INT8), t([2], B.Dtype.FP32), t([8, 4]))

"""Loader for the gfx950 kernel library and its C-ABI signatures.

``load()`` opens ``neurogrid_amd/lib/libgpu_engine.so`` (built by
``neurogrid_amd.build``) and declares argument/return types for every entry
point in ``include/*.h``. There is no fallback: if the library is missing
the import fails with an error that says how to build it.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libgpu_engine.so"

_vp, _cvp, _i, _sz, _f = C.c_void_p, C.c_void_p, C.c_int, C.c_size_t, C.c_float
_ip = C.POINTER(C.c_int)


class DeviceInfo(C.Structure):
    """Layout of DeviceInfo in include/memory.h (reference gpu/cuda/memory.h:12-17)."""

    _fields_ = [("name", C.c_char * 256), ("major", C.c_int), ("minor", C.c_int), ("total_memory", C.c_size_t)]


# name -> (restype, argtypes). One entry per declaration in include/*.h.
SIGNATURES: dict[str, tuple] = {
    # memory.h
    "cuda_init": (_i, [_i]),
    "cuda_shutdown": (None, []),
    "cuda_get_device_count": (_i, [_ip]),
    "cuda_set_device": (_i, [_i]),
    "cuda_get_device_info": (_i, [C.POINTER(DeviceInfo)]),
    "cuda_sync_device": (_i, []),
    "cuda_get_memory_used": (_i, [C.POINTER(C.c_size_t)]),
    "cuda_malloc": (_i, [C.POINTER(C.c_void_p), _sz]),
    "cuda_free": (None, [_vp]),
    "cuda_copy_to_device": (_i, [_vp, _cvp, _sz, _i]),
    "cuda_copy_to_host": (_i, [_vp, _cvp, _sz, _i]),
    "cuda_copy_int8_to_device": (_i, [_vp, _cvp, _sz]),
    "cuda_copy_int8_to_host": (_i, [_vp, _cvp, _sz]),
    # stream.h
    "ng_get_stream": (_vp, []),
    "ng_set_stream": (None, [_vp]),
    # kernels.h
    "cuda_rmsnorm": (_i, [_vp, _cvp, _cvp, _i, _i, _f]),
    "cuda_silu": (_i, [_vp, _cvp, _sz]),
    "cuda_add": (_i, [_vp, _cvp, _cvp, _sz]),
    "cuda_mul": (_i, [_vp, _cvp, _cvp, _sz]),
    "cuda_rope": (_i, [_vp, _cvp, _ip, _i, _i, _i, _i]),
    "cuda_rope_styled": (_i, [_vp, _cvp, _ip, _i, _i, _i, _i, _i]),
    "cuda_rope_with_theta": (_i, [_vp, _cvp, _ip, _i, _i, _i, _i, _i, _f]),
    "cuda_silu_mul": (_i, [_vp, _cvp, _cvp, _sz]),
    "cuda_add_rmsnorm": (_i, [_vp, _vp, _cvp, _cvp, _cvp, _i, _i, _f]),
    "cuda_softmax": (_i, [_vp, _cvp, _i, _i]),
    "cuda_scale": (_i, [_vp, _cvp, _f, _sz]),
    "cuda_gather_embeddings": (_i, [_vp, _cvp, _ip, _i, _i]),
    # bf16_utils.h
    "cuda_bf16_rmsnorm": (_i, [_vp, _cvp, _cvp, _i, _i, _f]),
    "cuda_bf16_silu": (_i, [_vp, _cvp, _sz]),
    "cuda_bf16_add": (_i, [_vp, _cvp, _cvp, _sz]),
    "cuda_bf16_mul": (_i, [_vp, _cvp, _cvp, _sz]),
    "cuda_bf16_to_fp32": (_i, [_vp, _cvp, _sz]),
    "cuda_fp32_to_bf16": (_i, [_vp, _cvp, _sz]),
    "cuda_fp16_to_bf16": (_i, [_vp, _cvp, _sz]),
    "cuda_bf16_to_fp16": (_i, [_vp, _cvp, _sz]),
    "cuda_bf16_rope_with_theta": (_i, [_vp, _cvp, _ip, _i, _i, _i, _i, _i, _f]),
    "cuda_check_bf16_support": (_i, [_ip]),
    # quantize.h
    "cuda_quantize_per_tensor": (_i, [_vp, _vp, _cvp, _sz]),
    "cuda_dequantize_per_tensor": (_i, [_vp, _cvp, _cvp, _sz]),
    "cuda_quantize_weights": (_i, [_vp, _vp, _cvp, _i, _i]),
    "cuda_quantize_weights_per_row": (_i, [_vp, _vp, _cvp, _i, _i]),
    # neurogrid_ext.h
    "ng_version": (C.c_char_p, []),
    "ng_rmsnorm_quant_int8": (_i, [_vp, _vp, _cvp, _cvp, _i, _i, _f]),
    "ng_add_rmsnorm_quant_int8": (_i, [_vp, _vp, _vp, _cvp, _cvp, _cvp, _i, _i, _f]),
    "ng_bf16_add_rmsnorm": (_i, [_vp, _vp, _cvp, _cvp, _cvp, _i, _i, _f]),
    "ng_bf16_silu_mul": (_i, [_vp, _cvp, _cvp, _sz]),
    "ng_fp32_to_fp16": (_i, [_vp, _cvp, _sz]),
    "ng_fp16_to_fp32": (_i, [_vp, _cvp, _sz]),
    "ng_bf16_to_fp16_truncate": (_i, [_vp, _cvp, _sz]),
    "cuda_dequantize_weights": (_i, [_vp, _cvp, _cvp, _i, _i, _i]),
    "ng_gather_embeddings_checked": (_i, [_vp, _cvp, _ip, _i, _i, _i, _ip]),
    "ng_rope_qk_with_theta": (_i, [_vp, _cvp, _vp, _cvp, _ip, _i, _i, _i, _i, _i, _i, _f]),
    "ng_bf16_rope_qk_with_theta": (_i, [_vp, _cvp, _vp, _cvp, _ip, _i, _i, _i, _i, _i, _i, _f]),
    "ng_per_head_rmsnorm": (_i, [_vp, _cvp, _cvp, _i, _i, _i, _f]),
    "ng_bf16_per_head_rmsnorm": (_i, [_vp, _cvp, _cvp, _i, _i, _i, _f]),
    "ng_qk_rmsnorm_rope_with_theta": (_i, [_vp, _cvp, _vp, _cvp, _cvp, _cvp, _ip, _i, _i, _i, _i, _i, _f, _i, _f]),
    "ng_bf16_qk_rmsnorm_rope_with_theta": (_i, [_vp, _cvp, _vp, _cvp, _cvp, _cvp, _ip, _i, _i, _i, _i, _i, _f, _i,
                                                _f]),
    # matmul.h
    "cuda_gemm_fp16": (_i, [_vp, _cvp, _cvp, _i, _i, _i, C.c_bool, C.c_bool]),
    "cuda_gemm_int8": (_i, [_vp, _cvp, _cvp, _cvp, _i, _i, _i, C.c_bool]),
    "ng_gemm_int8_noalloc": (_i, [_vp, _cvp, _cvp, _cvp, _i, _i, _i, C.c_bool]),
    "ng_gemm_int8_shared_a": (_i, [_i, C.POINTER(_vp), _cvp, C.POINTER(_cvp), C.POINTER(_cvp), _ip, _i, _i]),
    "ng_rmsnorm_gemm_int8_shared_a": (_i, [_i, _vp, C.POINTER(_vp), _cvp, _cvp, _f, C.POINTER(_cvp),
                                           C.POINTER(_cvp), _ip, _i, _i]),
    "ng_add_rmsnorm_gemm_int8_shared_a": (_i, [_i, _vp, _vp, C.POINTER(_vp), _cvp, _cvp, _cvp, _f,
                                               C.POINTER(_cvp), C.POINTER(_cvp), _ip, _i, _i]),
    "ng_gemm_int8_silu_mul": (_i, [_vp, _vp, _vp, _cvp, _cvp, _cvp, _cvp, _cvp, _i, _i, _i]),
    "ng_gemm_int8_add": (_i, [_vp, _vp, _cvp, _cvp, _cvp, _cvp, _i, _i, _i]),
    "ng_rmsnorm_qkv_rope_int8": (_i, [_vp, _vp, _vp, _vp, _cvp, _cvp, _f, C.POINTER(_cvp), C.POINTER(_cvp), _ip, _i,
                                      _i, _i, _i, _i, _f]),
}

_LIB = None


def load() -> C.CDLL:
    """Open the library once and attach signatures; raise if it is not built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is not built; run `python -m neurogrid_amd.build` "
            "(or __graft_entry__.build()) first. There is no CPU fallback."
        )
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib

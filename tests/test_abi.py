"""The C-ABI library loads on the CPU and exports every declared entry point.

No kernel is launched here: error paths that reject arguments before any HIP
call are the only calls made.
"""
from __future__ import annotations

import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions() -> set[str]:
    names = set()
    for h in HEADERS:
        text = h.read_text()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"#[^\n]*", "", text)
        for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_]*)\s*\(([^;{}]*)\)\s*;", text):
            names.add(m.group(1))
    return names


def test_headers_declare_the_reference_boundary():
    names = declared_functions()
    # the reference's hot-path and plumbing symbols (gpu/cuda/*.h, gpu/bindings/gpu.h)
    for sym in [
        "cuda_rmsnorm", "cuda_add_rmsnorm", "cuda_silu", "cuda_mul", "cuda_add", "cuda_silu_mul",
        "cuda_rope", "cuda_rope_styled", "cuda_rope_with_theta", "cuda_softmax", "cuda_scale",
        "cuda_gather_embeddings", "cuda_bf16_rmsnorm", "cuda_bf16_silu", "cuda_bf16_add", "cuda_bf16_mul",
        "cuda_bf16_to_fp32", "cuda_fp32_to_bf16", "cuda_fp16_to_bf16", "cuda_bf16_to_fp16",
        "cuda_bf16_rope_with_theta", "cuda_check_bf16_support", "cuda_quantize_per_tensor",
        "cuda_dequantize_per_tensor", "cuda_quantize_weights", "cuda_quantize_weights_per_row",
        "ng_get_stream", "ng_set_stream", "cuda_init", "cuda_shutdown", "cuda_get_device_count",
        "cuda_set_device", "cuda_get_device_info", "cuda_sync_device", "cuda_get_memory_used",
        "cuda_malloc", "cuda_free", "cuda_copy_to_device", "cuda_copy_to_host",
        "cuda_copy_int8_to_device", "cuda_copy_int8_to_host", "cuda_gemm_int8",
    ]:
        assert sym in names, sym


def test_library_exports_every_declared_symbol():
    from neurogrid_amd import _lib

    L = _lib.load()
    names = declared_functions()
    missing = [n for n in sorted(names) if not hasattr(L, n)]
    assert not missing, missing
    # the ctypes signature table covers exactly the declared set
    assert set(_lib.SIGNATURES) == names


def test_exports_are_dynamic_symbols():
    from neurogrid_amd import _lib

    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert declared_functions() <= exported


def test_library_is_built_for_gfx950_only():
    from neurogrid_amd import _lib

    blob = _lib.LIB_PATH.read_bytes()
    targets = set(re.findall(rb"amdgcn-amd-amdhsa--(gfx[0-9a-z]+)", blob))
    assert targets == {b"gfx950"}


def test_argument_errors_return_minus_one_without_touching_the_gpu(capfd):
    from neurogrid_amd import _lib

    L = _lib.load()
    p = C.c_void_p(256)
    ip = C.cast(p, C.POINTER(C.c_int))
    assert L.cuda_rmsnorm(None, p, p, 1, 8, 1e-5) == -1
    assert L.cuda_rmsnorm(p, p, p, 0, 8, 1e-5) == -1           # zero tokens: the reference's 0-block launch fails too
    assert L.cuda_add_rmsnorm(p, p, p, p, None, 1, 8, 1e-5) == -1
    assert L.cuda_silu_mul(p, p, p, 0) == -1
    assert L.cuda_add(p, None, p, 8) == -1
    assert L.cuda_rope_with_theta(p, p, ip, 1, 1, 1, 3, 0, 1e4) == -1   # odd head_dim
    assert L.cuda_rope_with_theta(p, p, ip, 1, 1, 1, 512, 0, 1e4) == -1  # head_dim > 256
    assert L.cuda_gather_embeddings(p, p, ip, 0, 4) == -1
    assert L.ng_gather_embeddings_checked(p, p, ip, 8, 4, 0, ip) == -1
    assert L.cuda_quantize_weights_per_row(p, p, p, 0, 8) == -1
    assert L.ng_rmsnorm_quant_int8(p, None, p, p, 1, 8, 1e-5) == -1
    assert L.cuda_dequantize_weights(p, p, p, 4, 0, 1) == -1
    assert L.cuda_copy_to_device(p, p, 4, 7) == -1               # unknown dtype code
    assert L.cuda_gemm_int8(p, p, None, p, 4, 64, 16, True) == -1
    assert L.cuda_gemm_int8(p, p, p, p, 4, 0, 16, True) == -1
    assert L.cuda_gemm_fp16(p, None, p, 4, 64, 16, False, False) == -1
    assert L.ng_gemm_int8_noalloc(p, p, None, p, 4, 64, 16, True) == -1
    assert L.ng_gemm_int8_noalloc(p, p, p, p, 129, 72, 16, True) == -1     # K % 16 != 0: hipBLASLt path
    assert L.ng_gemm_int8_noalloc(p, p, p, p, 4, 64, 16, False) == -1
    pv = (C.c_void_p * 2)(256, 512)
    pn = (C.c_void_p * 2)(256, None)
    nv = (C.c_int * 2)(16, 0)
    assert L.ng_gemm_int8_shared_a(0, pv, p, pv, pv, nv, 1, 64) == -1    # count outside 1..4
    assert L.ng_gemm_int8_shared_a(5, pv, p, pv, pv, nv, 1, 64) == -1
    assert L.ng_gemm_int8_shared_a(2, pv, p, pn, pv, nv, 1, 64) == -1    # null weights of product 1
    assert L.ng_gemm_int8_shared_a(2, pv, p, pv, pv, nv, 1, 64) == -1    # n[1] == 0
    assert L.ng_gemm_int8_shared_a(1, None, p, pv, pv, nv, 1, 64) == -1
    e = C.c_float(1e-5)
    assert L.ng_rmsnorm_gemm_int8_shared_a(0, p, pv, p, p, e, pv, pv, nv, 1, 64) == -1   # count outside 1..4
    assert L.ng_rmsnorm_gemm_int8_shared_a(1, None, pv, p, p, e, pv, pv, nv, 1, 64) == -1  # null normed
    assert L.ng_rmsnorm_gemm_int8_shared_a(2, p, pv, p, p, e, pv, pv, nv, 1, 64) == -1   # n[1] == 0
    assert L.ng_rmsnorm_gemm_int8_shared_a(1, p, pv, p, p, e, pv, pv, nv, 0, 64) == -1   # M == 0
    assert L.ng_add_rmsnorm_gemm_int8_shared_a(1, p, None, pv, p, p, p, e, pv, pv, nv, 1, 64) == -1  # null residual_out
    assert L.ng_add_rmsnorm_gemm_int8_shared_a(2, p, p, pv, p, p, p, e, pn, pv, nv, 1, 64) == -1  # null weights of product 1
    assert L.ng_add_rmsnorm_gemm_int8_shared_a(5, p, p, pv, p, p, p, e, pv, pv, nv, 1, 64) == -1
    assert L.ng_gemm_int8_silu_mul(p, p, p, p, None, p, p, p, 1, 64, 16) == -1     # null gate weights
    assert L.ng_gemm_int8_silu_mul(p, p, p, p, p, p, p, p, 1, 64, 0) == -1        # N == 0
    assert L.ng_gemm_int8_add(p, p, p, p, p, None, 1, 64, 16) == -1                 # null residual
    assert L.ng_gemm_int8_add(p, p, p, p, p, p, 0, 64, 16) == -1                    # M == 0
    pv3 = (C.c_void_p * 3)(256, 512, 768)
    f = C.c_float(1e4)
    assert L.ng_rmsnorm_qkv_rope_int8(p, p, p, p, p, p, e, pv3, pv3, ip, 1, 64, 2, 1, 3, f) == -1   # odd head_dim
    assert L.ng_rmsnorm_qkv_rope_int8(p, p, p, p, p, p, e, pv3, pv3, None, 1, 64, 2, 1, 8, f) == -1  # no positions
    assert L.ng_rmsnorm_qkv_rope_int8(p, p, p, p, p, p, e, pv3, pv3, ip, 1, 64, 2, 1, 512, f) == -1  # head_dim > 256
    assert L.ng_rmsnorm_qkv_rope_int8(p, p, p, p, p, p, e, pv3, pv3, ip, 1, 64, 2, 1 << 24, 256, f) == -1  # kv rows
    err = capfd.readouterr().err
    assert "neurogrid-amd:" in err and "null pointer" in err


def test_version_string():
    from neurogrid_amd import _lib

    assert b"gfx950" in _lib.load().ng_version()

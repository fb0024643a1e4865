"""Every compute entry point captured into a HIP graph and replayed.

The reference's decode path switches the library stream to a capture stream
and records the per-layer calls into a CUDA graph (decode_all.cu:509-603,
stream.cu:4-12). For each entry point here the test
  1. runs it eagerly on the capture stream (this also sizes the GEMM entry
     points' per-stream buffers, which cannot be allocated during capture),
  2. captures the same call into a graph,
  3. replays the graph three times; before each replay the outputs are zeroed
     from the host and unrelated eager work runs on the same stream,
and checks every replay against the eager run: bit for bit for the kernels
of this library, within the fp16 bar (|d| <= 1e-2 or 2 ulp) for the calls that
go through hipBLASLt. Inputs are never written, so a replay recomputes the
same values. No entry point may record a memset node (a kernel fills instead).

A last test captures a split-K GEMM, then makes an eager call whose partial
sums need a larger buffer, and replays the graph: the buffer the graph holds
must still be valid.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, HipRuntime, assert_bits_equal, assert_close16, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

T, H, I, NQ, NKV, D, V = 24, 512, 1024, 4, 2, 128, 100
GK, GN = 512, 256
GNW = 12288  # wide N for the GEMM
EPS, THETA = C.c_float(1e-5), C.c_float(1e6)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


@pytest.fixture(scope="module")
def inp():
    rng = np.random.Generator(np.random.PCG64(7))

    def n(*shape, s=1.0):
        return (rng.standard_normal(shape) * s).astype(np.float32)

    a = {}
    for tag, cvt in (("h", f16_bits), ("b", bf16_bits)):
        a[f"x{tag}"] = cvt(n(T, H))
        a[f"r{tag}"] = cvt(n(T, H, s=2.0))
        a[f"w{tag}"] = cvt(1.0 + n(H, s=0.02))
        a[f"g{tag}"] = cvt(n(T, I))
        a[f"u{tag}"] = cvt(n(T, I))
        a[f"q{tag}"] = cvt(n(T, NQ, D))
        a[f"k{tag}"] = cvt(n(T, NKV, D))
        a[f"qw{tag}"] = cvt(1.0 + n(D, s=0.1))
        a[f"kw{tag}"] = cvt(1.0 + n(D, s=0.1))
        a[f"tab{tag}"] = cvt(n(V, H, s=0.02))
    a["xf"] = n(T, H)
    a["pos"] = rng.integers(0, 4096, T).astype(np.int32)
    a["ids"] = rng.integers(0, V, T).astype(np.int32)
    bad = a["ids"].copy()
    bad[[3, 17]] = [V + 5, -1]
    a["ids_bad"] = bad
    a["wq"] = rng.integers(-127, 128, (GN, GK)).astype(np.int8)
    a["wq_kn"] = rng.integers(-127, 128, (GK, GN)).astype(np.int8)
    a["wsc"] = rng.uniform(1e-3, 1e-2, GN).astype(np.float32)
    a["wq_wide"] = rng.integers(-127, 128, (GNW, GK)).astype(np.int8)
    a["wsc_wide"] = rng.uniform(1e-3, 1e-2, GNW).astype(np.float32)
    a["tsc"] = np.array([0.0125], np.float32)
    a["wh"] = f16_bits(n(GK, GN, s=0.05))
    for m in (1, 3, 16, 24, 40, 64, 100, 200, 4096):
        a[f"a{m}"] = f16_bits(n(m, GK))
    bufs = {k: dev(v) for k, v in a.items()}
    yield bufs
    for b in bufs.values():
        b.free()


# name -> (outputs {name: (dtype, shape)}, call(lib, i, o) -> rc, bit-exact?)
E2 = np.uint16


def _ops():
    ops = {}

    def add(name, outs, fn, exact=True):
        ops[name] = (outs, fn, exact)

    for tag, pre in (("h", "cuda_"), ("b", "cuda_bf16_")):
        add(f"{pre}rmsnorm", {"y": (E2, (T, H))},
            lambda L, i, o, p=pre, t=tag: getattr(L, f"{p}rmsnorm")(o["y"].vp, i[f"x{t}"].vp, i[f"w{t}"].vp, T, H, EPS))
        add(f"{pre}silu", {"y": (E2, (T, I))},
            lambda L, i, o, p=pre, t=tag: getattr(L, f"{p}silu")(o["y"].vp, i[f"g{t}"].vp, T * I))
        add(f"{pre}add", {"y": (E2, (T, H))},
            lambda L, i, o, p=pre, t=tag: getattr(L, f"{p}add")(o["y"].vp, i[f"x{t}"].vp, i[f"r{t}"].vp, T * H))
        add(f"{pre}mul", {"y": (E2, (T, I))},
            lambda L, i, o, p=pre, t=tag: getattr(L, f"{p}mul")(o["y"].vp, i[f"g{t}"].vp, i[f"u{t}"].vp, T * I))
        add(f"{pre}rope_with_theta", {"y": (E2, (T, NQ, D))},
            lambda L, i, o, p=pre, t=tag: getattr(L, f"{p}rope_with_theta")(
                o["y"].vp, i[f"q{t}"].vp, i["pos"].ip, 1, T, NQ, D, 1, THETA))
    add("cuda_silu_mul", {"y": (E2, (T, I))},
        lambda L, i, o: L.cuda_silu_mul(o["y"].vp, i["gh"].vp, i["uh"].vp, T * I))
    add("ng_bf16_silu_mul", {"y": (E2, (T, I))},
        lambda L, i, o: L.ng_bf16_silu_mul(o["y"].vp, i["gb"].vp, i["ub"].vp, T * I))
    add("cuda_add_rmsnorm", {"y": (E2, (T, H)), "ro": (E2, (T, H))},
        lambda L, i, o: L.cuda_add_rmsnorm(o["y"].vp, o["ro"].vp, i["xh"].vp, i["rh"].vp, i["wh"].vp, T, H, EPS))
    add("ng_bf16_add_rmsnorm", {"y": (E2, (T, H)), "ro": (E2, (T, H))},
        lambda L, i, o: L.ng_bf16_add_rmsnorm(o["y"].vp, o["ro"].vp, i["xb"].vp, i["rb"].vp, i["wb"].vp, T, H, EPS))
    add("cuda_rope", {"y": (E2, (T, NQ, D))},
        lambda L, i, o: L.cuda_rope(o["y"].vp, i["qh"].vp, i["pos"].ip, 1, T, NQ, D))
    add("cuda_rope_styled", {"y": (E2, (T, NKV, D))},
        lambda L, i, o: L.cuda_rope_styled(o["y"].vp, i["kh"].vp, i["pos"].ip, 1, T, NKV, D, 1))
    for tag, pre in (("h", "ng_"), ("b", "ng_bf16_")):
        add(f"{pre}rope_qk_with_theta", {"q": (E2, (T, NQ, D)), "k": (E2, (T, NKV, D))},
            lambda L, i, o, p=pre, t=tag: getattr(L, f"{p}rope_qk_with_theta")(
                o["q"].vp, i[f"q{t}"].vp, o["k"].vp, i[f"k{t}"].vp, i["pos"].ip, 1, T, NQ, NKV, D, 0, THETA))
        add(f"{pre}per_head_rmsnorm", {"y": (E2, (T, NQ, D))},
            lambda L, i, o, p=pre, t=tag: getattr(L, f"{p}per_head_rmsnorm")(
                o["y"].vp, i[f"q{t}"].vp, i[f"qw{t}"].vp, T, NQ, D, EPS))
        add(f"{pre}qk_rmsnorm_rope_with_theta", {"q": (E2, (T, NQ, D)), "k": (E2, (T, NKV, D))},
            lambda L, i, o, p=pre, t=tag: getattr(L, f"{p}qk_rmsnorm_rope_with_theta")(
                o["q"].vp, i[f"q{t}"].vp, o["k"].vp, i[f"k{t}"].vp, i[f"qw{t}"].vp, i[f"kw{t}"].vp, i["pos"].ip,
                1, T, NQ, NKV, D, EPS, 0, THETA))
    add("cuda_softmax", {"y": (E2, (T, H))}, lambda L, i, o: L.cuda_softmax(o["y"].vp, i["xh"].vp, T, H))
    add("cuda_scale", {"y": (E2, (T, H))}, lambda L, i, o: L.cuda_scale(o["y"].vp, i["xh"].vp, C.c_float(0.37), T * H))
    add("cuda_gather_embeddings", {"y": (E2, (T, H))},
        lambda L, i, o: L.cuda_gather_embeddings(o["y"].vp, i["tabh"].vp, i["ids"].ip, H, T))
    add("ng_gather_embeddings_checked", {"y": (E2, (T, H)), "n": (np.int32, (1,))},
        lambda L, i, o: L.ng_gather_embeddings_checked(o["y"].vp, i["tabb"].vp, i["ids_bad"].ip, H, T, V, o["n"].ip))
    # dtype converters
    add("cuda_bf16_to_fp32", {"y": (np.float32, (T, H))}, lambda L, i, o: L.cuda_bf16_to_fp32(o["y"].vp, i["xb"].vp, T * H))
    add("cuda_fp32_to_bf16", {"y": (E2, (T, H))}, lambda L, i, o: L.cuda_fp32_to_bf16(o["y"].vp, i["xf"].vp, T * H))
    add("cuda_fp16_to_bf16", {"y": (E2, (T, H))}, lambda L, i, o: L.cuda_fp16_to_bf16(o["y"].vp, i["xh"].vp, T * H))
    add("cuda_bf16_to_fp16", {"y": (E2, (T, H))}, lambda L, i, o: L.cuda_bf16_to_fp16(o["y"].vp, i["xb"].vp, T * H))
    add("ng_fp32_to_fp16", {"y": (E2, (T, H))}, lambda L, i, o: L.ng_fp32_to_fp16(o["y"].vp, i["xf"].vp, T * H))
    add("ng_fp16_to_fp32", {"y": (np.float32, (T, H))}, lambda L, i, o: L.ng_fp16_to_fp32(o["y"].vp, i["xh"].vp, T * H))
    add("ng_bf16_to_fp16_truncate", {"y": (E2, (T, H))},
        lambda L, i, o: L.ng_bf16_to_fp16_truncate(o["y"].vp, i["xb"].vp, T * H))
    # quantisation
    add("ng_rmsnorm_quant_int8", {"q": (np.int8, (T, H)), "s": (np.float32, (T,))},
        lambda L, i, o: L.ng_rmsnorm_quant_int8(o["q"].vp, o["s"].vp, i["xh"].vp, i["wh"].vp, T, H, EPS))
    add("ng_add_rmsnorm_quant_int8", {"q": (np.int8, (T, H)), "s": (np.float32, (T,)), "ro": (E2, (T, H))},
        lambda L, i, o: L.ng_add_rmsnorm_quant_int8(o["q"].vp, o["s"].vp, o["ro"].vp, i["xh"].vp, i["rh"].vp,
                                                    i["wh"].vp, T, H, EPS))
    add("cuda_quantize_per_tensor", {"q": (np.int8, (T, H)), "s": (np.float32, (1,))},
        lambda L, i, o: L.cuda_quantize_per_tensor(o["q"].vp, o["s"].vp, i["xh"].vp, T * H))
    add("cuda_dequantize_per_tensor", {"y": (E2, (GN, GK))},
        lambda L, i, o: L.cuda_dequantize_per_tensor(o["y"].vp, i["wq"].vp, i["tsc"].vp, GN * GK))
    add("cuda_quantize_weights", {"q": (np.int8, (T, H)), "s": (np.float32, (H,))},
        lambda L, i, o: L.cuda_quantize_weights(o["q"].vp, o["s"].vp, i["xh"].vp, T, H))
    add("cuda_quantize_weights_per_row", {"q": (np.int8, (T, H)), "s": (np.float32, (T,))},
        lambda L, i, o: L.cuda_quantize_weights_per_row(o["q"].vp, o["s"].vp, i["xh"].vp, T, H))
    add("cuda_dequantize_weights_row", {"y": (E2, (GN, GK))},
        lambda L, i, o: L.cuda_dequantize_weights(o["y"].vp, i["wq"].vp, i["wsc"].vp, GN, GK, 1))
    add("cuda_dequantize_weights_col", {"y": (E2, (GK, GN))},
        lambda L, i, o: L.cuda_dequantize_weights(o["y"].vp, i["wq_kn"].vp, i["wsc"].vp, GK, GN, 0))
    # GEMMs: GEMV (M <= 4), small-M MFMA, split-K at three tile heights, the
    # prefill kernel with two K slices (M > 128), the library path
    # (transpose_b false), and the fp16 GEMM.
    for m in (1, 3, 16, 40, 64, 100):
        add(f"cuda_gemm_int8_M{m}", {"y": (E2, (m, GN))},
            lambda L, i, o, m=m: L.cuda_gemm_int8(o["y"].vp, i[f"a{m}"].vp, i["wq"].vp, i["wsc"].vp, m, GK, GN, True))
    # N >= 12288: one slice of K, two wave groups per block
    add("cuda_gemm_int8_M40_wide", {"y": (E2, (40, GNW))},
        lambda L, i, o: L.cuda_gemm_int8(o["y"].vp, i["a40"].vp, i["wq_wide"].vp, i["wsc_wide"].vp, 40, GK, GNW, True))
    add("cuda_gemm_int8_M200_prefill", {"y": (E2, (200, GN))},
        lambda L, i, o: L.cuda_gemm_int8(o["y"].vp, i["a200"].vp, i["wq"].vp, i["wsc"].vp, 200, GK, GN, True))
    # the allocation-free entry point: split-K weight streaming (M = 64: two
    # slices of K) and the prefill kernel with K slices (M = 200), partial sums
    # in the library's fixed device array
    add("ng_gemm_int8_noalloc_M64", {"y": (E2, (64, GN))},
        lambda L, i, o: L.ng_gemm_int8_noalloc(o["y"].vp, i["a64"].vp, i["wq"].vp, i["wsc"].vp, 64, GK, GN, True))
    add("ng_gemm_int8_noalloc_M200_prefill", {"y": (E2, (200, GN))},
        lambda L, i, o: L.ng_gemm_int8_noalloc(o["y"].vp, i["a200"].vp, i["wq"].vp, i["wsc"].vp, 200, GK, GN, True))
    # products that share A in one launch: the prefill kernel with two K slices (M = 200)
    add("ng_gemm_int8_shared_a_M200_prefill", {"y": (E2, (200, GN)), "y2": (E2, (200, GN))},
        lambda L, i, o: L.ng_gemm_int8_shared_a(
            2, (C.c_void_p * 2)(o["y"].ptr, o["y2"].ptr), i["a200"].vp, (C.c_void_p * 2)(i["wq"].ptr, i["wq"].ptr),
            (C.c_void_p * 2)(i["wsc"].ptr, i["wsc"].ptr), (C.c_int * 2)(GN, GN), 200, GK))
    # the split kernel with two K slices and the shared reduction (M = 24)
    add("ng_gemm_int8_shared_a_M24_split", {"y": (E2, (24, GN)), "y2": (E2, (24, GN))},
        lambda L, i, o: L.ng_gemm_int8_shared_a(
            2, (C.c_void_p * 2)(o["y"].ptr, o["y2"].ptr), i["a24"].vp, (C.c_void_p * 2)(i["wq"].ptr, i["wq"].ptr),
            (C.c_void_p * 2)(i["wsc"].ptr, i["wsc"].ptr), (C.c_int * 2)(GN, GN), 24, GK))
    # the GEMV kernel (M = 1), the small-M MFMA kernel (M = 16)
    add("ng_gemm_int8_shared_a_M16", {"y": (E2, (16, GN)), "y2": (E2, (16, GN))},
        lambda L, i, o: L.ng_gemm_int8_shared_a(
            2, (C.c_void_p * 2)(o["y"].ptr, o["y2"].ptr), i["a16"].vp, (C.c_void_p * 2)(i["wq"].ptr, i["wq"].ptr),
            (C.c_void_p * 2)(i["wsc"].ptr, i["wsc"].ptr), (C.c_int * 2)(GN, GN), 16, GK))
    add("ng_gemm_int8_shared_a_M1", {"y": (E2, (1, GN)), "y2": (E2, (1, GNW))},
        lambda L, i, o: L.ng_gemm_int8_shared_a(
            2, (C.c_void_p * 2)(o["y"].ptr, o["y2"].ptr), i["a1"].vp, (C.c_void_p * 2)(i["wq"].ptr, i["wq_wide"].ptr),
            (C.c_void_p * 2)(i["wsc"].ptr, i["wsc_wide"].ptr), (C.c_int * 2)(GN, GNW), 1, GK))
    # RMSNorm (add + RMSNorm) folded into the shared GEMV launch (M = 2, 1), and
    # a set with more GEMV blocks than the fused launch takes: the two calls
    add("ng_rmsnorm_gemm_int8_shared_a_M2", {"n": (E2, (2, GK)), "y": (E2, (2, GN)), "y2": (E2, (2, GN))},
        lambda L, i, o: L.ng_rmsnorm_gemm_int8_shared_a(
            2, o["n"].vp, (C.c_void_p * 2)(o["y"].ptr, o["y2"].ptr), i["xh"].vp, i["wh"].vp, EPS,
            (C.c_void_p * 2)(i["wq"].ptr, i["wq"].ptr), (C.c_void_p * 2)(i["wsc"].ptr, i["wsc"].ptr),
            (C.c_int * 2)(GN, GN), 2, GK))
    add("ng_add_rmsnorm_gemm_int8_shared_a_M1", {"n": (E2, (1, GK)), "ro": (E2, (1, GK)), "y": (E2, (1, GN))},
        lambda L, i, o: L.ng_add_rmsnorm_gemm_int8_shared_a(
            1, o["n"].vp, o["ro"].vp, (C.c_void_p * 1)(o["y"].ptr), i["xh"].vp, i["rh"].vp, i["wh"].vp, EPS,
            (C.c_void_p * 1)(i["wq"].ptr), (C.c_void_p * 1)(i["wsc"].ptr), (C.c_int * 1)(GN), 1, GK))
    add("ng_add_rmsnorm_gemm_int8_shared_a_M1_two_calls",
        {"n": (E2, (1, GK)), "ro": (E2, (1, GK)), "y": (E2, (1, GN)), "y2": (E2, (1, GNW))},
        lambda L, i, o: L.ng_add_rmsnorm_gemm_int8_shared_a(
            2, o["n"].vp, o["ro"].vp, (C.c_void_p * 2)(o["y"].ptr, o["y2"].ptr), i["xh"].vp, i["rh"].vp, i["wh"].vp,
            EPS, (C.c_void_p * 2)(i["wq"].ptr, i["wq_wide"].ptr), (C.c_void_p * 2)(i["wsc"].ptr, i["wsc_wide"].ptr),
            (C.c_int * 2)(GN, GNW), 1, GK))
    # gate/up and SwiGLU: one launch at M = 1 (in place on gate), the two calls at M = 16, the shared split
    # launch and the reduction's SwiGLU form at M = 24 (two K slices; the first 24 rows of a40)
    add("ng_gemm_int8_silu_mul_M1", {"g": (E2, (1, GN)), "u": (E2, (1, GN))},
        lambda L, i, o: L.ng_gemm_int8_silu_mul(o["g"].vp, o["g"].vp, o["u"].vp, i["a1"].vp, i["wq"].vp, i["wsc"].vp,
                                                i["wq"].vp, i["wsc"].vp, 1, GK, GN))
    add("ng_gemm_int8_silu_mul_M16", {"o": (E2, (16, GN)), "g": (E2, (16, GN)), "u": (E2, (16, GN))},
        lambda L, i, o: L.ng_gemm_int8_silu_mul(o["o"].vp, o["g"].vp, o["u"].vp, i["a16"].vp, i["wq"].vp, i["wsc"].vp,
                                                i["wq"].vp, i["wsc"].vp, 16, GK, GN))
    add("ng_gemm_int8_silu_mul_M24_sliced", {"o": (E2, (24, GN)), "g": (E2, (24, GN)), "u": (E2, (24, GN))},
        lambda L, i, o: L.ng_gemm_int8_silu_mul(o["o"].vp, o["g"].vp, o["u"].vp, i["a40"].vp, i["wq"].vp, i["wsc"].vp,
                                                i["wq"].vp, i["wsc"].vp, 24, GK, GN))
    # RMSNorm, q/k/v and RoPE on q and k (heads of 64): one launch at M = 1 (1 token at position 7)
    add("ng_rmsnorm_qkv_rope_int8_M1", {"n": (E2, (1, GK)), "q": (E2, (1, GN)), "k": (E2, (1, GN)),
                                        "v": (E2, (1, GN))},
        lambda L, i, o: L.ng_rmsnorm_qkv_rope_int8(
            o["n"].vp, o["q"].vp, o["k"].vp, o["v"].vp, i["xh"].vp, i["wh"].vp, EPS,
            (C.c_void_p * 3)(i["wq"].ptr, i["wq"].ptr, i["wq"].ptr), (C.c_void_p * 3)(i["wsc"].ptr, i["wsc"].ptr,
                                                                                   i["wsc"].ptr),
            i["pos"].ip, 1, GK, GN // 64, GN // 64, 64, THETA))
    # a product and the residual add after it: one launch at M = 1, the two calls at M = 16
    add("ng_gemm_int8_add_M1", {"o": (E2, (1, GN)), "c": (E2, (1, GN))},
        lambda L, i, o: L.ng_gemm_int8_add(o["o"].vp, o["c"].vp, i["a1"].vp, i["wq"].vp, i["wsc"].vp, i["xh"].vp,
                                           1, GK, GN))
    add("ng_gemm_int8_add_M16", {"o": (E2, (16, GN)), "c": (E2, (16, GN))},
        lambda L, i, o: L.ng_gemm_int8_add(o["o"].vp, o["c"].vp, i["a16"].vp, i["wq"].vp, i["wsc"].vp, i["xh"].vp,
                                           16, GK, GN))
    # from 4096 rows of A on: B dequantized into the stream's fp16 buffer, then hipBLASLt
    add("cuda_gemm_int8_M4096_library", {"y": (E2, (4096, GN))},
        lambda L, i, o: L.cuda_gemm_int8(o["y"].vp, i["a4096"].vp, i["wq"].vp, i["wsc"].vp, 4096, GK, GN, True),
        False)
    add("cuda_gemm_int8_kn_library", {"y": (E2, (16, GN))},
        lambda L, i, o: L.cuda_gemm_int8(o["y"].vp, i["a16"].vp, i["wq_kn"].vp, i["wsc"].vp, 16, GK, GN, False),
        False)
    add("cuda_gemm_fp16", {"y": (E2, (40, GN))},
        lambda L, i, o: L.cuda_gemm_fp16(o["y"].vp, i["a40"].vp, i["wh"].vp, 40, GK, GN, False, False), False)
    return ops


OPS = _ops()


@pytest.fixture()
def capture_stream(lib):
    hip = HipRuntime()
    stream = hip.stream()
    lib.ng_set_stream(stream)
    try:
        yield hip, stream
    finally:
        lib.ng_set_stream(None)
        hip.h.hipStreamDestroy(stream)


def replay_and_check(lib, hip, stream, outs, call, exact, label, between=None):
    def snapshot():
        return {n: get(b, outs[n][0], outs[n][1]) for n, b in bufs.items()}

    bufs = {n: empty(int(np.prod(shape)) * np.dtype(dt).itemsize) for n, (dt, shape) in outs.items()}
    scratch = empty(T * H * 2)
    try:
        for n, (dt, shape) in outs.items():
            bufs[n].upload(np.zeros(shape, dt))
        ok(call(bufs), f"{label} eager")
        hip.check(hip.h.hipStreamSynchronize(stream), "hipStreamSynchronize")
        eager = snapshot()
        graph, ex = hip.capture(stream, lambda: ok(call(bufs), f"{label} under capture"))
        try:
            for rep in range(3):
                for n, (dt, shape) in outs.items():
                    bufs[n].upload(np.zeros(shape, dt))
                if between is not None:
                    between(rep)
                ok(lib.cuda_add(scratch.vp, scratch.vp, scratch.vp, T * H))
                hip.check(hip.h.hipStreamSynchronize(stream), "hipStreamSynchronize")
                hip.launch(ex, stream)
                got = snapshot()
                for n in outs:
                    if exact or outs[n][0] != E2:
                        assert_bits_equal(got[n], eager[n], f"{label} replay {rep}: {n}")
                    else:
                        assert_close16(got[n], eager[n], "f16", f"{label} replay {rep}: {n}")
        finally:
            hip.destroy(graph, ex)
        return eager
    finally:
        for b in bufs.values():
            b.free()
        scratch.free()


@pytest.mark.parametrize("name", list(OPS))
def test_capture_replay(lib, inp, capture_stream, name):
    hip, stream = capture_stream
    outs, fn, exact = OPS[name]
    banner(f"graph capture: {name}")
    eager = replay_and_check(lib, hip, stream, outs, lambda o: fn(lib, inp, o), exact, name)
    if name == "ng_gather_embeddings_checked":
        assert int(eager["n"][0]) == 2


def test_capture_survives_buffer_growth(lib, inp, capture_stream):
    """A graph holding a split-K GEMM keeps replaying correctly after an eager
    call on the same stream has replaced the partial-sum buffer by a larger one."""
    hip, stream = capture_stream
    banner("graph capture: split-K GEMM, then buffer growth, then replay")
    K, N = 4096, 4096
    rng = np.random.Generator(np.random.PCG64(3))
    a = dev(f16_bits(rng.standard_normal((128, K)).astype(np.float32)))
    w = dev(rng.integers(-127, 128, (N, K)).astype(np.int8))
    sc = dev(rng.uniform(1e-3, 1e-2, N).astype(np.float32))
    big = empty(128 * N * 2)
    # (M, N) of the eager calls: their split-K partial sums take 2, 4 and 8 MB
    # (8, 4 and 4 slices of M x N floats), each more than the buffer holds.
    shapes = [(64, 1024), (64, 4096), (128, 4096)]

    def grow_partials(rep):
        m, n = shapes[rep]
        ok(lib.cuda_gemm_int8(big.vp, a.vp, w.vp, sc.vp, m, K, n, True), "eager larger GEMM")

    try:
        outs = {"y": (E2, (64, GN))}
        replay_and_check(
            lib, hip, stream, outs,
            lambda o: lib.cuda_gemm_int8(o["y"].vp, inp["a64"].vp, inp["wq"].vp, inp["wsc"].vp, 64, GK, GN, True),
            True, "split-K GEMM across buffer growth", between=grow_partials)
    finally:
        for b in (a, w, sc, big):
            b.free()

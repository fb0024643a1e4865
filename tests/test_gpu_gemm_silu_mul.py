"""ng_gemm_int8_silu_mul on the GPU: gate/up and SwiGLU in one call.

Bar: out, gate and up are bit-identical to the calls they replace,
ng_gemm_int8_shared_a (gate and up on one A, each bit for bit its own
cuda_gemm_int8) and then cuda_silu_mul(out, gate, up), on the same inputs:
in the fused GEMV launch (M <= 4 on the GEMV kernel's shapes), in the split
kernel's SwiGLU form (3 to 128 rows where gate/up takes the two-group split
kernel with one K slice: every one of its four shapes, ragged N), in the
split-K reduction's SwiGLU form (the one-group split shapes with several K
slices: Llama-2-7B and TinyLlama widths, each of the four shapes, N not a
multiple of 4), and where the call is the two calls (the small-M MFMA kernel,
token tiles, K not a multiple of 16, M > 128), with out apart from
gate and up or in place on either, as the engine runs SwiGLU in place on gate
(layer.cu:585-588).
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(71))

# (M, K, N): Mistral-7B and Llama-2-7B gate/up at 1-2 tokens, M = 3-4 below
# N = 8192, ragged N and K (K % 1024 != 0), tiny shapes; then shapes that are
# the two calls.
FUSED = [(1, 4096, 14336), (2, 4096, 14336), (1, 4096, 11008), (2, 5120, 13824), (3, 4096, 4096), (4, 2048, 5000),
         (1, 4112, 1000), (3, 2064, 17), (1, 16, 5)]
# the split kernel's SwiGLU form: <1,4,2> at 3-16 rows, <2,4,2> at 17-32,
# <4,4,2> at 33-64, <8,4,2> at 65-128 (Mistral-7B), N not a multiple of 32
# (12300), Llama-2-13B's width, K with a half last batch (4160)
SPLIT = [(3, 4096, 14336), (4, 4096, 14336), (8, 4096, 14336), (16, 4096, 14336), (17, 4096, 14336),
         (32, 4096, 14336), (40, 4096, 14336), (64, 4096, 14336), (65, 4096, 14336), (128, 4096, 14336),
         (8, 4096, 12300), (20, 5120, 13824), (12, 4160, 12400)]
# the reduction's SwiGLU form: <1,4,1> at 3-16 rows, <2,4,1> at 17-32,
# <4,4,1> at 33-64, <8,4,1> at 65-128 (Llama-2-7B: 2 K slices), TinyLlama's
# width (3 slices), N % 4 != 0 (one output per thread), K with a half last
# batch
SLICED = [(3, 4096, 11008), (8, 4096, 11008), (16, 4096, 11008), (17, 4096, 11008), (40, 4096, 11008),
          (100, 4096, 11008), (24, 2048, 5632), (24, 2048, 5634), (8, 4160, 11000)]
TWO_CALLS = [(8, 4096, 4096), (1, 4104, 64), (40, 1024, 2048), (200, 1024, 2048)]


def f16bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def problem(M, K, N, big=False):
    a = f16bits(RNG.standard_normal((M, K)) * (8 if big else 1))
    bg = RNG.integers(-128, 128, size=(N, K)).astype(np.int8)
    bu = RNG.integers(-128, 128, size=(N, K)).astype(np.int8)
    sg = RNG.uniform(1e-3, 1e-2, N).astype(np.float16).astype(np.float32)
    su = RNG.uniform(1e-3, 1e-2, N).astype(np.float16).astype(np.float32)
    return a, bg, bu, sg, su


def run(lib, a, bg, bu, sg, su, fused: bool, alias: str = ""):
    M, K = a.shape
    N = bg.shape[0]
    ab, bgb, bub, sgb, sub = dev(a), dev(bg), dev(bu), dev(sg), dev(su)
    gb, ub = empty(M * N * 2), empty(M * N * 2)
    ob = gb if alias == "gate" else ub if alias == "up" else empty(M * N * 2)
    if fused:
        ok(lib.ng_gemm_int8_silu_mul(ob.vp, gb.vp, ub.vp, ab.vp, bgb.vp, sgb.vp, bub.vp, sub.vp, M, K, N),
           "ng_gemm_int8_silu_mul")
    else:
        cnt = 2
        ok(lib.ng_gemm_int8_shared_a(cnt, (C.c_void_p * 2)(gb.ptr, ub.ptr), ab.vp, (C.c_void_p * 2)(bgb.ptr, bub.ptr),
                                     (C.c_void_p * 2)(sgb.ptr, sub.ptr), (C.c_int * 2)(N, N), M, K),
           "ng_gemm_int8_shared_a")
        ok(lib.cuda_silu_mul(ob.vp, gb.vp, ub.vp, M * N), "cuda_silu_mul")
    out = {"out": get(ob, np.uint16, (M, N))}
    if alias != "gate":
        out["gate"] = get(gb, np.uint16, (M, N))
    if alias != "up":
        out["up"] = get(ub, np.uint16, (M, N))
    return out


def check(got, want):
    assert got.keys() == want.keys()
    for k in want:
        assert_bits_equal(got[k], want[k], k)


@pytest.mark.parametrize("M,K,N", FUSED + SPLIT + SLICED + TWO_CALLS)
def test_silu_mul_is_the_two_calls(lib, M, K, N):
    banner(f"gemm_int8_silu_mul M={M} K={K} N={N}")
    p = problem(M, K, N)
    check(run(lib, *p, fused=True), run(lib, *p, fused=False))


@pytest.mark.parametrize("alias", ["gate", "up"])
@pytest.mark.parametrize("M,K,N", [(1, 4096, 14336), (2, 4112, 1000), (8, 1024, 2048), (8, 4096, 14336),
                                   (100, 4096, 12300), (8, 4096, 11008), (24, 2048, 5634)])
def test_silu_mul_in_place(lib, M, K, N, alias):
    banner(f"gemm_int8_silu_mul in place on {alias} M={M} K={K} N={N}")
    p = problem(M, K, N)
    check(run(lib, *p, fused=True, alias=alias), run(lib, *p, fused=False, alias=alias))


def test_silu_mul_large_and_nonfinite(lib):
    """Large activations (gate values that overflow fp16 to inf, sig at its
    limits) and inf / NaN in A: the same bits as the two calls."""
    banner("gemm_int8_silu_mul large and non-finite")
    a, bg, bu, sg, su = problem(2, 4096, 4096, big=True)
    a[0, 5] = 0x7C00
    a[1, 77] = 0x7E00
    check(run(lib, a, bg, bu, sg, su, fused=True), run(lib, a, bg, bu, sg, su, fused=False))


def test_silu_mul_consecutive_calls(lib):
    banner("gemm_int8_silu_mul: a call, then a smaller one")
    for M, K, N in ((2, 4096, 14336), (1, 2048, 300), (64, 4096, 14336), (8, 4096, 14336)):
        p = problem(M, K, N)
        check(run(lib, *p, fused=True), run(lib, *p, fused=False))


def test_silu_mul_unaligned_is_the_two_calls(lib):
    """A 2 bytes off 16-byte alignment: the two calls, their bits."""
    banner("gemm_int8_silu_mul unaligned A")
    M, K, N = 2, 4096, 1000
    a, bg, bu, sg, su = problem(M, K, N)
    outs = []
    for fused in (True, False):
        ab = empty(a.nbytes + 2)
        ab.upload(np.concatenate([np.zeros(1, np.uint16), a.ravel()]))
        bgb, bub, sgb, sub = dev(bg), dev(bu), dev(sg), dev(su)
        gb, ub, ob = empty(M * N * 2), empty(M * N * 2), empty(M * N * 2)
        if fused:
            ok(lib.ng_gemm_int8_silu_mul(ob.vp, gb.vp, ub.vp, ab.offset(2), bgb.vp, sgb.vp, bub.vp, sub.vp, M, K, N),
               "ng_gemm_int8_silu_mul")
        else:
            ok(lib.ng_gemm_int8_shared_a(2, (C.c_void_p * 2)(gb.ptr, ub.ptr), ab.offset(2),
                                         (C.c_void_p * 2)(bgb.ptr, bub.ptr), (C.c_void_p * 2)(sgb.ptr, sub.ptr),
                                         (C.c_int * 2)(N, N), M, K), "ng_gemm_int8_shared_a")
            ok(lib.cuda_silu_mul(ob.vp, gb.vp, ub.vp, M * N), "cuda_silu_mul")
        outs.append([get(x, np.uint16, (M, N)) for x in (ob, gb, ub)])
    for name, g, w in zip(("out", "gate", "up"), outs[0], outs[1]):
        assert_bits_equal(g, w, name)

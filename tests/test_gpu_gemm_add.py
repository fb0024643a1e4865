"""ng_gemm_int8_add on the GPU: a product and the residual add after it.

Bar: c and out are bit-identical to the calls they replace,
cuda_gemm_int8(c, a, b, scale, M, K, N, true) and then cuda_add(out, c,
residual, M N), on the same inputs: in the fused GEMV launch (M <= 4 on the
GEMV kernel's shapes), in the split-K reduction's epilogue (up to 128 rows on
the split kernel with several K slices, with 4-wide and scalar reductions, and
on the prefill kernel's 128 x 128 tiles with K slices), after a launch of one K
slice or the small-M MFMA kernel (the add as its own launch), and as the two
calls (K not a multiple of 16, 4096 rows and more), with
out apart from c and the residual or in place on either (the engine writes
the layer output apart, layer.cu:593-598).
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import assert_bits_equal, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(73))

# (M, K, N): Mistral-7B's down projection at 1-2 tokens, Llama-2-7B's, M = 3-4
# below 8192, ragged N and K, tiny shapes (the fused GEMV launch); down at
# 4, 8, 20 and 64 tokens and token tiles at 40 (the split reduction with the
# add), N not a multiple of 4 (its scalar form), gate's shape at 8 tokens
# (one K slice) and the small-M MFMA kernel; then the two calls.
FUSED = [(1, 14336, 4096), (2, 14336, 4096), (1, 11008, 4096), (2, 13824, 5120), (3, 4096, 4096), (4, 2048, 5000),
         (1, 4112, 1000), (3, 2064, 17), (1, 16, 5)]
SPLIT = [(4, 14336, 4096), (8, 14336, 4096), (20, 4096, 4096), (64, 14336, 4096), (40, 1024, 2048),
         (24, 4096, 1002), (8, 4096, 14336), (8, 4096, 4096)]
# the prefill kernel: 128 x 128 tiles with K slices (512, 1000 and 2048 rows,
# the add in the reduction), 256 x 256 tiles in one slice (3072 rows: the add
# after it)
PREFILL = [(512, 14336, 4096), (1000, 4096, 1000), (2048, 14336, 4096), (3072, 4096, 4096)]
TWO_CALLS = [(1, 4104, 64), (4096, 1024, 512)]


def f16bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def problem(M, K, N):
    a = f16bits(RNG.standard_normal((M, K)))
    b = RNG.integers(-128, 128, size=(N, K)).astype(np.int8)
    s = RNG.uniform(1e-3, 1e-2, N).astype(np.float16).astype(np.float32)
    res = f16bits(RNG.standard_normal((M, N)) * 4)
    return a, b, s, res


def run(lib, a, b, s, res, fused: bool, alias: str = ""):
    M, K = a.shape
    N = b.shape[0]
    ab, bb, sb, rb = dev(a), dev(b), dev(s), dev(res)
    cb = empty(M * N * 2)
    ob = cb if alias == "c" else rb if alias == "residual" else empty(M * N * 2)
    if fused:
        ok(lib.ng_gemm_int8_add(ob.vp, cb.vp, ab.vp, bb.vp, sb.vp, rb.vp, M, K, N), "ng_gemm_int8_add")
    else:
        ok(lib.cuda_gemm_int8(cb.vp, ab.vp, bb.vp, sb.vp, M, K, N, True), "cuda_gemm_int8")
        ok(lib.cuda_add(ob.vp, cb.vp, rb.vp, M * N), "cuda_add")
    out = {"out": get(ob, np.uint16, (M, N))}
    if alias != "c":
        out["c"] = get(cb, np.uint16, (M, N))
    return out


def check(got, want):
    assert got.keys() == want.keys()
    for k in want:
        assert_bits_equal(got[k], want[k], k)


@pytest.mark.parametrize("M,K,N", FUSED + SPLIT + PREFILL + TWO_CALLS)
def test_gemm_add_is_the_two_calls(lib, ora, M, K, N):
    banner(f"gemm_int8_add M={M} K={K} N={N}")
    p = problem(M, K, N)
    got = run(lib, *p, fused=True)
    check(got, run(lib, *p, fused=False))
    assert_bits_equal(got["out"], ora.elementwise("add", got["c"], p[3]), "out vs oracle add of c and the residual")


@pytest.mark.parametrize("alias", ["c", "residual"])
@pytest.mark.parametrize("M,K,N", [(1, 14336, 4096), (2, 4112, 1000), (8, 1024, 2048), (8, 14336, 4096),
                                   (24, 4096, 1002)])
def test_gemm_add_in_place(lib, M, K, N, alias):
    banner(f"gemm_int8_add in place on {alias} M={M} K={K} N={N}")
    p = problem(M, K, N)
    check(run(lib, *p, fused=True, alias=alias), run(lib, *p, fused=False, alias=alias))


def test_gemm_add_consecutive_calls(lib):
    banner("gemm_int8_add: a call, then a smaller one")
    for M, K, N in ((2, 14336, 4096), (1, 2048, 300), (64, 14336, 4096), (8, 14336, 4096)):
        p = problem(M, K, N)
        check(run(lib, *p, fused=True), run(lib, *p, fused=False))


@pytest.mark.parametrize("M,K,N", [(1, 4096, 1000), (8, 14336, 4096)])
def test_gemm_add_unaligned_is_the_two_calls(lib, M, K, N):
    """A and the residual 2 bytes off 16-byte alignment: the two calls, their bits."""
    banner(f"gemm_int8_add unaligned A and residual M={M}")
    a, b, s, res = problem(M, K, N)
    outs = []
    for fused in (True, False):
        ab, rb = empty(a.nbytes + 2), empty(res.nbytes + 2)
        ab.upload(np.concatenate([np.zeros(1, np.uint16), a.ravel()]))
        rb.upload(np.concatenate([np.zeros(1, np.uint16), res.ravel()]))
        bb, sb = dev(b), dev(s)
        cb, ob = empty(M * N * 2), empty(M * N * 2)
        if fused:
            ok(lib.ng_gemm_int8_add(ob.vp, cb.vp, ab.offset(2), bb.vp, sb.vp, rb.offset(2), M, K, N), "ng_gemm_int8_add")
        else:
            ok(lib.cuda_gemm_int8(cb.vp, ab.offset(2), bb.vp, sb.vp, M, K, N, True), "cuda_gemm_int8")
            ok(lib.cuda_add(ob.vp, cb.vp, rb.offset(2), M * N), "cuda_add")
        outs.append((get(ob, np.uint16, (M, N)), get(cb, np.uint16, (M, N))))
    assert_bits_equal(outs[0][0], outs[1][0], "out")
    assert_bits_equal(outs[0][1], outs[1][1], "c")


@pytest.mark.parametrize("M,K,N", [(8, 14336, 4096), (1, 14336, 4096)])
def test_gemm_add_unaligned_residual(lib, M, K, N):
    """Only the residual (and out) 2 bytes off 8-byte alignment: the split
    reduction takes its scalar form with the add; the GEMV launch is the two
    calls. Their bits either way."""
    banner(f"gemm_int8_add unaligned residual M={M}")
    a, b, s, res = problem(M, K, N)
    outs = []
    for fused in (True, False):
        ab, bb, sb = dev(a), dev(b), dev(s)
        rb, ob = empty(res.nbytes + 2), empty(res.nbytes + 2)
        rb.upload(np.concatenate([np.zeros(1, np.uint16), res.ravel()]))
        cb = empty(M * N * 2)
        if fused:
            ok(lib.ng_gemm_int8_add(ob.offset(2), cb.vp, ab.vp, bb.vp, sb.vp, rb.offset(2), M, K, N), "ng_gemm_int8_add")
        else:
            ok(lib.cuda_gemm_int8(cb.vp, ab.vp, bb.vp, sb.vp, M, K, N, True), "cuda_gemm_int8")
            ok(lib.cuda_add(ob.offset(2), cb.vp, rb.offset(2), M * N), "cuda_add")
        outs.append((get(ob, np.uint16, (M * N + 1,))[1:].reshape(M, N), get(cb, np.uint16, (M, N))))
    assert_bits_equal(outs[0][0], outs[1][0], "out")
    assert_bits_equal(outs[0][1], outs[1][1], "c")

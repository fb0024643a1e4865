"""ng_rmsnorm_qkv_rope_int8 on the GPU: RMSNorm, q/k/v and RoPE on q and k.

Bar: normed, q, k and v are bit-identical to the calls the entry point
replaces, ng_rmsnorm_gemm_int8_shared_a (itself bit for bit cuda_rmsnorm and
one cuda_gemm_int8 per projection) and then ng_rope_qk_with_theta(q, q, k, k,
positions, 1, M, Hq, Hkv, D, 0, theta), on the same inputs: where the
rotation runs in the products' launch (decode shapes: the GEMV kernel at one
or two tokens, at most 1024 blocks, D a multiple of 8) and where the call is
the two calls. q and k are also checked against the oracle's RoPE applied to
the separately computed products, so the rotation is pinned on its own.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, assert_close16, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(79))
EPS = 1e-5

# (M, hidden, Hq, Hkv, D, theta, positions): Mistral-7B at 1-2 tokens,
# TinyLlama (D = 64), D = 256 and D = 96 (one head pair per block group),
# positions up to 32768, theta 1e4 and 1e6; then the two calls: Mistral-7B at
# 4 tokens, Llama-2-7B (Hkv = Hq: 1536 blocks), D not a multiple of 8.
FUSED = [
    (1, 4096, 32, 8, 128, 1e6, [17]),
    (2, 4096, 32, 8, 128, 1e6, [4095, 32768]),
    (1, 2048, 32, 4, 64, 1e4, [0]),
    (2, 2048, 32, 4, 64, 1e4, [1, 2]),
    (1, 2048, 8, 1, 256, 1e4, [777]),
    (2, 3072, 32, 8, 96, 1e4, [123, 9000]),
]
TWO_CALLS = [
    (4, 4096, 32, 8, 128, 1e6, [5, 6, 7, 8]),
    (1, 4096, 32, 32, 128, 1e4, [100]),
    (1, 1024, 4, 2, 6, 1e4, [3]),
]


def f16bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def problem(M, hidden, hq, hkv, D):
    x = f16bits(RNG.standard_normal((M, hidden)) * 2)
    w = f16bits(1 + 0.05 * RNG.standard_normal(hidden))
    ns = [hq * D, hkv * D, hkv * D]
    qs = [RNG.integers(-128, 128, size=(n, hidden)).astype(np.int8) for n in ns]
    scales = [RNG.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32) for n in ns]
    return x, w, qs, scales


def ptrs(bufs):
    return (C.c_void_p * len(bufs))(*[b.ptr for b in bufs])


def run(lib, case, fused: bool, p):
    M, hidden, hq, hkv, D, theta, pos = case
    x, w, qs, scales = p
    xb, wb = dev(x), dev(w)
    posb = dev(np.asarray(pos, np.int32))
    qb = [dev(q) for q in qs]
    sb = [dev(s) for s in scales]
    ns = [q.shape[0] for q in qs]
    yb = empty(M * hidden * 2)
    cb = [empty(M * n * 2) for n in ns]
    ip = C.cast(C.c_void_p(posb.ptr), C.POINTER(C.c_int))
    if fused:
        ok(lib.ng_rmsnorm_qkv_rope_int8(yb.vp, cb[0].vp, cb[1].vp, cb[2].vp, xb.vp, wb.vp, C.c_float(EPS), ptrs(qb),
                                        ptrs(sb), ip, M, hidden, hq, hkv, D, C.c_float(theta)),
           "ng_rmsnorm_qkv_rope_int8")
    else:
        ok(lib.ng_rmsnorm_gemm_int8_shared_a(3, yb.vp, ptrs(cb), xb.vp, wb.vp, C.c_float(EPS), ptrs(qb), ptrs(sb),
                                             (C.c_int * 3)(*ns), M, hidden), "ng_rmsnorm_gemm_int8_shared_a")
        ok(lib.ng_rope_qk_with_theta(cb[0].vp, cb[0].vp, cb[1].vp, cb[1].vp, ip, 1, M, hq, hkv, D, 0,
                                     C.c_float(theta)), "ng_rope_qk_with_theta")
    out = {"normed": get(yb, np.uint16, (M, hidden))}
    for name, c, n in zip(("q", "k", "v"), cb, ns):
        out[name] = get(c, np.uint16, (M, n))
    return out


def unrotated(lib, case, p):
    """q and k before RoPE: the norm and the products alone."""
    M, hidden, hq, hkv, D, theta, pos = case
    x, w, qs, scales = p
    xb, wb = dev(x), dev(w)
    qb = [dev(q) for q in qs]
    sb = [dev(s) for s in scales]
    ns = [q.shape[0] for q in qs]
    yb = empty(M * hidden * 2)
    cb = [empty(M * n * 2) for n in ns]
    ok(lib.ng_rmsnorm_gemm_int8_shared_a(3, yb.vp, ptrs(cb), xb.vp, wb.vp, C.c_float(EPS), ptrs(qb), ptrs(sb),
                                         (C.c_int * 3)(*ns), M, hidden), "ng_rmsnorm_gemm_int8_shared_a")
    return [get(c, np.uint16, (M, n)) for c, n in zip(cb[:2], ns[:2])]


@pytest.mark.parametrize("case", FUSED + TWO_CALLS, ids=lambda c: f"M{c[0]}-H{c[1]}-{c[2]}x{c[3]}-D{c[4]}")
def test_qkv_rope_is_the_two_calls(lib, ora, case):
    M, hidden, hq, hkv, D, theta, pos = case
    banner(f"rmsnorm_qkv_rope_int8 M={M} hidden={hidden} heads={hq}/{hkv} D={D} theta={theta} pos={pos}")
    p = problem(M, hidden, hq, hkv, D)
    got = run(lib, case, True, p)
    want = run(lib, case, False, p)
    for k in want:
        assert_bits_equal(got[k], want[k], k)
    # the rotation on its own: the oracle's RoPE of the unrotated products, to
    # the RoPE bar (2 ulp or 1e-2)
    q0, k0 = unrotated(lib, case, p)
    posa = np.asarray(pos, np.int32)
    for name, t0, nh in (("q", q0, hq), ("k", k0, hkv)):
        ref = ora.rope(t0.reshape(M, nh, D), posa, 0, theta).reshape(M, nh * D)
        assert_close16(got[name], ref, "f16", f"{name} vs oracle RoPE")


def test_qkv_rope_consecutive_calls(lib):
    banner("rmsnorm_qkv_rope_int8: a call, then a smaller one")
    for case in (FUSED[1], FUSED[2]):
        p = problem(*case[:5])
        got, want = run(lib, case, True, p), run(lib, case, False, p)
        for k in want:
            assert_bits_equal(got[k], want[k], k)


def test_qkv_rope_unaligned_is_the_two_calls(lib):
    """x 2 bytes off 16-byte alignment: the two calls, their bits."""
    banner("rmsnorm_qkv_rope_int8 unaligned x")
    M, hidden, hq, hkv, D, theta = 1, 2048, 32, 4, 64, 1e4
    x, w, qs, scales = problem(M, hidden, hq, hkv, D)
    ns = [q.shape[0] for q in qs]
    outs = []
    for fused in (True, False):
        xb = empty(x.nbytes + 2)
        xb.upload(np.concatenate([np.zeros(1, np.uint16), x.ravel()]))
        wb, posb = dev(w), dev(np.array([42], np.int32))
        ip = C.cast(C.c_void_p(posb.ptr), C.POINTER(C.c_int))
        qb, sb = [dev(q) for q in qs], [dev(s) for s in scales]
        yb = empty(M * hidden * 2)
        cb = [empty(M * n * 2) for n in ns]
        if fused:
            ok(lib.ng_rmsnorm_qkv_rope_int8(yb.vp, cb[0].vp, cb[1].vp, cb[2].vp, xb.offset(2), wb.vp, C.c_float(EPS),
                                            ptrs(qb), ptrs(sb), ip, M, hidden, hq, hkv, D, C.c_float(theta)), "fused")
        else:
            ok(lib.ng_rmsnorm_gemm_int8_shared_a(3, yb.vp, ptrs(cb), xb.offset(2), wb.vp, C.c_float(EPS), ptrs(qb),
                                                 ptrs(sb), (C.c_int * 3)(*ns), M, hidden), "norm + q/k/v")
            ok(lib.ng_rope_qk_with_theta(cb[0].vp, cb[0].vp, cb[1].vp, cb[1].vp, ip, 1, M, hq, hkv, D, 0,
                                         C.c_float(theta)), "rope")
        outs.append([get(yb, np.uint16, (M, hidden))] + [get(c, np.uint16, (M, n)) for c, n in zip(cb, ns)])
    for name, g, wv in zip(("normed", "q", "k", "v"), outs[0], outs[1]):
        assert_bits_equal(g, wv, name)

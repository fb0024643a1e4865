"""ng_rmsnorm_gemm_int8_shared_a / ng_add_rmsnorm_gemm_int8_shared_a on the GPU.

Bar: normed, residual_out and every C_i are bit-identical to the two calls
they replace, cuda_rmsnorm (cuda_add_rmsnorm) and then ng_gemm_int8_shared_a
on the normalised rows, on the same inputs. That holds both in the fused
launch (one or two rows, every product on the GEMV kernel with one shape,
K <= 8192, at most 1024 blocks, outputs apart from inputs) and where the call
is the two calls (three or more rows, more blocks, K past 8192, mixed shapes,
in-place buffers). The two calls are pinned
elsewhere (the norms against the oracle, the shared products against
cuda_gemm_int8); normed is also checked against the oracle here. Rows whose
sum of squares sits on an fp32 rounding boundary take the norm's exact limb
reduction inside the fused kernel too.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, banner, dev, empty, get, ok
from test_gpu_norm import adversarial_rows

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(53))
EPS = 1e-5

# The fused launch takes one or two rows, every product on the GEMV kernel
# with one shape, K <= 8192 and at most 1024 blocks of 8 rows of B. FUSED:
# q/k/v at Mistral-7B (768 blocks), Llama-2-13B widths with fewer rows, K of
# one segment per wave (K <= 4096) and of two (up to 8192, one wave with a
# single segment at K = 6160), waves with no segment (K = 2064, 16), ragged K
# and rows of B. TWO_CALLS: three or four rows, more blocks (gate/up,
# Llama-2-13B's q/k/v), K past 8192, M > 4, products of two GEMV shapes, K not
# a multiple of 16.
FUSED = [
    (1, 4096, [4096, 1024, 1024]),
    (2, 4096, [4096, 1024, 1024]),
    (1, 5120, [4096, 1024, 1024]),
    (2, 5120, [1024, 1024, 1024]),
    (1, 8192, [4096, 1000]),
    (2, 8192, [3000, 4096]),
    (2, 6160, [1000, 77]),
    (1, 4112, [1000, 333, 7, 64]),
    (2, 2064, [17, 1, 40]),
    (1, 16, [5, 9]),
]
TWO_CALLS = [
    (3, 4096, [1024, 1024]),
    (4, 4096, [2048, 1024, 1024]),
    (4, 5120, [1024, 1024, 1024]),
    (3, 6160, [1000, 77]),
    (4, 4096, [4096, 1024, 1024]),
    (1, 4096, [14336, 14336]),
    (2, 4096, [14336, 14336]),
    (1, 5120, [5120, 5120, 5120]),
    (2, 12288, [3000, 4096]),
    (4, 8192, [4096, 1024]),
    (8, 4096, [4096, 1024, 1024]),
    (3, 4096, [4096, 12300]),
    (1, 4104, [64, 8]),
]


def f16bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def problem(M: int, K: int, ns):
    x = f16bits(RNG.standard_normal((M, K)) * 2)
    r = f16bits(RNG.standard_normal((M, K)))
    w = f16bits(1 + 0.05 * RNG.standard_normal(K))
    qs = [RNG.integers(-128, 128, size=(n, K)).astype(np.int8) for n in ns]
    scales = [RNG.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32) for n in ns]
    return x, r, w, qs, scales


def ptrs(bufs):
    return (C.c_void_p * len(bufs))(*[b.ptr for b in bufs])


class Buffers:
    """Device copies of one problem; add=True also holds the residual."""

    def __init__(self, x, r, w, qs, scales, add: bool, inplace: bool = False):
        M, K = x.shape
        self.M, self.K, self.ns = M, K, [q.shape[0] for q in qs]
        self.xb, self.wb = dev(x), dev(w)
        self.rb = dev(r) if add else None
        self.qb = [dev(q) for q in qs]
        self.sb = [dev(s) for s in scales]
        self.cb = [empty(M * n * 2) for n in self.ns]
        # in place as the engine's FFN step: normed over x, residual_out over residual_in
        self.yb = self.xb if inplace else empty(M * K * 2)
        self.rob = (self.rb if inplace else empty(M * K * 2)) if add else None

    def products(self):
        cnt = len(self.ns)
        return (ptrs(self.qb), ptrs(self.sb), (C.c_int * cnt)(*self.ns))

    def outputs(self):
        out = {"normed": get(self.yb, np.uint16, (self.M, self.K))}
        if self.rob is not None:
            out["residual_out"] = get(self.rob, np.uint16, (self.M, self.K))
        for i, (c, n) in enumerate(zip(self.cb, self.ns)):
            out[f"C_{i}"] = get(c, np.uint16, (self.M, n))
        return out


def fused(lib, x, r, w, qs, scales, add: bool, inplace: bool = False):
    bf = Buffers(x, r, w, qs, scales, add, inplace)
    b, s, n = bf.products()
    cnt = len(qs)
    if add:
        rc = lib.ng_add_rmsnorm_gemm_int8_shared_a(cnt, bf.yb.vp, bf.rob.vp, ptrs(bf.cb), bf.xb.vp, bf.rb.vp, bf.wb.vp,
                                                   C.c_float(EPS), b, s, n, bf.M, bf.K)
    else:
        rc = lib.ng_rmsnorm_gemm_int8_shared_a(cnt, bf.yb.vp, ptrs(bf.cb), bf.xb.vp, bf.wb.vp, C.c_float(EPS),
                                               b, s, n, bf.M, bf.K)
    ok(rc, "norm + gemm_int8_shared_a")
    return bf.outputs()


def two_calls(lib, x, r, w, qs, scales, add: bool):
    bf = Buffers(x, r, w, qs, scales, add)
    if add:
        ok(lib.cuda_add_rmsnorm(bf.yb.vp, bf.rob.vp, bf.xb.vp, bf.rb.vp, bf.wb.vp, bf.M, bf.K, C.c_float(EPS)),
           "cuda_add_rmsnorm")
    else:
        ok(lib.cuda_rmsnorm(bf.yb.vp, bf.xb.vp, bf.wb.vp, bf.M, bf.K, C.c_float(EPS)), "cuda_rmsnorm")
    b, s, n = bf.products()
    ok(lib.ng_gemm_int8_shared_a(len(qs), ptrs(bf.cb), bf.yb.vp, b, s, n, bf.M, bf.K), "ng_gemm_int8_shared_a")
    return bf.outputs()


def check(got, want):
    assert got.keys() == want.keys()
    for k in want:
        assert_bits_equal(got[k], want[k], k)


@pytest.mark.parametrize("add", [False, True], ids=["rmsnorm", "add_rmsnorm"])
@pytest.mark.parametrize("M,K,ns", FUSED + TWO_CALLS)
def test_norm_shared_is_the_two_calls(lib, ora, M, K, ns, add):
    banner(f"{'add_' if add else ''}rmsnorm_gemm_int8_shared_a M={M} K={K} n={ns}")
    x, r, w, qs, scales = problem(M, K, ns)
    got = fused(lib, x, r, w, qs, scales, add)
    check(got, two_calls(lib, x, r, w, qs, scales, add))
    if add:
        want_y, want_r = ora.add_rmsnorm(x, r, w, EPS)
        assert_bits_equal(got["residual_out"], want_r, "residual_out vs oracle")
    else:
        want_y = ora.rmsnorm(x, w, EPS)
    assert_bits_equal(got["normed"], want_y, "normed vs oracle")


@pytest.mark.parametrize("add", [False, True], ids=["rmsnorm", "add_rmsnorm"])
@pytest.mark.parametrize("K", [4096, 5120, 4112, 8192])
def test_norm_shared_exact_path_rows(lib, ora, K, add):
    """Rows whose sum of squares the fp64 fast path cannot round: the fused
    kernel's exact limb reduction, one, two and four rows at a time."""
    banner(f"{'add_' if add else ''}rmsnorm_gemm_int8_shared_a exact-path rows K={K}")
    adv = f16bits(adversarial_rows(K))
    w = f16bits(np.ones(K))
    for rows in ([0], [3, 4], [0, 1, 2, 4]):
        x = adv[rows]
        M = len(rows)
        r = np.zeros_like(x)
        _, _, _, qs, scales = problem(M, K, [1024, 512])
        got = fused(lib, x, r, w, qs, scales, add)
        check(got, two_calls(lib, x, r, w, qs, scales, add))
        want_y = ora.add_rmsnorm(x, r, w, EPS)[0] if add else ora.rmsnorm(x, w, EPS)
        assert_bits_equal(got["normed"], want_y, f"rows {rows} normed vs oracle")


@pytest.mark.parametrize("add", [False, True], ids=["rmsnorm", "add_rmsnorm"])
def test_norm_shared_nonfinite_rows(lib, add):
    """inf and NaN in the input rows: the fused launch gives the two calls'
    bits (the same instructions on the same values)."""
    M, K = 2, 4096
    banner(f"{'add_' if add else ''}rmsnorm_gemm_int8_shared_a non-finite rows")
    x, r, w, qs, scales = problem(M, K, [4096, 1024])
    x[0, 17] = 0x7C00   # +inf
    x[1, 4000] = 0x7E00  # NaN
    check(fused(lib, x, r, w, qs, scales, add), two_calls(lib, x, r, w, qs, scales, add))


@pytest.mark.parametrize("add", [False, True], ids=["rmsnorm", "add_rmsnorm"])
@pytest.mark.parametrize("M,K,ns", [(1, 4096, [14336, 14336]), (4, 4096, [4096, 1024, 1024])])
def test_norm_shared_in_place(lib, M, K, ns, add):
    """normed over x (and residual_out over residual_in), as the engine's FFN
    step runs: the two calls, with their bits."""
    banner(f"{'add_' if add else ''}rmsnorm_gemm_int8_shared_a in place M={M} K={K}")
    x, r, w, qs, scales = problem(M, K, ns)
    check(fused(lib, x, r, w, qs, scales, add, inplace=True), two_calls(lib, x, r, w, qs, scales, add))


def test_norm_shared_consecutive_calls(lib):
    banner("add_rmsnorm_gemm_int8_shared_a: a call, then a smaller one")
    for M, K, ns in ((2, 4096, [2048, 1024, 1024]), (1, 2048, [300, 48])):
        x, r, w, qs, scales = problem(M, K, ns)
        check(fused(lib, x, r, w, qs, scales, True), two_calls(lib, x, r, w, qs, scales, True))


@pytest.mark.parametrize("add", [False, True], ids=["rmsnorm", "add_rmsnorm"])
def test_norm_shared_unaligned_is_the_two_calls(lib, add):
    """x (and the residual) 2 bytes off 16-byte alignment: the two calls, their bits."""
    banner(f"{'add_' if add else ''}rmsnorm_gemm_int8_shared_a unaligned rows")
    M, K, ns = 1, 4096, [4096, 1024, 1024]
    x, r, w, qs, scales = problem(M, K, ns)
    outs = []
    for fused_call in (True, False):
        xb, rb = empty(x.nbytes + 2), empty(r.nbytes + 2)
        xb.upload(np.concatenate([np.zeros(1, np.uint16), x.ravel()]))
        rb.upload(np.concatenate([np.zeros(1, np.uint16), r.ravel()]))
        wb = dev(w)
        qb, sb = [dev(q) for q in qs], [dev(s) for s in scales]
        yb, rob = empty(M * K * 2), empty(M * K * 2)
        cb = [empty(M * n * 2) for n in ns]
        b3, s3, n3 = ptrs(qb), ptrs(sb), (C.c_int * 3)(*ns)
        if fused_call and add:
            ok(lib.ng_add_rmsnorm_gemm_int8_shared_a(3, yb.vp, rob.vp, ptrs(cb), xb.offset(2), rb.offset(2), wb.vp,
                                                     C.c_float(EPS), b3, s3, n3, M, K), "fused")
        elif fused_call:
            ok(lib.ng_rmsnorm_gemm_int8_shared_a(3, yb.vp, ptrs(cb), xb.offset(2), wb.vp, C.c_float(EPS), b3, s3, n3,
                                                 M, K), "fused")
        else:
            if add:
                ok(lib.cuda_add_rmsnorm(yb.vp, rob.vp, xb.offset(2), rb.offset(2), wb.vp, M, K, C.c_float(EPS)), "norm")
            else:
                ok(lib.cuda_rmsnorm(yb.vp, xb.offset(2), wb.vp, M, K, C.c_float(EPS)), "norm")
            ok(lib.ng_gemm_int8_shared_a(3, ptrs(cb), yb.vp, b3, s3, n3, M, K), "ng_gemm_int8_shared_a")
        o = [get(yb, np.uint16, (M, K))] + [get(c, np.uint16, (M, n)) for c, n in zip(cb, ns)]
        if add:
            o.append(get(rob, np.uint16, (M, K)))
        outs.append(o)
    for i, (g, wv) in enumerate(zip(outs[0], outs[1])):
        assert_bits_equal(g, wv, f"output {i}")

"""ng_gemm_int8_shared_a on the GPU: int8-weight products that share one A.

Bars:
  * every C_i is bit-identical to its own cuda_gemm_int8(c_i, a, b_i, scale_i,
    M, K, n_i, true) on the same inputs (random activations, random codes and
    scales), whether a product ran in a shared launch (with the products of
    the same launch shape: the GEMV kernel, the small-M MFMA kernel, or the
    split kernel and its reduction) or as its own call;
  * exact inputs (activations on a grid 2^-e, so that every partial sum of
    A @ q is exact in fp32) give fp16(fp32(sum_k a_k q_k) * scale[n]) bit for
    bit, the weight-streaming paths' formula, checked against numpy;
  * a second call with other inputs and fewer products leaves nothing behind.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(47))

# (M, K, [n_i]): q/k/v and gate/up at Mistral-7B and Llama-2-13B sizes on the
# GEMV kernel (M <= 4), ragged rows of B and K (K % 1024 != 0), four products,
# one product, tiny K; q/k/v on the small-M MFMA kernel (4 < M <= 16); then
# the split kernel's shared forms and the sets that cannot share a launch.
SETS = [
    (1, 4096, [4096, 1024, 1024]),
    (2, 4096, [4096, 1024, 1024]),
    (3, 4096, [4096, 1024, 1024]),
    (4, 4096, [4096, 1024, 1024]),
    (1, 4096, [14336, 14336]),
    (2, 4096, [14336, 14336]),
    (1, 14336, [4096]),
    (1, 5120, [5120, 5120, 5120]),
    (2, 4112, [1000, 333, 7, 64]),
    (3, 2064, [17, 1, 40]),
    (1, 16, [5, 9]),
    (8, 4096, [4096, 1024, 1024]),
    (16, 4096, [4096, 1024, 1024]),
    (5, 4160, [1000, 77, 2048]),
    # one split-kernel launch (and one reduction): q/k/v at 17-32 tokens, with
    # a half last batch of K (K % 128 == 64), and with reductions of two forms;
    # gate/up from 3 to 128 tokens (one slice of K, two wave groups per block)
    (17, 4096, [4096, 1024, 1024]),
    (32, 4096, [4096, 1024, 1024]),
    (24, 4160, [1000, 77, 2048]),
    (20, 2048, [1000, 1001]),
    (4, 4096, [14336, 14336]),
    (3, 4096, [14336, 12300]),
    (8, 4096, [14336, 14336]),
    (20, 4096, [14336, 14336]),
    (64, 4096, [14336, 14336]),
    (100, 4096, [14336, 14336]),
    # the one-group split shapes with several K slices (Llama-2-7B's gate/up at
    # 3-16, 17-32, 33-64 and 65-128 tokens, q/k/v of TinyLlama's width at 24)
    (8, 4096, [11008, 11008]),
    (24, 4096, [11008, 11008]),
    (40, 4096, [11008, 11008]),
    (100, 4096, [11008, 11008]),
    (24, 2048, [5632, 5634]),
    # the fused prefill kernel (129-4095 tokens): q/k/v on 128 x 128 tiles with
    # K slices of several counts, ragged shapes, gate/up on 256 x 256 tiles,
    # and q on 256 x 256 tiles beside k/v on 128 x 128 (two launches); from
    # 4096 tokens on hipBLASLt, one call each
    (512, 4096, [4096, 1024, 1024]),
    (300, 1040, [4100, 1000, 77]),
    (200, 4096, [14336, 4096]),
    (1024, 4096, [14336, 14336]),
    (2048, 4096, [4096, 1024, 1024]),
    (3000, 4096, [4096, 1024, 1024]),
    (4096, 4096, [4096, 1024]),
    # products of different shapes, grouped: k and v with token tiles in one
    # launch beside q alone (M = 33-128), two GEMV products and two split ones
    # in two launches, a small-M MFMA product with a split one, a GEMV product
    # with a split one; and down's deep shape, which has no shared form
    (64, 4096, [4096, 1024, 1024]),
    (33, 4096, [4096, 1024, 1024]),
    (100, 4160, [1000, 2048, 77]),
    (3, 4096, [4096, 12300, 1024, 14336]),
    (12, 4096, [4096, 14336]),
    (3, 4096, [4096, 12300]),
    (20, 14336, [4096, 4096]),
]


def f16bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def f16val(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def exact_activations(M: int, K: int) -> np.ndarray:
    """j * 2^-e in [-1, 1] with K * 128 * 2^e <= 2^23 (every partial sum exact)."""
    e = min(6, 16 - math.ceil(math.log2(K)))
    return f16bits(RNG.integers(-(2 ** e), 2 ** e + 1, size=(M, K)) * 2.0 ** -e)


def problem(M: int, K: int, ns, exact: bool):
    a = exact_activations(M, K) if exact else f16bits(RNG.standard_normal((M, K)))
    qs = [RNG.integers(-128, 128, size=(n, K)).astype(np.int8) for n in ns]
    scales = [RNG.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32) for n in ns]
    return a, qs, scales


def shared(lib, a, qs, scales, M, K):
    ab = dev(a)
    qb = [dev(q) for q in qs]
    sb = [dev(s) for s in scales]
    cb = [empty(M * q.shape[0] * 2) for q in qs]
    cnt = len(qs)
    rc = lib.ng_gemm_int8_shared_a(cnt, (C.c_void_p * cnt)(*[c.ptr for c in cb]), ab.vp,
                                   (C.c_void_p * cnt)(*[b.ptr for b in qb]),
                                   (C.c_void_p * cnt)(*[s.ptr for s in sb]),
                                   (C.c_int * cnt)(*[q.shape[0] for q in qs]), M, K)
    ok(rc, "ng_gemm_int8_shared_a")
    return [get(c, np.uint16, (M, q.shape[0])) for c, q in zip(cb, qs)]


def separate(lib, a, qs, scales, M, K):
    ab = dev(a)
    out = []
    for q, s in zip(qs, scales):
        qb, sb = dev(q), dev(s)
        cb = empty(M * q.shape[0] * 2)
        ok(lib.cuda_gemm_int8(cb.vp, ab.vp, qb.vp, sb.vp, M, K, q.shape[0], True), "cuda_gemm_int8")
        out.append(get(cb, np.uint16, (M, q.shape[0])))
    return out


@pytest.mark.parametrize("M,K,ns", SETS)
def test_shared_a_is_cuda_gemm_int8_bit_for_bit(lib, M, K, ns):
    banner(f"gemm_int8_shared_a random M={M} K={K} n={ns}")
    a, qs, scales = problem(M, K, ns, exact=False)
    got = shared(lib, a, qs, scales, M, K)
    want = separate(lib, a, qs, scales, M, K)
    for i, (g, w) in enumerate(zip(got, want)):
        assert_bits_equal(g, w, f"C_{i}")


@pytest.mark.parametrize("M,K,ns", [(1, 4096, [4096, 1024, 1024]), (4, 4096, [4096, 1024, 1024]),
                                    (1, 4096, [14336, 14336]), (2, 4112, [1000, 333, 7, 64]),
                                    (3, 2064, [17, 1, 40]), (8, 4096, [4096, 1024, 1024]),
                                    (5, 4160, [1000, 77, 2048]), (3, 4096, [4096, 12300]),
                                    (24, 4160, [1000, 77, 2048]), (20, 2048, [1000, 1001]),
                                    (8, 4096, [14336, 14336]), (100, 4096, [14336, 14336]),
                                    (64, 4096, [4096, 1024, 1024]), (3, 4096, [4096, 12300, 1024, 14336]),
                                    (512, 4096, [4096, 1024, 1024]), (300, 1040, [4100, 1000, 77])])
def test_shared_a_exact_inputs(lib, M, K, ns):
    banner(f"gemm_int8_shared_a exact M={M} K={K} n={ns}")
    a, qs, scales = problem(M, K, ns, exact=True)
    got = shared(lib, a, qs, scales, M, K)
    for i, (g, q, s) in enumerate(zip(got, qs, scales)):
        S = f16val(a) @ q.astype(np.float64).T
        want = (S.astype(np.float32) * s[None, :]).astype(np.float16).view(np.uint16)
        assert_bits_equal(g, want, f"C_{i}")


def test_shared_a_split_consecutive_calls(lib):
    banner("gemm_int8_shared_a split kernel: a call, then a smaller one, then a larger one")
    K = 4096
    sets = [(32, [4096, 1024, 1024]), (17, [2000, 48, 1024]), (32, [4096, 4096, 1024, 1024])]
    for M, ns in sets:
        a, qs, scales = problem(M, K, ns, exact=False)
        got = shared(lib, a, qs, scales, M, K)
        for i, (g, w) in enumerate(zip(got, separate(lib, a, qs, scales, M, K))):
            assert_bits_equal(g, w, f"M={M} C_{i}")


def test_shared_a_consecutive_calls(lib):
    banner("gemm_int8_shared_a two calls, the second smaller")
    M, K = 1, 4096
    a, qs, scales = problem(M, K, [4096, 1024, 1024], exact=False)
    first = shared(lib, a, qs, scales, M, K)
    a2, qs2, scales2 = problem(M, K, [2000, 48], exact=False)
    second = shared(lib, a2, qs2, scales2, M, K)
    for i, (g, w) in enumerate(zip(first, separate(lib, a, qs, scales, M, K))):
        assert_bits_equal(g, w, f"first C_{i}")
    for i, (g, w) in enumerate(zip(second, separate(lib, a2, qs2, scales2, M, K))):
        assert_bits_equal(g, w, f"second C_{i}")

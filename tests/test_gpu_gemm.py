"""cuda_gemm_int8 and cuda_gemm_fp16 on the GPU.

Bars:
  * exact inputs (activations on a grid 2^-e with |a| <= 1, so every partial
    sum of A @ q is exact in fp32 whatever the summation order) give
    bit-exact results: fp16(fp32(S) * scale[n]) on the weight-streaming path,
    where S = sum_k a_k q_k; fp16(S') on the dequantize + hipBLASLt path with
    power-of-two scales (fp16(q * s) exact, S' = sum_k a_k w_k exact);
  * random inputs stay within ulp16(ref) + 2^-9 * sum_k |a_k w_k| of the
    reference's composition (oracle.gemm_int8: fp16 weights fp16(q * s), then
    the product), which covers the reference's rounding of w to fp16 (2^-11),
    fp32 accumulation over K <= 16384 (K * 2^-24 < 2^-10) and the output
    rounding;
  * the reference's own tests (tests/matmul_test.go:19-255): the same shapes,
    distributions and absolute tolerances.
"""
from __future__ import annotations

import math
import subprocess
import sys
import textwrap
from pathlib import Path

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(31))


def f16bits(x) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def f16val(bits) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def exact_activations(M: int, K: int) -> np.ndarray:
    """Values j * 2^-e in [-1, 1] with K * 128 * 2^e <= 2^23: every partial
    sum of A @ q (|q| <= 128) is a multiple of 2^-e below 2^23 * 2^-e."""
    e = min(6, 16 - math.ceil(math.log2(K)))
    j = RNG.integers(-(2 ** e), 2 ** e + 1, size=(M, K))
    return f16bits(j * 2.0 ** -e)


def codes(shape) -> np.ndarray:
    return RNG.integers(-128, 128, size=shape).astype(np.int8)


def gemm_int8(lib, a, q, scale, M, K, N, tb: bool) -> np.ndarray:
    ab, qb, sb = dev(a), dev(q), dev(np.asarray(scale, np.float32))
    cb = empty(M * N * 2)
    ok(lib.cuda_gemm_int8(cb.vp, ab.vp, qb.vp, sb.vp, M, K, N, tb), "cuda_gemm_int8")
    return get(cb, np.uint16, (M, N))


def gemm_int8_fused(lib, a, q, scale, M, K, N) -> np.ndarray:
    """The fused int8 kernels at any M, through ng_gemm_int8_noalloc (same
    kernels and launch shapes as cuda_gemm_int8 up to LT_MIN_M rows of A)."""
    ab, qb, sb = dev(a), dev(q), dev(np.asarray(scale, np.float32))
    cb = empty(M * N * 2)
    ok(lib.ng_gemm_int8_noalloc(cb.vp, ab.vp, qb.vp, sb.vp, M, K, N, True), "ng_gemm_int8_noalloc")
    return get(cb, np.uint16, (M, N))


# From this many rows of A on, cuda_gemm_int8 in the engine's layout runs the
# reference's composition (B dequantized to fp16 into the stream's buffer,
# then hipBLASLt) instead of the fused prefill kernel (matmul.hip, kLtMinM).
LT_MIN_M = 4096


def gemm_fp16(lib, a, b, M, K, N, ta: bool, tb: bool) -> np.ndarray:
    ab, bb = dev(a), dev(b)
    cb = empty(M * N * 2)
    ok(lib.cuda_gemm_fp16(cb.vp, ab.vp, bb.vp, M, K, N, ta, tb), "cuda_gemm_fp16")
    return get(cb, np.uint16, (M, N))


def ulp16(v) -> np.ndarray:
    v = np.abs(np.asarray(v, np.float64))
    return 2.0 ** (np.floor(np.log2(np.maximum(v, 2.0 ** -14))) - 10)


def assert_within_bound(got_bits, a, q, scale, tb: bool, what: str, ora) -> None:
    ref = ora.gemm_int8(a, q, scale, tb)
    x = np.abs(f16val(a))
    w = np.abs(f16val(ora.dequant(q, scale, "row" if tb else "col")))
    mag = x @ (w.T if tb else w)
    d = np.abs(f16val(got_bits) - ref)
    bound = ulp16(ref) + 2.0 ** -9 * mag
    bad = d > bound
    assert not bad.any(), f"{what}: {bad.sum()} outside the bound; max |d| {d.max():.3g}, " \
                          f"max |d|/bound {(d / bound).max():.3g}"


def assert_fused_tight(got_bits, a, q, scale, what: str) -> None:
    """The fused int8 kernels' own semantics, fp16(RN32(S32) * scale[n]) with
    S32 the fp32 sum of a_k * q_k (each product exact in fp32) in the matrix
    cores' order, against the exact S (float64, whose own error is below
    K 2^-53 of sum |a q|). Bound: the fp32 accumulation, at most (K / 8 + 64)
    rounded additions on any path (MFMA k-groups, K slices, the in-order slice
    reduction), each within 2^-24 of the partial sum magnitude, so
    (K / 8 + 64) 2^-24 sum_k |a_k q_k| scale[n]; the fp32 product with the
    scale (2^-24 relative) and the fp16 rounding of the result (half an fp16
    ulp, taken as one). At K = 4096 that is about 3e-5 of sum |a w|, 70 times
    tighter than the bound to the reference's composition, whose fp16
    rounding of q * s it need not cover."""
    x = f16val(a)
    qq = q.astype(np.float64)
    K = qq.shape[1]
    ref = (x @ qq.T) * scale[None, :].astype(np.float64)
    mag = (np.abs(x) @ np.abs(qq).T) * scale[None, :].astype(np.float64)
    d = np.abs(f16val(got_bits) - ref)
    bound = ulp16(ref) + (K / 8 + 64) * 2.0 ** -24 * mag + 2.0 ** -24 * np.abs(ref)
    bad = d > bound
    assert not bad.any(), f"{what}: {bad.sum()} outside the fused-semantics bound; max |d| {d.max():.3g}, " \
                          f"max |d|/bound {(d / bound).max():.3g}"


# M, K, N: the weight-streaming path takes transpose_b, M <= 128 and K % 64 == 0
# (K % 16 == 0 for M <= 4). M <= 4 runs the GEMV kernel (K in 1024-code
# segments, the last one possibly partial); M > 16, and 4 < M <= 16 with K or
# N >= 8192, the split-K kernel with 1 to 8 slices of K (4 waves per block, 8
# for K >= 8192 and M > 16); 4 < M <= 16 otherwise the MFMA kernel that reads
# A from L2.
FUSED = [
    (1, 4096, 4096), (3, 4096, 1024), (16, 4096, 4096), (17, 4096, 1000), (32, 1024, 512), (33, 4096, 4096),
    (64, 4096, 4096), (64, 4096, 1024), (8, 14336, 4096), (64, 14336, 4096), (5, 64, 16), (2, 128, 7),
    (64, 4096, 14336), (1, 4096, 14336), (3, 4096, 8192), (5, 4096, 8192), (20, 1024, 8200), (40, 512, 8208),
    (2, 256, 9000), (48, 4096, 1024), (65, 4096, 1024), (96, 4096, 4096), (128, 14336, 4096), (100, 1024, 300),
    (7, 8192, 64), (128, 64, 64), (4, 4096, 4096), (1, 1040, 100), (4, 2064, 33), (2, 14352, 64),
    (3, 16, 5), (12, 1024, 4096),
    # K >= 8192 with M > 16: eight waves per block in the split kernel (one case with K % 128 == 64)
    (24, 8192, 1000), (100, 8256, 384), (48, 9216, 2048),
    # M = 3, 4 with K or N >= 8192: the split kernel (two wave groups per block for N >= 12288 at K < 8192)
    (4, 4096, 14336), (3, 4096, 12300), (3, 14336, 4096), (4, 14336, 100), (4, 8256, 200),
    # N >= 12288 at K < 8192: two wave groups per block at every tile height, odd batch counts, a half batch
    (128, 4096, 14336), (80, 4160, 12288), (20, 1088, 13000), (33, 2048, 12290), (9, 192, 12288),
    (3, 64, 12288), (4, 128, 12300), (70, 64, 12288),
    # N <= 2048 at K < 8192 with M > 32: token tiles of 32 rows of A as separate blocks
    (96, 4096, 1000), (128, 4096, 2048), (33, 1024, 64), (127, 4160, 1030),
]


@pytest.mark.parametrize("M,K,N", FUSED)
def test_int8_weight_streaming_bit_exact(lib, M, K, N):
    banner(f"gemm_int8 streaming exact M={M} K={K} N={N}")
    a = exact_activations(M, K)
    q = codes((N, K))
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float16).astype(np.float32)
    got = gemm_int8(lib, a, q, scale, M, K, N, True)
    S = f16val(a) @ q.astype(np.float64).T
    want = (S.astype(np.float32) * scale[None, :]).astype(np.float16).view(np.uint16)
    assert_bits_equal(got, want, "C")


@pytest.mark.parametrize("M,K,N", [(1, 4096, 4096), (64, 4096, 2048), (16, 14336, 512), (30, 2048, 300),
                                   (12, 4096, 14336), (128, 4096, 1024)])
def test_int8_weight_streaming_random(lib, ora, M, K, N):
    banner(f"gemm_int8 streaming random M={M} K={K} N={N}")
    a = f16bits(RNG.standard_normal((M, K)))
    q = codes((N, K))
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float32)
    got = gemm_int8(lib, a, q, scale, M, K, N, True)
    assert_within_bound(got, a, q, scale, True, "C", ora)
    assert_fused_tight(got, a, q, scale, "C")


INF_SHAPES = [(1, 1040, 100), (2, 14352, 64), (4, 2064, 33), (8, 4160, 512), (12, 1088, 4096), (64, 4096, 4096),
              (33, 8256, 384), (80, 4160, 12288), (3, 4096, 12300), (20, 1088, 13000), (128, 14336, 4096),
              (100, 4160, 1000)]


@pytest.mark.parametrize("M,K,N", INF_SHAPES)
def test_int8_weight_streaming_inf_activations(lib, M, K, N):
    """One infinite activation per row. The reference's product gives
    +-inf in every column whose weight at that k is nonzero and NaN where it is
    zero (inf * 0). The infs sit at the ends of 64- and 128-k batches and at
    the last k, which the kernels' padding (partial last batch, batches past a
    K slice, lanes past K) loads again: padding must not turn them into NaN."""
    banner(f"gemm_int8 streaming inf activations M={M} K={K} N={N}")
    a = exact_activations(M, K)
    cand = sorted({K - 1, K - 64, K - 65, 0} | {min(K - 1, 64 * j + 63) for j in range(K // 64 + 1)})
    ks = np.array([cand[(m * 7) % len(cand)] for m in range(M)])
    sgn = np.where(np.arange(M) % 2 == 0, 1.0, -1.0)
    a[np.arange(M), ks] = f16bits(sgn * np.inf)
    q = codes((N, K))
    q[: max(1, N // 9), ks[0]] = 0     # some zero codes under the first row's inf: NaN there
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float16).astype(np.float32)
    got = f16val(gemm_int8(lib, a, q, scale, M, K, N, True))
    qk = q[:, ks].T.astype(np.float64)          # [M, N]: the code under each row's inf
    with np.errstate(invalid="ignore"):
        want = np.where(qk == 0, np.nan, sgn[:, None] * np.sign(qk) * np.inf)
    nan_w = np.isnan(want)
    assert (np.isnan(got) == nan_w).all(), f"NaN pattern: {(np.isnan(got) != nan_w).sum()} outputs differ"
    assert (got[~nan_w] == want[~nan_w]).all(), "signed infinities differ"


# The prefill kernel (transpose_b, M > 128, K % 16 == 0): ragged M and N,
# K with a partial last step of 128 (K % 128 = 64, 16), full model shapes.
# 256 x 256 tiles from 192 of them on: 1000 x 14336, 777 x 16000 (ragged in M
# and N), 3072 x 4096, 1000 x 4112 x 12300 (K % 64 = 16).
PREFILL = [(129, 4096, 1024), (256, 4096, 4096), (4096, 4096, 1024), (200, 4160, 1000), (300, 1040, 384),
           (4100, 1024, 300), (130, 14336, 256), (1000, 4096, 14336), (2049, 2048, 2056), (640, 16, 64),
           (777, 1024, 16000), (3072, 4096, 4096), (1000, 4112, 12300)]


@pytest.mark.parametrize("M,K,N", PREFILL)
def test_int8_prefill_bit_exact(lib, M, K, N):
    banner(f"gemm_int8 prefill exact M={M} K={K} N={N}")
    a = exact_activations(M, K)
    q = codes((N, K))
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float16).astype(np.float32)
    got = gemm_int8(lib, a, q, scale, M, K, N, True) if M < LT_MIN_M else gemm_int8_fused(lib, a, q, scale, M, K, N)
    S = f16val(a) @ q.astype(np.float64).T
    want = (S.astype(np.float32) * scale[None, :]).astype(np.float16).view(np.uint16)
    assert_bits_equal(got, want, "C")


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 4096), (512, 14336, 1024), (300, 1040, 4100), (2048, 14336, 4096)])
def test_int8_prefill_random(lib, ora, M, K, N):
    banner(f"gemm_int8 prefill random M={M} K={K} N={N}")
    a = f16bits(RNG.standard_normal((M, K)))
    q = codes((N, K))
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float32)
    got = gemm_int8(lib, a, q, scale, M, K, N, True)
    assert_within_bound(got, a, q, scale, True, "C", ora)
    if M < LT_MIN_M:
        assert_fused_tight(got, a, q, scale, "C")
    else:
        fused = gemm_int8_fused(lib, a, q, scale, M, K, N)
        assert_within_bound(fused, a, q, scale, True, "C (fused kernel)", ora)
        assert_fused_tight(fused, a, q, scale, "C (fused kernel)")


# From LT_MIN_M rows on, cuda_gemm_int8 (transpose_b) dequantizes B to fp16 and
# multiplies with hipBLASLt, as the reference does. With power-of-two scales
# every fp16(q * s) is exact and so is every partial sum: the result is fp16
# of the exact product, bit for bit. Shapes: Mistral-7B's k_proj and q_proj at
# 4096 tokens, ragged M and N, K = 14336 (down_proj).
LT_ROWS = [(4096, 4096, 1024), (4096, 4096, 4096), (4100, 1024, 300), (4096, 14336, 512)]


@pytest.mark.parametrize("M,K,N", LT_ROWS)
def test_int8_prefill_library_rows_bit_exact(lib, M, K, N):
    banner(f"gemm_int8 dequant + hipBLASLt exact M={M} K={K} N={N}")
    a = exact_activations(M, K)
    q = codes((N, K))
    scale = (2.0 ** -RNG.integers(6, 10, N)).astype(np.float32)
    got = gemm_int8(lib, a, q, scale, M, K, N, True)
    S = f16val(a) @ (q.astype(np.float64) * scale[:, None]).T
    assert_bits_equal(got, S.astype(np.float16).view(np.uint16), "C")


@pytest.mark.parametrize("M,K,N", [(4096, 4096, 4096), (4096, 4096, 1024)])
def test_int8_prefill_library_rows_is_the_composition(lib, ora, M, K, N):
    """From LT_MIN_M rows on, cuda_gemm_int8 on random inputs gives the bits of
    the reference's two calls made separately: cuda_dequantize_weights into
    an fp16 buffer, then cuda_gemm_fp16 (matmul.cu:205-236), which use the
    same hipBLASLt algorithm for the shape."""
    banner(f"gemm_int8 = dequantize + gemm_fp16, random M={M} K={K} N={N}")
    a = f16bits(RNG.standard_normal((M, K)))
    q = codes((N, K))
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float32)
    got = gemm_int8(lib, a, q, scale, M, K, N, True)
    wb, qb, sb = empty(2 * N * K), dev(q), dev(scale)
    ok(lib.cuda_dequantize_weights(wb.vp, qb.vp, sb.vp, N, K, 1), "cuda_dequantize_weights")
    want = gemm_fp16(lib, a, get(wb, np.uint16, (N, K)), M, K, N, False, True)
    assert_bits_equal(got, want, "C")
    assert_within_bound(got, a, q, scale, True, "C", ora)


@pytest.mark.parametrize("M,K,N", [(256, 4160, 512), (129, 1040, 300), (1024, 4096, 1024), (777, 1024, 16000)])
def test_int8_prefill_inf_activations(lib, M, K, N):
    test_int8_weight_streaming_inf_activations(lib, M, K, N)


# The dequantize + hipBLASLt path: B [K, N] with per-column scales, or
# transpose_b with K not a multiple of 16 (of 64 for 4 < M <= 128).
LIBRARY = [
    (4, 256, 128, False), (129, 4104, 1024, True), (256, 1024, 512, False), (7, 200, 96, True),
    (512, 4104, 4096, True), (33, 1024, 4096, False),
]


@pytest.mark.parametrize("M,K,N,tb", LIBRARY)
def test_int8_dequant_library_bit_exact(lib, M, K, N, tb):
    banner(f"gemm_int8 library exact M={M} K={K} N={N} tb={tb}")
    a = exact_activations(M, K)
    q = codes((N, K) if tb else (K, N))
    p = RNG.integers(6, 10, N)
    scale = (2.0 ** -p).astype(np.float32)
    got = gemm_int8(lib, a, q, scale, M, K, N, tb)
    w = q.astype(np.float64) * scale[:, None] if tb else q.astype(np.float64) * scale[None, :]
    S = f16val(a) @ (w.T if tb else w)
    assert_bits_equal(got, S.astype(np.float16).view(np.uint16), "C")


@pytest.mark.parametrize("M,K,N,tb", [(129, 4104, 1024, True), (16, 1024, 512, False), (100, 960, 200, True)])
def test_int8_dequant_library_random(lib, ora, M, K, N, tb):
    banner(f"gemm_int8 library random M={M} K={K} N={N} tb={tb}")
    a = f16bits(RNG.standard_normal((M, K)))
    q = codes((N, K) if tb else (K, N))
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float32)
    got = gemm_int8(lib, a, q, scale, M, K, N, tb)
    assert_within_bound(got, a, q, scale, tb, "C", ora)


def test_int8_paths_agree(lib, ora):
    """The same product through both kernel families (M <= 128 streams the
    weights, M = 129 takes the prefill kernel): both within the bound."""
    banner("gemm_int8 both paths")
    K, N = 4096, 2048
    a = f16bits(RNG.standard_normal((129, K)))
    q = codes((N, K))
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float32)
    big = gemm_int8(lib, a, q, scale, 129, K, N, True)
    small = gemm_int8(lib, a[:128], q, scale, 128, K, N, True)
    assert_within_bound(big[:128], a[:128], q, scale, True, "prefill", ora)
    assert_within_bound(small, a[:128], q, scale, True, "streaming", ora)


@pytest.mark.parametrize("M", [16, 64, 300, 2048])
def test_int8_streaming_is_deterministic(lib, M):
    banner(f"gemm_int8 streaming repeat M={M}")
    K, N = 4096, 4096
    a = f16bits(RNG.standard_normal((M, K)))
    q = codes((N, K))
    scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float32)
    ab, qb, sb = dev(a), dev(q), dev(scale)
    outs = []
    for _ in range(3):
        cb = empty(M * N * 2)
        ok(lib.cuda_gemm_int8(cb.vp, ab.vp, qb.vp, sb.vp, M, K, N, True))
        outs.append(get(cb, np.uint16, (M, N)))
    assert_bits_equal(outs[1], outs[0], "repeat 1")
    assert_bits_equal(outs[2], outs[0], "repeat 2")


def test_int8_split_partials_grow(lib):
    """The split kernel's per-stream partial-sum buffer grows from a small call
    to a larger one and is reused by a smaller one after that."""
    banner("gemm_int8 split partials growth")
    for (M, K, N) in [(20, 1024, 128), (100, 14336, 4096), (33, 4096, 512)]:
        a = exact_activations(M, K)
        q = codes((N, K))
        scale = RNG.uniform(1e-3, 1e-2, N).astype(np.float16).astype(np.float32)
        got = gemm_int8(lib, a, q, scale, M, K, N, True)
        S = f16val(a) @ q.astype(np.float64).T
        want = (S.astype(np.float32) * scale[None, :]).astype(np.float16).view(np.uint16)
        assert_bits_equal(got, want, f"C {M}x{K}x{N}")


def test_int8_library_buffer_grows(lib):
    """The per-stream fp16 weight copy grows from a small call to a larger one
    and is reused by a smaller one after that."""
    banner("gemm_int8 library buffer growth")
    for (M, K, N) in [(170, 128, 64), (170, 2048, 2048), (170, 256, 64)]:
        a = exact_activations(M, K)
        q = codes((K, N))
        scale = np.full(N, 2.0 ** -7, np.float32)
        got = gemm_int8(lib, a, q, scale, M, K, N, False)
        S = f16val(a) @ (q.astype(np.float64) * 2.0 ** -7)
        assert_bits_equal(got, S.astype(np.float16).view(np.uint16), f"C {M}x{K}x{N}")


def test_int8_across_shutdown_and_init():
    """cuda_shutdown resets the device. The GEMM buffers, plans and hipBLASLt
    handle made before it are released first, and calls after cuda_init build
    new ones. Runs in a child process: the reset releases every device
    allocation of the process, including other tests' buffers."""
    banner("gemm_int8 across cuda_shutdown / cuda_init (child process)")
    root = str(Path(__file__).resolve().parent.parent)
    script = textwrap.dedent(f"""
        import sys
        sys.path.insert(0, {root!r})
        import numpy as np
        from neurogrid_amd import _lib
        from neurogrid_amd.device import DeviceBuffer as DB
        L = _lib.load()
        rng = np.random.Generator(np.random.PCG64(3))
        for rnd in range(2):
            assert L.cuda_init(0) == 0
            # streaming (tb, small M), split-K (M = 40) and dequant + hipBLASLt (M = 200)
            for M, K, N, tb in [(1, 256, 64, True), (40, 512, 128, True), (200, 128, 64, False)]:
                a = (rng.integers(-64, 65, (M, K)) / 64.0).astype(np.float16)
                q = rng.integers(-128, 128, (N, K) if tb else (K, N)).astype(np.int8)
                s = np.full(N, 2.0 ** -7, np.float32)
                ab, qb, sb, cb = DB.from_array(a.view(np.uint16)), DB.from_array(q), DB.from_array(s), DB(2 * M * N)
                assert L.cuda_gemm_int8(cb.vp, ab.vp, qb.vp, sb.vp, M, K, N, tb) == 0
                got = cb.download(np.uint16, (M, N))
                w = q.astype(np.float64) * 2.0 ** -7
                want = (a.astype(np.float64) @ (w.T if tb else w)).astype(np.float16).view(np.uint16)
                assert (got == want).all(), (rnd, M, K, N, tb)
                for b in (ab, qb, sb, cb):
                    b.free()
            L.cuda_shutdown()
        print("ok", flush=True)
    """)
    r = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr


@pytest.mark.parametrize("ta", [False, True])
@pytest.mark.parametrize("tb", [False, True])
@pytest.mark.parametrize("M,K,N", [(32, 128, 64), (5, 96, 40), (256, 1024, 384)])
def test_fp16_gemm_bit_exact(lib, M, K, N, ta, tb):
    banner(f"gemm_fp16 exact M={M} K={K} N={N} ta={ta} tb={tb}")
    # A on a 2^-3 grid in [-1, 1], B on a 2^-3 grid in [-1, 1]: sums exact in fp32.
    a = f16bits(RNG.integers(-8, 9, (K, M) if ta else (M, K)) / 8.0)
    b = f16bits(RNG.integers(-8, 9, (N, K) if tb else (K, N)) / 8.0)
    got = gemm_fp16(lib, a, b, M, K, N, ta, tb)
    x, w = f16val(a), f16val(b)
    S = (x.T if ta else x) @ (w.T if tb else w)
    assert_bits_equal(got, S.astype(np.float16).view(np.uint16), "C")


# ---- the reference's own tests (tests/matmul_test.go) -------------------------

def _ref_uniform(n):
    return RNG.random(n, dtype=np.float32) * 2 - 1


def _cpu_matmul(a, b):
    return (a.astype(np.float32) @ b.astype(np.float32)).astype(np.float32)


def test_reference_kat_gemm_fp16(lib):
    """TestGEMMFP16 (matmul_test.go:19-92): [32,128] x [128,64], U(-1,1), max |d| < 0.1."""
    banner("reference TestGEMMFP16")
    M, K, N = 32, 128, 64
    A = _ref_uniform(M * K).reshape(M, K)
    B = _ref_uniform(K * N).reshape(K, N)
    got = f16val(gemm_fp16(lib, f16bits(A), f16bits(B), M, K, N, False, False))
    assert np.abs(got - _cpu_matmul(A, B)).max() < 0.1


def test_reference_kat_gemm_int8(lib):
    """TestGEMMINT8 (matmul_test.go:98-179): A [32,128] U(-1,1), B int8 [128,64]
    uniform over [-128,127], scales 0.01, transpose_b false, max |d| < 5e-2."""
    banner("reference TestGEMMINT8")
    M, K, N = 32, 128, 64
    A = _ref_uniform(M * K).reshape(M, K)
    q = codes((K, N))
    scale = np.full(N, 0.01, np.float32)
    got = f16val(gemm_int8(lib, f16bits(A), q, scale, M, K, N, False))
    assert np.abs(got - _cpu_matmul(A, q.astype(np.float32) * scale[None, :])).max() < 5e-2


def test_reference_kat_gemm_int8_engine_layout(lib):
    """TestGEMMINT8's data in the engine's layout (B [N, K], transpose_b), which
    takes the weight-streaming path."""
    banner("reference TestGEMMINT8, transpose_b")
    M, K, N = 32, 128, 64
    A = _ref_uniform(M * K).reshape(M, K)
    q = codes((N, K))
    scale = np.full(N, 0.01, np.float32)
    got = f16val(gemm_int8(lib, f16bits(A), q, scale, M, K, N, True))
    assert np.abs(got - _cpu_matmul(A, (q.astype(np.float32) * scale[:, None]).T)).max() < 5e-2


def test_reference_kat_gemm_transpose(lib):
    """TestGEMMTranspose (matmul_test.go:183-255): A stored [K, M], C = A^T @ B, max |d| < 0.1."""
    banner("reference TestGEMMTranspose")
    M, K, N = 32, 128, 64
    A = _ref_uniform(K * M).reshape(K, M)
    B = _ref_uniform(K * N).reshape(K, N)
    got = f16val(gemm_fp16(lib, f16bits(A), f16bits(B), M, K, N, True, False))
    assert np.abs(got - _cpu_matmul(A.T, B)).max() < 0.1

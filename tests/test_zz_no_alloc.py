"""ng_gemm_int8_noalloc: cuda_gemm_int8's weight-streaming (M <= 128) and
prefill (M > 128) paths with their split-K partial sums in the library's
fixed device array instead of an allocated buffer.

Checked through the C ABI against cuda_gemm_int8 itself (the same kernels and
launch shapes, so the bar is bit-exact): two calls in a row, the second with a
smaller input, so that the second reads none of the first call's leftovers;
then shapes covering every kernel family, and device memory unchanged across
calls. From 4096 rows on the inputs are exact (activations on a 2^-e grid,
power-of-two scales), on which any correct path gives fp16 of the exact
product, so the comparison stays bit-exact whichever path cuda_gemm_int8
takes there. Shapes that only the hipBLASLt path takes are refused on the
host.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(97))


# From this many rows of A on, cuda_gemm_int8 takes the dequantize + hipBLASLt
# composition (matmul.hip, kLtMinM).
LT_MIN_M = 4096


def inputs(M, K, N, exact=False):
    if exact:
        e = min(6, 16 - int(np.ceil(np.log2(K))))   # every partial sum exact in fp32
        a = (RNG.integers(-(2 ** e), 2 ** e + 1, (M, K)) * 2.0 ** -e).astype(np.float16).view(np.uint16)
        s = (2.0 ** -RNG.integers(6, 10, N)).astype(np.float32)
    else:
        a = np.asarray(RNG.standard_normal((M, K)), np.float32).astype(np.float16).view(np.uint16)
        s = RNG.uniform(1e-3, 1e-2, N).astype(np.float32)
    q = RNG.integers(-128, 128, (N, K)).astype(np.int8)
    return dev(a), dev(q), dev(s)


def both(lib, M, K, N):
    """(cuda_gemm_int8 output, ng_gemm_int8_noalloc output) on the same inputs."""
    ab, qb, sb = inputs(M, K, N, exact=M >= LT_MIN_M)
    c_ref, c_new = empty(2 * M * N), empty(2 * M * N)
    ok(lib.cuda_gemm_int8(c_ref.vp, ab.vp, qb.vp, sb.vp, M, K, N, True), "cuda_gemm_int8")
    ok(lib.ng_gemm_int8_noalloc(c_new.vp, ab.vp, qb.vp, sb.vp, M, K, N, True), "ng_gemm_int8_noalloc")
    return get(c_ref, np.uint16, (M, N)), get(c_new, np.uint16, (M, N))


def test_noalloc_two_calls_second_smaller(lib):
    # 1st: down_proj at M = 64 (8 slices of K: 8 MiB of partial sums);
    # 2nd: smaller, also split (q_proj-like at M = 20, fewer outputs and slices).
    first, second = (64, 14336, 4096), (20, 4096, 1000)
    banner(f"ng_gemm_int8_noalloc two calls: {first} then {second}")
    data = [inputs(*sh) for sh in (first, second)]
    refs = []
    for (M, K, N), (ab, qb, sb) in zip((first, second), data):
        c = empty(2 * M * N)
        ok(lib.cuda_gemm_int8(c.vp, ab.vp, qb.vp, sb.vp, M, K, N, True), "cuda_gemm_int8")
        refs.append(get(c, np.uint16, (M, N)))
    for (M, K, N), (ab, qb, sb), ref in zip((first, second), data, refs):
        c = empty(2 * M * N)
        ok(lib.ng_gemm_int8_noalloc(c.vp, ab.vp, qb.vp, sb.vp, M, K, N, True), "ng_gemm_int8_noalloc")
        assert_bits_equal(get(c, np.uint16, (M, N)), ref, f"noalloc {M}x{K}x{N}")


# GEMV (M <= 4), the small-M MFMA kernel, the split kernel with 1 to 8 slices
# (4 and 8 waves), and two wave groups per block (N >= 12288 at K < 8192).
# The prefill kernel with 1 to 8 slices of K, both tile shapes, ragged M and N.
SHAPES = [(1, 4096, 4096), (4, 2064, 33), (8, 4096, 4096), (12, 1088, 4096), (33, 4096, 1024),
          (64, 4096, 14336), (128, 14336, 4096), (100, 8256, 384), (128, 4096, 1024), (3, 4096, 12300),
          (129, 256, 64), (200, 4096, 1000), (512, 4096, 4096), (300, 14336, 4096), (1024, 4096, 14336),
          (3072, 4096, 4096), (4096, 4096, 1024)]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_noalloc_matches_cuda_gemm_int8(lib, M, K, N):
    banner(f"ng_gemm_int8_noalloc vs cuda_gemm_int8 M={M} K={K} N={N}")
    ref, got = both(lib, M, K, N)
    assert_bits_equal(got, ref, f"noalloc {M}x{K}x{N}")


def test_noalloc_allocates_nothing(lib):
    """Device memory in use is the same before and after a run of calls with
    shapes not seen before (the library's own buffers would grow)."""
    banner("ng_gemm_int8_noalloc device memory unchanged")
    shapes = [(96, 14336, 4096), (48, 8192, 8192), (2, 1024, 512), (384, 4096, 4096), (2000, 1024, 8000)]
    bufs = []
    for M, K, N in shapes:
        ab, qb, sb = inputs(M, K, N)
        bufs.append((M, K, N, ab, qb, sb, empty(2 * M * N)))
    ok(lib.cuda_sync_device(), "sync")
    used0 = C.c_size_t()
    ok(lib.cuda_get_memory_used(C.byref(used0)), "memory used")
    for M, K, N, ab, qb, sb, cb in bufs:
        ok(lib.ng_gemm_int8_noalloc(cb.vp, ab.vp, qb.vp, sb.vp, M, K, N, True), "ng_gemm_int8_noalloc")
    ok(lib.cuda_sync_device(), "sync")
    used1 = C.c_size_t()
    ok(lib.cuda_get_memory_used(C.byref(used1)), "memory used")
    assert used1.value == used0.value, f"device memory in use changed: {used0.value} -> {used1.value}"


def test_noalloc_refuses_other_paths(lib, capfd):
    banner("ng_gemm_int8_noalloc refuses shapes that only the hipBLASLt path takes")
    ab, qb, sb = inputs(129, 256, 64)
    cb = empty(2 * 129 * 64)
    assert lib.ng_gemm_int8_noalloc(cb.vp, ab.vp, qb.vp, sb.vp, 129, 200, 64, True) == -1   # M > 128, K % 16 != 0
    assert lib.ng_gemm_int8_noalloc(cb.vp, ab.vp, qb.vp, sb.vp, 4, 256, 64, False) == -1    # not transpose_b
    assert lib.ng_gemm_int8_noalloc(cb.vp, ab.vp, qb.vp, sb.vp, 8, 200, 64, True) == -1     # K % 64 != 0
    assert "call cuda_gemm_int8 instead" in capfd.readouterr().err

"""Tensors past 2^31 elements on the GPU: every offset is 64-bit.

The reference forms element indices in int (kernels.cu:126-359, one thread per
element: blockIdx.x * blockDim.x + threadIdx.x), which wraps at 2^31
elements. This library takes size_t counts (element-wise entry points) or int
rows x int columns (row kernels, gather, per-row int8) and forms every offset
in 64 bits, so these shapes work. Each case fills a tensor of more than 2^31
elements by repeating a random block whose length is a prime (65521 or
65519): an offset that wrapped by any power of two would read other values.
Elements (or rows) on both sides of 2^31 are checked against the oracle, bit
for bit. RoPE refuses tensors of 2^31 elements or more (its wave index is 32-bit);
that error path is checked too.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(61))
P1, P2 = 65521, 65519     # primes: no power-of-two wrap keeps the pattern
H = 4096
T = (1 << 19) + 5         # T * H = 2^31 + 20480 elements


def block(period: int, scale: float) -> np.ndarray:
    return (RNG.standard_normal(period) * scale).astype(np.float16).view(np.uint16)


def periodic(n: int, period: int, scale: float) -> np.ndarray:
    return np.resize(block(period, scale), n)


def edge_rows(rows: int):
    """Rows at both ends and around element 2^31 (row 2^31 / H = 2^19)."""
    b = (1 << 31) // H
    return np.array(sorted({0, 1, b - 2, b - 1, b, b + 1, rows - 1}))


def test_add_past_2_31_elements(lib, ora):
    n = (1 << 31) + 8 * 64 * 3 + 5           # the ragged tail takes the scalar path
    banner(f"cuda_add n={n}")
    ba, bb = block(P1, 1.0), block(P2, 2.0)
    ad, bd = dev(np.resize(ba, n)), dev(np.resize(bb, n))
    cd = empty(2 * n)
    ok(lib.cuda_add(cd.vp, ad.vp, bd.vp, n), "cuda_add")
    ad.free(), bd.free()
    got = get(cd, np.uint16, (n,))
    cd.free()
    for lo, hi in ((0, 1 << 16), ((1 << 31) - (1 << 16), n)):   # the second window runs past 2^31 to the end
        idx = np.arange(lo, hi)
        assert_bits_equal(got[lo:hi], ora.elementwise("add", ba[idx % P1], bb[idx % P2]), f"add [{lo}, {hi})")


def test_rmsnorm_past_2_31_elements(lib, ora):
    banner(f"cuda_rmsnorm T={T} H={H}")
    x = periodic(T * H, P1, 1.0).reshape(T, H)
    w = (1.0 + 0.02 * RNG.standard_normal(H)).astype(np.float16).view(np.uint16)
    xb, wb = dev(x), dev(w)
    yb = empty(2 * T * H)
    ok(lib.cuda_rmsnorm(yb.vp, xb.vp, wb.vp, T, H, C.c_float(1e-5)), "cuda_rmsnorm")
    xb.free()
    got = get(yb, np.uint16, (T, H))
    yb.free()
    rows = edge_rows(T)
    assert_bits_equal(got[rows], ora.rmsnorm(x[rows], w, 1e-5), "rmsnorm rows")


def test_gather_past_2_31_elements(lib, ora):
    banner(f"cuda_gather_embeddings T={T} H={H}")
    V = 4099
    table = (RNG.standard_normal((V, H)) * 0.02).astype(np.float16).view(np.uint16)
    ids = ((np.arange(T, dtype=np.int64) * 7919) % V).astype(np.int32)
    tb, ib = dev(table), dev(ids)
    ob = empty(2 * T * H)
    ok(lib.cuda_gather_embeddings(ob.vp, tb.vp, C.cast(C.c_void_p(ib.ptr), C.POINTER(C.c_int)), H, T),
       "cuda_gather_embeddings")
    got = get(ob, np.uint16, (T, H))
    ob.free()
    rows = edge_rows(T)
    assert_bits_equal(got[rows], ora.gather(table, ids[rows]), "gathered rows")


def test_quantize_rows_past_2_31_elements(lib, ora):
    banner(f"cuda_quantize_weights_per_row rows={T} cols={H}")
    x = periodic(T * H, P2, 3.0).reshape(T, H)
    xb = dev(x)
    qb, sb = empty(T * H), empty(4 * T)
    ok(lib.cuda_quantize_weights_per_row(qb.vp, sb.vp, xb.vp, T, H), "cuda_quantize_weights_per_row")
    xb.free()
    q = get(qb, np.int8, (T, H))
    s = get(sb, np.float32, (T,))
    qb.free(), sb.free()
    rows = edge_rows(T)
    wq, ws = ora.quant_rows(x[rows])
    assert_bits_equal(q[rows].view(np.uint8), wq.view(np.uint8), "codes")
    assert_bits_equal(s[rows].view(np.uint32), ws.view(np.uint32), "scales")


def test_rope_refuses_2_31_elements(lib):
    banner("cuda_rope_with_theta refuses 2^31 elements")
    p = C.c_void_p(256)
    ip = C.cast(p, C.POINTER(C.c_int))
    # 2^31 elements: 2^17 tokens x 128 heads x 128; refused before any launch
    assert lib.cuda_rope_with_theta(p, p, ip, 1, 1 << 17, 128, 128, 0, C.c_float(1e4)) == -1

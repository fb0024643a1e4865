"""Element-wise kernels on the GPU vs the oracle.

add, mul, scale and the converters are exactly rounded: bit-exact.
silu and silu_mul use hardware exp2/rcp: within |d| <= 1e-2 or 2 ulp, and the
fraction of bit-identical outputs is checked to stay high.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, assert_close16, banner, dev, empty, get, ok

# numpy's float32 -> float16 casts of values beyond the fp16 range give inf,
# the expected result, and warn about it.
pytestmark = [pytest.mark.gpu, pytest.mark.filterwarnings("ignore:overflow encountered in cast:RuntimeWarning")]

RNG = np.random.Generator(np.random.PCG64(5))


def bits(x, dtype):
    x = np.asarray(x, np.float32)
    if dtype == "bf16":
        from oracle.oracle import f32_to_bf16_bits

        return f32_to_bf16_bits(x)
    return x.astype(np.float16).view(np.uint16)


FNS = {
    ("f16", "add"): "cuda_add", ("f16", "mul"): "cuda_mul", ("f16", "silu"): "cuda_silu",
    ("f16", "silu_mul"): "cuda_silu_mul", ("bf16", "add"): "cuda_bf16_add", ("bf16", "mul"): "cuda_bf16_mul",
    ("bf16", "silu"): "cuda_bf16_silu", ("bf16", "silu_mul"): "ng_bf16_silu_mul",
}


def run(lib, dtype, op, a, b=None, off=0, inplace=False):
    n = a.size
    ab = empty(a.nbytes + 2 * off)
    ab.upload(np.concatenate([np.zeros(off, np.uint16), a]))
    bb = None
    if b is not None:
        bb = empty(b.nbytes + 2 * off)
        bb.upload(np.concatenate([np.zeros(off, np.uint16), b]))
    ob = ab if inplace else empty(a.nbytes + 2 * off)
    fn = getattr(lib, FNS[(dtype, op)])
    if b is None:
        ok(fn(ob.offset(2 * off), ab.offset(2 * off), n), op)
    else:
        ok(fn(ob.offset(2 * off), ab.offset(2 * off), bb.offset(2 * off), n), op)
    return get(ob, np.uint16, (n + off,))[off:]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("op", ["add", "mul", "silu", "silu_mul"])
@pytest.mark.parametrize("n,off", [(1, 0), (7, 0), (4096, 0), (1 << 20, 0), (1000003, 0), (4099, 1), (65536, 3)])
def test_elementwise(lib, ora, dtype, op, n, off):
    banner(f"elementwise {dtype} {op} n={n} off={off}")
    a = bits(RNG.standard_normal(n) * 4, dtype)
    b = bits(RNG.standard_normal(n), dtype) if op in ("add", "mul", "silu_mul") else None
    got = run(lib, dtype, op, a, b, off)
    want = ora.elementwise(op, a, b, dtype=dtype)
    if op in ("add", "mul"):
        assert_bits_equal(got, want, f"{op} {dtype}")
    else:
        frac = assert_close16(got, want, dtype, f"{op} {dtype}")
        if n >= 4096:
            assert frac > 0.99, frac


def test_silu_mul_in_place_like_the_engine(lib, ora):
    # gpu/engine/layer.cu:1049: cuda_silu_mul(gate, gate, up, n)
    banner("silu_mul in place")
    n = 1 << 16
    g, u = bits(RNG.standard_normal(n) * 3, "f16"), bits(RNG.standard_normal(n), "f16")
    gb, ub = dev(g), dev(u)
    ok(lib.cuda_silu_mul(gb.vp, gb.vp, ub.vp, n))
    assert_close16(get(gb, np.uint16, (n,)), ora.elementwise("silu_mul", g, u), "f16", "in place")


def test_silu_all_fp16_inputs(lib, ora):
    banner("silu all fp16 inputs")
    h = np.arange(65536, dtype=np.uint16)
    h = h[np.isfinite(h.view(np.float16))]
    frac = assert_close16(run(lib, "f16", "silu", h), ora.elementwise("silu", h), "f16", "silu all")
    assert frac > 0.99


def test_scale_bit_exact(lib, ora):
    banner("scale")
    n = 100001
    a = bits(RNG.standard_normal(n) * 50, "f16")
    ab, ob = dev(a), empty(2 * n)
    ok(lib.cuda_scale(ob.vp, ab.vp, C.c_float(0.125 + 1e-3), n))
    assert_bits_equal(get(ob, np.uint16, (n,)), ora.elementwise("scale", a, s=np.float32(0.125 + 1e-3)), "scale")


@pytest.mark.parametrize("n", [1, 8, 1000, 8 * 777 + 5, 1 << 20])
def test_converters_exact(lib, ora, n):
    banner(f"converters n={n}")
    x = (RNG.standard_normal(n) * 10.0 ** RNG.integers(-6, 6, n)).astype(np.float32)
    xb = dev(x)
    o16 = empty(2 * n)
    ok(lib.cuda_fp32_to_bf16(o16.vp, xb.vp, n))
    bf = get(o16, np.uint16, (n,))
    assert_bits_equal(bf, ora.f32_to_bf16_bits(x), "fp32->bf16")
    o32 = empty(4 * n)
    ok(lib.cuda_bf16_to_fp32(o32.vp, o16.vp, n))
    assert_bits_equal(get(o32, np.float32, (n,)).view(np.uint32), ora.bf16_bits_to_f32(bf).view(np.uint32),
                      "bf16->fp32")
    ok(lib.ng_fp32_to_fp16(o16.vp, xb.vp, n))
    h = get(o16, np.uint16, (n,))
    assert_bits_equal(h, x.astype(np.float16).view(np.uint16), "fp32->fp16")
    ok(lib.ng_fp16_to_fp32(o32.vp, o16.vp, n))
    assert_bits_equal(get(o32, np.float32, (n,)), h.view(np.float16).astype(np.float32), "fp16->fp32")
    hb = dev(h)
    ok(lib.cuda_fp16_to_bf16(o16.vp, hb.vp, n))
    assert_bits_equal(get(o16, np.uint16, (n,)), ora.f32_to_bf16_bits(h.view(np.float16).astype(np.float32)),
                      "fp16->bf16")
    bb = dev(bf)
    ok(lib.cuda_bf16_to_fp16(o16.vp, bb.vp, n))
    assert_bits_equal(get(o16, np.uint16, (n,)), ora.bf16_bits_to_f32(bf).astype(np.float16).view(np.uint16),
                      "bf16->fp16")


@pytest.mark.parametrize("off,extra", [(0, 0), (1, 7)])
def test_bf16_to_fp16_truncate_every_pattern(lib, ora, off, extra):
    """All 65 536 bf16 patterns (plus a ragged tail, from an unaligned start)
    through the loader's truncating conversion, bit-exact with the oracle."""
    banner(f"bf16->fp16 truncate off={off} extra={extra}")
    x = np.concatenate([np.arange(65536, dtype=np.uint16), RNG.integers(0, 65536, extra).astype(np.uint16)])
    n = x.size
    xb = dev(np.concatenate([np.zeros(off, np.uint16), x]))
    ob = empty(2 * (n + off))
    ok(lib.ng_bf16_to_fp16_truncate(C.c_void_p(ob.ptr + 2 * off), C.c_void_p(xb.ptr + 2 * off), n))
    got = get(ob, np.uint16, (n + off,))[off:]
    assert_bits_equal(got, ora.bf16_to_f16_trunc(x), "bf16->fp16 truncate")


def test_softmax_close(lib, ora):
    banner("softmax")
    x = bits(RNG.standard_normal((33, 1000)) * 4, "f16")
    xb, ob = dev(x), empty(x.nbytes)
    ok(lib.cuda_softmax(ob.vp, xb.vp, 33, 1000))
    assert_close16(get(ob, np.uint16, x.shape), ora.softmax(x), "f16", "softmax")

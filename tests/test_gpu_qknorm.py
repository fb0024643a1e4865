"""Per-head RMSNorm (QK LayerNorm) and its fusion with RoPE, on the GPU.

ng_per_head_rmsnorm must equal the oracle's RMSNorm of the tokens * heads rows
of head_dim elements bit for bit (the same exact statistic as cuda_rmsnorm).
ng_qk_rmsnorm_rope_with_theta must equal the composition it fuses, run on the
GPU as separate launches (ng_per_head_rmsnorm on Q and K, then
ng_rope_qk_with_theta) bit for bit, and the oracle's RMSNorm followed by its
RoPE to |d| <= 1e-2 or 2 ulp (the rotation's sin/cos).
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, assert_close16, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(21))


def bits(x, dtype):
    x = np.asarray(x, np.float32)
    if dtype == "bf16":
        from oracle.oracle import f32_to_bf16_bits

        return f32_to_bf16_bits(x)
    return x.astype(np.float16).view(np.uint16)


def per_head(lib, x, w, eps, dtype):
    T, nh, D = x.shape
    xb, wb, ob = dev(x), dev(w), empty(x.nbytes)
    fn = lib.ng_bf16_per_head_rmsnorm if dtype == "bf16" else lib.ng_per_head_rmsnorm
    ok(fn(ob.vp, xb.vp, wb.vp, T, nh, D, C.c_float(eps)), "per_head_rmsnorm")
    return get(ob, np.uint16, x.shape)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("T,nh,D", [(64, 32, 128), (7, 8, 64), (5, 6, 256), (9, 3, 80), (1, 1, 8)])
def test_per_head_rmsnorm_bit_exact(lib, ora, dtype, T, nh, D):
    banner(f"per-head rmsnorm {dtype} T={T} nh={nh} D={D}")
    x = bits(RNG.standard_normal((T, nh, D)) * 3, dtype)
    w = bits(1 + 0.1 * RNG.standard_normal(D), dtype)
    got = per_head(lib, x, w, 1e-5, dtype)
    want = ora.rmsnorm(x.reshape(-1, D), w, 1e-5, dtype).reshape(x.shape)
    assert_bits_equal(got, want, "per-head rmsnorm")


def adversarial_heads(D, n):
    """Heads whose exact sum of squares sits on an fp32 rounding boundary."""
    out = np.zeros((n, D), np.float32)
    for i in range(n):
        out[i, 0], out[i, D // 2] = 2.0 ** 15, 8.0
        if i % 3 == 1:
            out[i, D - 1] = 2.0 ** -24
        if i % 3 == 2:
            out[i, 3], out[i, D - 5] = 1.0, 2.0 ** -12
    return out


QKN_CASES = [
    # (T, nq, nkv, D, theta, maxpos)
    (512, 32, 8, 128, 1e6, 4096),
    (64, 32, 8, 128, 1e6, 4096),     # decode: passes split over waves
    (40, 16, 8, 64, 1e4, 128),
    (20, 6, 3, 256, 5e5, 32768),
    (20, 5, 2, 80, 1e4, 1000),       # head_dim 80: separate launches
]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("inplace", [False, True])
@pytest.mark.parametrize("T,nq,nkv,D,theta,maxpos", QKN_CASES)
def test_qk_rmsnorm_rope(lib, ora, dtype, style, inplace, T, nq, nkv, D, theta, maxpos):
    banner(f"qk-norm+rope {dtype} style={style} inplace={inplace} T={T} nq={nq} nkv={nkv} D={D}")
    q = bits(RNG.standard_normal((T, nq, D)) * 2, dtype)
    k = bits(RNG.standard_normal((T, nkv, D)) * 2, dtype)
    if D == 128 and dtype == "f16":
        # heads that need the exact sum of squares
        q.reshape(-1, D)[5:11] = bits(adversarial_heads(D, 6), dtype)
        k.reshape(-1, D)[2:5] = bits(adversarial_heads(D, 3), dtype)
    wq = bits(1 + 0.1 * RNG.standard_normal(D), dtype)
    wk = bits(1 + 0.1 * RNG.standard_normal(D), dtype)
    pos = RNG.integers(0, maxpos, T).astype(np.int32)
    eps, th = 1e-5, C.c_float(theta)

    qb, kb, wqb, wkb, pb = dev(q), dev(k), dev(wq), dev(wk), dev(pos)
    qo = qb if inplace else empty(q.nbytes)
    ko = kb if inplace else empty(k.nbytes)
    fn = lib.ng_bf16_qk_rmsnorm_rope_with_theta if dtype == "bf16" else lib.ng_qk_rmsnorm_rope_with_theta
    ok(fn(qo.vp, qb.vp, ko.vp, kb.vp, wqb.vp, wkb.vp, pb.ip, 1, T, nq, nkv, D, C.c_float(eps), style, th), "fused")
    gq, gk = get(qo, np.uint16, q.shape), get(ko, np.uint16, k.shape)

    # the composition it fuses, as separate GPU launches
    nq_ = per_head(lib, q, wq, eps, dtype)
    nk_ = per_head(lib, k, wk, eps, dtype)
    cq, ck = dev(nq_), dev(nk_)
    rope = lib.ng_bf16_rope_qk_with_theta if dtype == "bf16" else lib.ng_rope_qk_with_theta
    ok(rope(cq.vp, cq.vp, ck.vp, ck.vp, pb.ip, 1, T, nq, nkv, D, style, th), "rope_qk")
    assert_bits_equal(gq, get(cq, np.uint16, q.shape), "Q vs composition")
    assert_bits_equal(gk, get(ck, np.uint16, k.shape), "K vs composition")

    # the oracle: RMSNorm per head, then RoPE
    oq = ora.rope(ora.rmsnorm(q.reshape(-1, D), wq, eps, dtype).reshape(q.shape), pos, style, theta, dtype)
    ok_ = ora.rope(ora.rmsnorm(k.reshape(-1, D), wk, eps, dtype).reshape(k.shape), pos, style, theta, dtype)
    assert_close16(gq, oq, dtype, "Q vs oracle")
    assert_close16(gk, ok_, dtype, "K vs oracle")

"""RoPE and embedding gather on the GPU vs the oracle.

RoPE: same fp32 angle on both sides (host-computed inv_freq, one fp32
product); sin/cos may differ in the last fp32 bit, so outputs are checked to
|d| <= 1e-2 or 2 ulp with a high bit-identical fraction. Gather: bit copy.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_util import C, assert_bits_equal, assert_close16, banner, dev, empty, get, ok

pytestmark = pytest.mark.gpu

RNG = np.random.Generator(np.random.PCG64(3))


def bits(x, dtype):
    x = np.asarray(x, np.float32)
    if dtype == "bf16":
        from oracle.oracle import f32_to_bf16_bits

        return f32_to_bf16_bits(x)
    return x.astype(np.float16).view(np.uint16)


def run_rope(lib, x, pos, style, theta, dtype, B=1, inplace=False, entry="theta"):
    T, nh, D = x.shape
    S = T // B
    xb, pb = dev(x), dev(pos.astype(np.int32))
    ob = xb if inplace else empty(x.nbytes)
    if entry == "theta":
        fn = lib.cuda_bf16_rope_with_theta if dtype == "bf16" else lib.cuda_rope_with_theta
        ok(fn(ob.vp, xb.vp, pb.ip, B, S, nh, D, style, C.c_float(theta)), "rope")
    elif entry == "styled":
        ok(lib.cuda_rope_styled(ob.vp, xb.vp, pb.ip, B, S, nh, D, style), "rope_styled")
    else:
        ok(lib.cuda_rope(ob.vp, xb.vp, pb.ip, B, S, nh, D), "rope")
    return get(ob, np.uint16, x.shape)


CASES = [
    # (T, nh, D, theta, maxpos)
    (4096, 32, 128, 1e6, 4096),     # Mistral-7B Q prefill
    (64, 8, 128, 1e6, 4096),        # Mistral-7B K decode
    (96, 40, 128, 1e4, 8192),       # Llama-2-13B heads
    (50, 32, 64, 1e4, 128),         # TinyLlama Q
    (50, 4, 64, 1e4, 128),          # TinyLlama K
    (20, 3, 256, 5e5, 32768),
    (20, 5, 80, 1e4, 1000),         # head_dim 80: split-half takes the scalar kernel
    (20, 5, 96, 1e4, 1000),
    (3, 1, 2, 1e4, 10),
]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("T,nh,D,theta,maxpos", CASES)
def test_rope_close(lib, ora, dtype, style, T, nh, D, theta, maxpos):
    banner(f"rope {dtype} style={style} T={T} nh={nh} D={D}")
    x = bits(RNG.standard_normal((T, nh, D)), dtype)
    pos = RNG.integers(0, maxpos, T).astype(np.int32)
    got = run_rope(lib, x, pos, style, theta, dtype)
    frac = assert_close16(got, ora.rope(x, pos, style, theta, dtype), dtype, "rope")
    if x.size >= 4096:
        assert frac > 0.95, frac


def test_rope_large_positions_bf16(lib, ora):
    # Mistral-Nemo case: positions up to 32768, theta 1e6.
    banner("rope bf16 large positions")
    x = bits(RNG.standard_normal((2048, 8, 128)), "bf16")
    pos = RNG.integers(0, 32768, 2048).astype(np.int32)
    assert_close16(run_rope(lib, x, pos, 0, 1e6, "bf16"), ora.rope(x, pos, 0, 1e6, "bf16"), "bf16", "rope nemo")


def test_rope_in_place_batched_and_defaults(lib, ora):
    banner("rope in place / batched / default entry points")
    B, S, nh, D = 3, 17, 8, 128
    x = bits(RNG.standard_normal((B * S, nh, D)), "f16")
    pos = np.tile(np.arange(S, dtype=np.int32), B)
    want = ora.rope(x, pos, 0, 1e4)
    assert_close16(run_rope(lib, x, pos, 0, 1e4, "f16", B=B, inplace=True), want, "f16", "in place")
    assert_close16(run_rope(lib, x, pos, 0, 0, "f16", B=B, entry="default"), want, "f16", "cuda_rope")
    assert_close16(run_rope(lib, x, pos, 1, 0, "f16", B=B, entry="styled"), ora.rope(x, pos, 1, 1e4), "f16",
                   "cuda_rope_styled")
    # any style other than 1 pairs split-half, as in the reference
    assert_close16(run_rope(lib, x, pos, 7, 1e4, "f16", B=B), want, "f16", "style 7")


def test_rope_position_zero_identity(lib):
    banner("rope identity at position 0")
    x = bits(RNG.standard_normal((16, 32, 128)), "f16")
    got = run_rope(lib, x, np.zeros(16, np.int32), 0, 1e6, "f16")
    assert_bits_equal(got, x, "identity")


# Kernel shapes covered: four rows per wave (T >= 4096, H <= 4096) with 2, 4 and
# 8 vectors per lane and a ragged last wave; one row per wave with 2, 4, 8 and
# 10 vectors per lane; rows of more than 5120 elements (chunked); H % 8 != 0.
@pytest.mark.parametrize("V,H,T", [(32000, 4096, 4096), (100, 128, 1), (1000, 2048, 7), (50, 4100, 9),
                                   (131072, 5120, 64), (1000, 256, 4096), (1000, 1024, 4099),
                                   (500, 2048, 4097), (300, 4096, 100), (64, 8192, 33)])
def test_gather_bit_exact(lib, ora, V, H, T):
    banner(f"gather V={V} H={H} T={T}")
    table = RNG.integers(0, 65536, (V, H)).astype(np.uint16)
    ids = RNG.integers(0, V, T).astype(np.int32)
    tb, ib, ob = dev(table), dev(ids), empty(2 * T * H)
    ok(lib.cuda_gather_embeddings(ob.vp, tb.vp, ib.ip, H, T), "gather")
    assert_bits_equal(get(ob, np.uint16, (T, H)), ora.gather(table, ids), "gather")


def test_gather_checked_zero_fills_bad_ids(lib):
    banner("gather checked")
    V, H = 100, 256
    table = RNG.integers(0, 65536, (V, H)).astype(np.uint16)
    ids = np.int32([5, -1, 99, 100, 7, 1 << 30])
    tb, ib, ob = dev(table), dev(ids), empty(2 * ids.size * H)
    eb = dev(np.zeros(1, np.int32))
    ok(lib.ng_gather_embeddings_checked(ob.vp, tb.vp, ib.ip, H, ids.size, V, eb.ip), "gather checked")
    got = get(ob, np.uint16, (ids.size, H))
    assert get(eb, np.int32, (1,))[0] == 3
    for i, t in enumerate(ids):
        want = table[t] if 0 <= t < V else np.zeros(H, np.uint16)
        assert_bits_equal(got[i], want, f"row {i}")


@pytest.mark.parametrize("T", [4101, 37])
def test_gather_checked_rows_per_wave(lib, T):
    """The checked gather with four rows per wave (T >= 4096, ragged last wave)
    and with one: bad ids anywhere, including the last rows, are zero-filled
    and counted."""
    banner(f"gather checked T={T}")
    V, H = 700, 1024
    table = RNG.integers(0, 65536, (V, H)).astype(np.uint16)
    ids = RNG.integers(0, V, T).astype(np.int32)
    bad_at = np.unique(np.concatenate([RNG.choice(T, min(T, 40), replace=False), [0, T - 1]]))
    ids[bad_at] = np.where(np.arange(bad_at.size) % 2 == 0, -3, V + 11)
    tb, ib, ob = dev(table), dev(ids), empty(2 * T * H)
    eb = dev(np.zeros(1, np.int32))
    ok(lib.ng_gather_embeddings_checked(ob.vp, tb.vp, ib.ip, H, T, V, eb.ip), "gather checked")
    got = get(ob, np.uint16, (T, H))
    assert get(eb, np.int32, (1,))[0] == bad_at.size
    valid = (ids >= 0) & (ids < V)
    want = np.zeros((T, H), np.uint16)
    want[valid] = table[ids[valid]]
    assert_bits_equal(got, want, "checked gather")


QK_CASES = [
    # (T, nq, nkv, D, theta, maxpos)
    (4096, 32, 8, 128, 1e6, 4096),     # Mistral-7B prefill
    (64, 32, 8, 128, 1e6, 4096),       # Mistral-7B decode: passes split over several waves
    (300, 40, 40, 128, 1e4, 8192),     # Llama-2-13B heads
    (50, 32, 4, 64, 1e4, 128),         # TinyLlama
    (20, 6, 3, 256, 5e5, 32768),
    (20, 5, 2, 80, 1e4, 1000),         # head_dim 80: two single launches
]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("style", [0, 1])
@pytest.mark.parametrize("inplace", [False, True])
@pytest.mark.parametrize("T,nq,nkv,D,theta,maxpos", QK_CASES)
def test_rope_qk_fused(lib, ora, dtype, style, inplace, T, nq, nkv, D, theta, maxpos):
    """ng_rope_qk_with_theta == the two cuda_rope_with_theta calls it fuses, and the oracle."""
    banner(f"rope_qk {dtype} style={style} inplace={inplace} T={T} nq={nq} nkv={nkv} D={D}")
    q = bits(RNG.standard_normal((T, nq, D)), dtype)
    k = bits(RNG.standard_normal((T, nkv, D)), dtype)
    pos = RNG.integers(0, maxpos, T).astype(np.int32)
    qb, kb, pb = dev(q), dev(k), dev(pos)
    qo = qb if inplace else empty(q.nbytes)
    ko = kb if inplace else empty(k.nbytes)
    fn = lib.ng_bf16_rope_qk_with_theta if dtype == "bf16" else lib.ng_rope_qk_with_theta
    ok(fn(qo.vp, qb.vp, ko.vp, kb.vp, pb.ip, 1, T, nq, nkv, D, style, C.c_float(theta)), "rope_qk")
    gq, gk = get(qo, np.uint16, q.shape), get(ko, np.uint16, k.shape)
    assert_bits_equal(gq, run_rope(lib, q, pos, style, theta, dtype), "fused Q vs single launch")
    assert_bits_equal(gk, run_rope(lib, k, pos, style, theta, dtype), "fused K vs single launch")
    assert_close16(gq, ora.rope(q, pos, style, theta, dtype), dtype, "Q vs oracle")
    assert_close16(gk, ora.rope(k, pos, style, theta, dtype), dtype, "K vs oracle")
